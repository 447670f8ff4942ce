"""XGBoost-compatible Python API of the MI355X (gfx950) hist engine.

Mirrors the reference's python-package/xgboost surface for tree_method='hist'
with depthwise growth: DMatrix, QuantileDMatrix, Booster, train and the
XGBRegressor/XGBClassifier estimators.
"""
from . import callback, interpret
from .config import config_context, get_config, set_config
from .core import Booster, DataIter, DMatrix, QuantileDMatrix, XGBoostError, build_info
from .sklearn import XGBClassifier, XGBModel, XGBRegressor
from .training import cv, train

__version__ = "3.5.0-dev"

__all__ = ["Booster", "callback", "interpret", "DataIter", "DMatrix", "QuantileDMatrix", "XGBoostError", "XGBClassifier", "XGBModel", "XGBRegressor",
           "build_info", "config_context", "cv", "get_config", "set_config", "train", "__version__"]
