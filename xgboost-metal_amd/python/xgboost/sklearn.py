"""scikit-learn estimators (reference python-package/xgboost/sklearn.py:867, 1309-1410, 1728-1840)."""
from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import numpy as np

from .core import Booster, DMatrix, XGBoostError
from .training import train

_PARAMS = ("max_depth", "max_leaves", "max_bin", "grow_policy", "learning_rate", "n_estimators", "verbosity",
           "objective", "booster", "tree_method", "n_jobs", "gamma", "min_child_weight", "max_delta_step",
           "subsample", "sampling_method", "colsample_bytree", "colsample_bylevel", "colsample_bynode", "reg_alpha",
           "reg_lambda", "scale_pos_weight", "base_score", "random_state", "missing", "num_parallel_tree",
           "monotone_constraints", "interaction_constraints", "importance_type", "device", "validate_parameters",
           "enable_categorical", "feature_types", "max_cat_to_onehot", "max_cat_threshold", "multi_strategy",
           "eval_metric", "early_stopping_rounds", "callbacks")


class XGBModel:
    def __init__(self, *, max_depth: Optional[int] = None, max_leaves: Optional[int] = None,
                 max_bin: Optional[int] = None, grow_policy: Optional[str] = None,
                 learning_rate: Optional[float] = None, n_estimators: Optional[int] = None,
                 verbosity: Optional[int] = None, objective: Any = None, booster: Optional[str] = None,
                 tree_method: Optional[str] = None, n_jobs: Optional[int] = None, gamma: Optional[float] = None,
                 min_child_weight: Optional[float] = None, max_delta_step: Optional[float] = None,
                 subsample: Optional[float] = None, sampling_method: Optional[str] = None,
                 colsample_bytree: Optional[float] = None, colsample_bylevel: Optional[float] = None,
                 colsample_bynode: Optional[float] = None, reg_alpha: Optional[float] = None,
                 reg_lambda: Optional[float] = None, scale_pos_weight: Optional[float] = None,
                 base_score: Optional[float] = None, random_state: Any = None, missing: float = np.nan,
                 num_parallel_tree: Optional[int] = None, monotone_constraints: Any = None,
                 interaction_constraints: Any = None, importance_type: Optional[str] = None,
                 device: Optional[str] = None, validate_parameters: Optional[bool] = None,
                 enable_categorical: bool = False, feature_types: Any = None, max_cat_to_onehot: Optional[int] = None,
                 max_cat_threshold: Optional[int] = None, multi_strategy: Optional[str] = None,
                 eval_metric: Any = None, early_stopping_rounds: Optional[int] = None, callbacks: Any = None,
                 **kwargs: Any) -> None:
        for name in _PARAMS:
            setattr(self, name, locals()[name])
        self.kwargs = kwargs
        self._Booster: Optional[Booster] = None

    # sklearn protocol
    def get_params(self, deep: bool = True) -> Dict[str, Any]:
        params = {name: getattr(self, name) for name in _PARAMS}
        params.update(self.kwargs)
        return params

    def set_params(self, **params: Any) -> "XGBModel":
        for key, value in params.items():
            if key in _PARAMS:
                setattr(self, key, value)
            else:
                self.kwargs[key] = value
        return self

    def get_xgb_params(self) -> Dict[str, Any]:
        skip = {"n_estimators", "missing", "importance_type", "enable_categorical", "feature_types",
                "early_stopping_rounds", "callbacks", "n_jobs", "random_state"}
        params = {k: v for k, v in self.get_params().items() if k not in skip and v is not None}
        if self.random_state is not None:
            params["seed"] = self.random_state
        if callable(params.get("objective")):
            params.pop("objective")
        params.setdefault("tree_method", "hist")
        return params

    def _n_estimators(self) -> int:
        return 100 if self.n_estimators is None else int(self.n_estimators)

    def get_booster(self) -> Booster:
        if self._Booster is None:
            raise XGBoostError("need to call fit or load_model beforehand")
        return self._Booster

    def _dmatrix(self, X: Any, y: Any = None, sample_weight: Any = None, base_margin: Any = None) -> DMatrix:
        return DMatrix(X, y, weight=sample_weight, base_margin=base_margin, missing=self.missing)

    def _fit(self, X: Any, y: Any, params: Dict[str, Any], sample_weight: Any, base_margin: Any,
             eval_set: Any, sample_weight_eval_set: Any, verbose: Any, xgb_model: Any) -> "XGBModel":
        dtrain = self._dmatrix(X, y, sample_weight, base_margin)
        evals = []
        if eval_set:
            for k, (ex, ey) in enumerate(eval_set):
                w = sample_weight_eval_set[k] if sample_weight_eval_set else None
                evals.append((self._dmatrix(ex, ey, w), f"validation_{k}"))
        self.evals_result_: Dict[str, Dict[str, list]] = {}
        obj = self.objective if callable(self.objective) else None
        if isinstance(xgb_model, XGBModel):
            xgb_model = xgb_model.get_booster()
        self._Booster = train(params, dtrain, self._n_estimators(), evals=evals, obj=obj,
                              early_stopping_rounds=self.early_stopping_rounds, evals_result=self.evals_result_,
                              verbose_eval=verbose, xgb_model=xgb_model, callbacks=self.callbacks)
        self.n_features_in_ = dtrain.num_col()
        return self

    def _iteration_range(self, iteration_range: Any) -> Tuple[int, int]:
        """The caller's range, else the rounds up to the early-stopping best (reference sklearn.py:1178)."""
        if iteration_range is not None:
            return tuple(iteration_range)
        try:
            return (0, self.get_booster().best_iteration + 1)
        except AttributeError:
            return (0, 0)

    def apply(self, X: Any, iteration_range: Any = None) -> np.ndarray:
        """Leaf index each row reaches in every tree, rows x trees (reference
        sklearn.py:1509); the rounds end at the early-stopping best unless given."""
        return self.get_booster().predict(self._dmatrix(X), pred_leaf=True,
                                          iteration_range=self._iteration_range(iteration_range))

    @property
    def best_iteration(self) -> int:
        return self.get_booster().best_iteration

    @property
    def best_score(self) -> float:
        return self.get_booster().best_score

    def evals_result(self) -> Dict[str, Dict[str, list]]:
        return self.evals_result_

    def save_model(self, fname: str) -> None:
        self.get_booster().save_model(fname)

    def load_model(self, fname: Any) -> None:
        if self._Booster is None:
            self._Booster = Booster()
        self._Booster.load_model(fname)

    @property
    def feature_importances_(self) -> np.ndarray:
        """Normalised ``get_score(importance_type or "gain")`` per feature (reference sklearn.py:1609)."""
        b = self.get_booster()
        score = b.get_score(importance_type=self.importance_type or "gain")
        names = b.feature_names if b.feature_names is not None else [f"f{i}" for i in range(b.num_features())]
        values = np.array([score.get(f, 0.0) for f in names], dtype=np.float32)
        total = values.sum()
        return values if total == 0 else values / total


class XGBRegressor(XGBModel):
    """Regression with ``reg:squarederror`` by default."""

    def __init__(self, *, objective: Any = "reg:squarederror", **kwargs: Any) -> None:
        super().__init__(objective=objective, **kwargs)

    def fit(self, X: Any, y: Any, *, sample_weight: Any = None, base_margin: Any = None, eval_set: Any = None,
            verbose: Any = True, xgb_model: Any = None, sample_weight_eval_set: Any = None,
            **kwargs: Any) -> "XGBRegressor":
        return self._fit(X, y, self.get_xgb_params(), sample_weight, base_margin, eval_set, sample_weight_eval_set,
                         verbose, xgb_model)

    def predict(self, X: Any, output_margin: bool = False, validate_features: bool = True, base_margin: Any = None,
                iteration_range: Any = None) -> np.ndarray:
        d = self._dmatrix(X, base_margin=base_margin)
        return self.get_booster().predict(d, output_margin=output_margin, iteration_range=self._iteration_range(iteration_range))

    def score(self, X: Any, y: Any, sample_weight: Any = None) -> float:
        pred = self.predict(X)
        y = np.asarray(y, dtype=np.float64)
        w = np.ones_like(y) if sample_weight is None else np.asarray(sample_weight, dtype=np.float64)
        u = (w * (y - pred) ** 2).sum()
        v = (w * (y - np.average(y, weights=w)) ** 2).sum()
        return float(1 - u / v)


class XGBClassifier(XGBModel):
    """Binary classification with ``binary:logistic``."""

    def __init__(self, *, objective: Any = "binary:logistic", **kwargs: Any) -> None:
        super().__init__(objective=objective, **kwargs)

    def fit(self, X: Any, y: Any, *, sample_weight: Any = None, base_margin: Any = None, eval_set: Any = None,
            verbose: Any = True, xgb_model: Any = None, sample_weight_eval_set: Any = None,
            **kwargs: Any) -> "XGBClassifier":
        y = np.asarray(y)
        self.classes_ = np.unique(y)
        if len(self.classes_) > 2:
            raise XGBoostError("Only binary classification is supported by this engine")
        self.n_classes_ = len(self.classes_)
        encoded = np.searchsorted(self.classes_, y).astype(np.float32)
        if eval_set:
            eval_set = [(ex, np.searchsorted(self.classes_, np.asarray(ey)).astype(np.float32)) for ex, ey in eval_set]
        return self._fit(X, encoded, self.get_xgb_params(), sample_weight, base_margin, eval_set,
                         sample_weight_eval_set, verbose, xgb_model)

    def predict_proba(self, X: Any, validate_features: bool = True, base_margin: Any = None,
                      iteration_range: Any = None) -> np.ndarray:
        d = self._dmatrix(X, base_margin=base_margin)
        p = self.get_booster().predict(d, iteration_range=self._iteration_range(iteration_range))
        return np.column_stack([1 - p, p])

    def predict(self, X: Any, output_margin: bool = False, validate_features: bool = True, base_margin: Any = None,
                iteration_range: Any = None) -> np.ndarray:
        d = self._dmatrix(X, base_margin=base_margin)
        p = self.get_booster().predict(d, output_margin=output_margin, iteration_range=self._iteration_range(iteration_range))
        if output_margin:
            return p
        return self.classes_[(p > 0.5).astype(int)]

    def score(self, X: Any, y: Any, sample_weight: Any = None) -> float:
        return float(np.average(self.predict(X) == np.asarray(y), weights=sample_weight))
