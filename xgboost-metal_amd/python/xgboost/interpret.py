"""SHAP values of a model, split into per-feature values and the bias
(reference python-package/xgboost/interpret.py:56 shap_values): the device's
exact path-dependent TreeSHAP through Booster.predict(pred_contribs=True)."""
from typing import Any, Optional, Tuple

import numpy as np

from .core import Booster, DMatrix

__all__ = ["shap_values"]


def shap_values(model: Any, X: Any, *, X_background: Any = None, output_margin: bool = False,
                iteration_range: Optional[Tuple[int, int]] = None, missing: Optional[float] = None,
                validate_features: bool = True) -> Tuple[np.ndarray, np.ndarray]:
    """Contributions of every feature to each row's margin and the bias term.

    `model` is a Booster or an estimator with get_booster(); `X` a DMatrix or
    anything DMatrix accepts (with the estimator's `missing` unless given).
    Interventional values over a background set (`X_background`) are not
    computed; `output_margin` is accepted for the signature's sake, the values
    being of the margin either way.  For an estimator the default rounds end
    at its early-stopping best, as its predict does.
    """
    if X_background is not None:
        raise NotImplementedError("`X_background` is not yet supported.")
    del output_margin
    if isinstance(model, Booster):
        booster = model
        rounds = iteration_range if iteration_range is not None else (0, 0)
    else:
        get_booster = getattr(model, "get_booster", None)
        if not callable(get_booster):
            raise TypeError("`model` must be an xgboost.Booster or an object with get_booster().")
        booster = get_booster()
        if not isinstance(booster, Booster):
            raise TypeError("`model.get_booster()` must return an xgboost.Booster.")
        pick = getattr(model, "_iteration_range", None)
        rounds = pick(iteration_range) if callable(pick) else (iteration_range or (0, 0))
    if isinstance(X, DMatrix):
        if missing is not None:
            raise ValueError("`missing` must not be specified when `X` is a DMatrix.")
        data = X
    else:
        fill = missing if missing is not None else getattr(model, "missing", None)
        data = DMatrix(X, missing=np.nan if fill is None else fill)
    contribs = booster.predict(data, pred_contribs=True, validate_features=validate_features,
                               iteration_range=tuple(rounds))
    return contribs[..., :-1], contribs[..., -1]
