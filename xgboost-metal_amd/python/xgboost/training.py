"""xgb.train (reference python-package/xgboost/training.py:60-216)."""
from __future__ import annotations

from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

from .core import Booster, DMatrix, XGBoostError


def _parse_eval(msg: str) -> List[Tuple[str, str, float]]:
    out = []
    for part in msg.split("\t")[1:]:
        name_metric, value = part.rsplit(":", 1)
        name, metric = name_metric.split("-", 1)
        out.append((name, metric, float(value)))
    return out


def train(params: Dict[str, Any], dtrain: DMatrix, num_boost_round: int = 10, *,
          evals: Optional[Sequence[Tuple[DMatrix, str]]] = None, obj: Optional[Callable] = None,
          maximize: Optional[bool] = None, early_stopping_rounds: Optional[int] = None,
          evals_result: Optional[Dict[str, Dict[str, List[float]]]] = None, verbose_eval: Any = True,
          xgb_model: Any = None, callbacks: Optional[Sequence[Any]] = None, custom_metric: Optional[Callable] = None,
          feval: Optional[Callable] = None) -> Booster:
    """Train a booster for ``num_boost_round`` rounds."""
    evals = list(evals) if evals else []
    params = dict(params or {})
    bst = Booster(params, [dtrain] + [d for d, _ in evals], model_file=xgb_model)
    start = bst.num_boosted_rounds() if xgb_model is not None else 0
    metric_fn = custom_metric or feval
    best_score = None
    best_iteration = 0
    for i in range(start, start + num_boost_round):
        bst.update(dtrain, i, fobj=obj)
        if evals:
            msg = bst.eval_set(evals, i, feval=metric_fn)
            parsed = _parse_eval(msg)
            if evals_result is not None:
                for name, metric, value in parsed:
                    evals_result.setdefault(name, {}).setdefault(metric, []).append(value)
            if verbose_eval and (verbose_eval is True or (isinstance(verbose_eval, int) and i % verbose_eval == 0)):
                print(msg)
            if early_stopping_rounds:
                name, metric, score = parsed[-1]
                better_high = maximize if maximize is not None else metric.startswith(("auc", "map", "ndcg"))
                improved = best_score is None or (score > best_score if better_high else score < best_score)
                if improved:
                    best_score, best_iteration = score, i
                elif i - best_iteration >= early_stopping_rounds:
                    break
    if early_stopping_rounds and best_score is not None:
        bst.set_attr(best_iteration=str(best_iteration), best_score=str(best_score))
        bst.best_iteration = best_iteration
        bst.best_score = best_score
    return bst


def cv(*args: Any, **kwargs: Any) -> Any:
    raise XGBoostError("xgboost.cv is not provided by the HIP hist engine")
