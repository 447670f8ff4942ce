"""xgb.train and xgb.cv (reference python-package/xgboost/training.py:60-560).

Both run the boosting loop under a ``CallbackContainer``: evaluation after
every round, ``EvaluationMonitor`` for ``verbose_eval``, ``EarlyStopping``
for ``early_stopping_rounds``, and any user callbacks.
"""
from __future__ import annotations

import copy
import ctypes
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .callback import CallbackContainer, EarlyStopping, EvaluationMonitor, TrainingCallback
from .core import _LIB, Booster, DMatrix, XGBoostError, _check_call


def train(params: Dict[str, Any], dtrain: DMatrix, num_boost_round: int = 10, *,
          evals: Optional[Sequence[Tuple[DMatrix, str]]] = None, obj: Optional[Callable] = None,
          maximize: Optional[bool] = None, early_stopping_rounds: Optional[int] = None,
          evals_result: Optional[Dict[str, Dict[str, List[float]]]] = None, verbose_eval: Any = True,
          xgb_model: Any = None, callbacks: Optional[Sequence[TrainingCallback]] = None,
          custom_metric: Optional[Callable] = None, feval: Optional[Callable] = None) -> Booster:
    """Train a booster for ``num_boost_round`` rounds (reference training.py:60-216)."""
    callbacks = [] if callbacks is None else copy.copy(list(callbacks))
    evals = list(evals) if evals else []
    for dmat, _ in evals:
        if not isinstance(dmat, DMatrix):
            raise TypeError("Invalid type for the `evals`.")
    bst = Booster(params, [dtrain] + [d for d, _ in evals], model_file=xgb_model)
    if verbose_eval:
        callbacks.append(EvaluationMonitor(period=1 if verbose_eval is True else int(verbose_eval)))
    if early_stopping_rounds:
        callbacks.append(EarlyStopping(rounds=early_stopping_rounds, maximize=maximize))
    container = CallbackContainer(callbacks, metric=custom_metric or feval, output_margin=callable(obj))
    bst = container.before_training(bst)
    for i in range(num_boost_round):
        if container.before_iteration(bst, i, dtrain, evals):
            break
        bst.update(dtrain, i, fobj=obj)
        if container.after_iteration(bst, i, dtrain, evals):
            break
    bst = container.after_training(bst)
    if evals_result is not None:
        evals_result.update(container.history)
    return bst.reset()


class CVPack:
    """One fold: its train and test matrices and booster (reference training.py:219)."""

    def __init__(self, dtrain: DMatrix, dtest: DMatrix, param: Any) -> None:
        self.dtrain = dtrain
        self.dtest = dtest
        self.watchlist = [(dtrain, "train"), (dtest, "test")]
        self.bst = Booster(param, [dtrain, dtest])

    def __getattr__(self, name: str) -> Any:
        def call(*args: Any, **kwargs: Any) -> Any:
            return getattr(self.bst, name)(*args, **kwargs)

        return call

    def update(self, iteration: int, fobj: Optional[Callable]) -> None:
        self.bst.update(self.dtrain, iteration, fobj)

    def eval(self, iteration: int, feval: Optional[Callable], output_margin: bool) -> str:
        return self.bst.eval_set(self.watchlist, iteration, feval, output_margin)


class _PackedBooster:
    """The folds as one model for the callbacks (reference training.py:246)."""

    def __init__(self, cvfolds: List[CVPack]) -> None:
        self.cvfolds = cvfolds

    def update(self, iteration: int, obj: Optional[Callable]) -> None:
        for fold in self.cvfolds:
            fold.update(iteration, obj)

    def eval(self, iteration: int, feval: Optional[Callable], output_margin: bool) -> List[str]:
        return [f.eval(iteration, feval, output_margin) for f in self.cvfolds]

    def set_attr(self, **kwargs: Any) -> None:
        for f in self.cvfolds:
            f.bst.set_attr(**kwargs)

    def attr(self, key: str) -> Optional[str]:
        return self.cvfolds[0].bst.attr(key)

    def set_param(self, params: Any, value: Any = None) -> None:
        for f in self.cvfolds:
            f.bst.set_param(params, value)

    def num_boosted_rounds(self) -> int:
        return self.cvfolds[0].bst.num_boosted_rounds()

    @property
    def best_iteration(self) -> int:
        return int(self.cvfolds[0].bst.attr("best_iteration"))

    @property
    def best_score(self) -> float:
        return float(self.cvfolds[0].bst.attr("best_score"))


def mknfold(*, dall: DMatrix, nfold: int, param: Dict[str, Any], seed: int, evals: Sequence[str] = (),
            fpreproc: Optional[Callable] = None, stratified: Optional[bool] = False, folds: Any = None,
            shuffle: bool = True) -> List[CVPack]:
    """The folds' CVPacks: built natively (XGDMatrixBuildCVFolds) unless
    ``folds`` gives index pairs or a splitter (reference training.py:363)."""
    evals = list(evals)
    np.random.seed(seed)
    if folds is None:
        c_train = (ctypes.c_void_p * nfold)()
        c_test = (ctypes.c_void_p * nfold)()
        _check_call(_LIB.XGDMatrixBuildCVFolds(dall.handle, ctypes.c_int(nfold), ctypes.c_uint(int(seed) & 0xFFFFFFFF),
                                               ctypes.c_int(1 if shuffle else 0), ctypes.c_int(1 if stratified else 0),
                                               c_train, c_test))
        pairs = [(DMatrix(ctypes.c_void_p(c_train[k])), DMatrix(ctypes.c_void_p(c_test[k]))) for k in range(nfold)]
    else:
        try:
            splits = [(x[0], x[1]) for x in folds]
        except TypeError:
            splits = list(folds.split(X=dall.get_label(), y=dall.get_label()))
        pairs = [(dall.slice(a), dall.slice(b)) for a, b in splits]
    packs = []
    base = dict(param)
    for dtrain, dtest in pairs:
        if fpreproc is not None:
            dtrain, dtest, tparam = fpreproc(dtrain, dtest, base.copy())
        else:
            tparam = base
        packs.append(CVPack(dtrain, dtest, list(tparam.items()) + [("eval_metric", m) for m in evals]))
    return packs


def cv(params: Any, dtrain: DMatrix, num_boost_round: int = 10, *, nfold: int = 3, stratified: bool = False,
       folds: Any = None, metrics: Sequence[str] = (), obj: Optional[Callable] = None, maximize: Optional[bool] = None,
       early_stopping_rounds: Optional[int] = None, fpreproc: Optional[Callable] = None, as_pandas: bool = True,
       verbose_eval: Any = None, show_stdv: bool = True, seed: int = 0,
       callbacks: Optional[Sequence[TrainingCallback]] = None, shuffle: bool = True,
       custom_metric: Optional[Callable] = None) -> Any:
    """Cross-validation: per-round mean and standard deviation of every
    train/test metric over the folds (reference training.py:437)."""
    if isinstance(metrics, str):
        metrics = [metrics]
    metrics = list(metrics)
    if isinstance(params, list):
        listed = [v for k, v in params if k == "eval_metric"]
        params = dict(params)
        if listed:
            params["eval_metric"] = listed
    else:
        params = dict(params)
    if not metrics and "eval_metric" in params:
        metrics = list(params["eval_metric"]) if isinstance(params["eval_metric"], list) else [params["eval_metric"]]
    params.pop("eval_metric", None)
    cvfolds = mknfold(dall=dtrain, nfold=nfold, param=params, seed=seed, evals=metrics, fpreproc=fpreproc,
                      stratified=stratified, folds=folds, shuffle=shuffle)
    callbacks = [] if callbacks is None else copy.copy(list(callbacks))
    if verbose_eval:
        callbacks.append(EvaluationMonitor(period=1 if verbose_eval is True else int(verbose_eval),
                                           show_stdv=show_stdv))
    if early_stopping_rounds:
        callbacks.append(EarlyStopping(rounds=early_stopping_rounds, maximize=maximize))
    container = CallbackContainer(callbacks, metric=custom_metric, is_cv=True)
    booster = _PackedBooster(cvfolds)
    container.before_training(booster)
    results: Dict[str, List[float]] = {}
    for i in range(num_boost_round):
        if container.before_iteration(booster, i, dtrain, None):
            break
        booster.update(i, obj)
        stop = container.after_iteration(booster, i, dtrain, None)
        for key, mean, std in container.aggregated_cv or []:
            results.setdefault(key + "-mean", []).append(mean)
            results.setdefault(key + "-std", []).append(std)
        if stop:
            for k in results:
                results[k] = results[k][: booster.best_iteration + 1]
            break
    container.after_training(booster)
    if as_pandas:
        try:
            import pandas as pd

            return pd.DataFrame.from_dict(results)
        except ImportError:
            pass
    return results


__all__ = ["train", "cv", "CVPack", "mknfold", "XGBoostError"]
