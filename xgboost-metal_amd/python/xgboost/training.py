"""``xgb.train`` and ``xgb.cv``.

The signatures, defaults and results are the reference package's
(python-package/xgboost/training.py:60-560):

- ``train`` boosts ``num_boost_round`` rounds on ``dtrain``, evaluates the
  ``evals`` matrices after every round, prints the scores (``verbose_eval``:
  True = every round, n = every n-th round), stops early after
  ``early_stopping_rounds`` rounds without improvement of the last metric on
  the last evaluation set, fills ``evals_result`` with the history and runs
  user ``callbacks``; it returns the booster with its training caches
  released (``Booster.reset``).
- ``cv`` trains one booster per fold and returns, per round, the mean and
  standard deviation over the folds of every train/test metric, as a pandas
  DataFrame when pandas is importable (``as_pandas``) and a dict of lists
  otherwise; early stopping keeps the rounds up to the best one.  Folds are
  built by the library (``XGDMatrixBuildCVFolds``: shuffled or not, with
  the ``std_shuffle`` parameter's draws like the column sample,
  stratified or not, from ``seed``) unless ``folds`` gives (train, test)
  index pairs or a splitter object.
"""
from __future__ import annotations

import ctypes
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .callback import CallbackContainer, EarlyStopping, EvaluationMonitor, TrainingCallback
from .config import config_context
from .core import _LIB, Booster, DMatrix, XGBoostError, _check_call

__all__ = ["train", "cv", "XGBoostError"]


def _default_callbacks(user: Optional[Sequence[TrainingCallback]], verbose_eval: Any,
                       early_stopping_rounds: Optional[int], maximize: Optional[bool],
                       show_stdv: bool = False) -> List[TrainingCallback]:
    """The user's callbacks, then the printer and the early stopper the
    keyword arguments ask for (the caller's list is not modified)."""
    hooks = list(user or [])
    if verbose_eval:
        period = 1 if verbose_eval is True else int(verbose_eval)
        hooks.append(EvaluationMonitor(period=period, show_stdv=show_stdv))
    if early_stopping_rounds:
        hooks.append(EarlyStopping(rounds=early_stopping_rounds, maximize=maximize))
    return hooks


def _boost(model: Any, rounds: int, container: CallbackContainer, step: Callable[[int], None],
           dtrain: DMatrix, watch: Optional[List[Tuple[DMatrix, str]]],
           record: Optional[Callable[[], None]] = None) -> Tuple[Any, bool]:
    """Runs up to ``rounds`` rounds of ``step`` between the container's hooks
    (``record`` after each round's evaluation).  Returns the model that
    after_training hands back and whether an after-round hook stopped the
    training."""
    model = container.before_training(model)
    stopped = False
    for rnd in range(rounds):
        if container.before_iteration(model, rnd, dtrain, watch):
            break
        step(rnd)
        stopped = container.after_iteration(model, rnd, dtrain, watch)
        if record is not None:
            record()
        if stopped:
            break
    return container.after_training(model), stopped


def train(params: Dict[str, Any], dtrain: DMatrix, num_boost_round: int = 10, *,
          evals: Optional[Sequence[Tuple[DMatrix, str]]] = None, obj: Optional[Callable] = None,
          maximize: Optional[bool] = None, early_stopping_rounds: Optional[int] = None,
          evals_result: Optional[Dict[str, Dict[str, List[float]]]] = None, verbose_eval: Any = True,
          xgb_model: Any = None, callbacks: Optional[Sequence[TrainingCallback]] = None,
          custom_metric: Optional[Callable] = None, feval: Optional[Callable] = None) -> Booster:
    """Trains a booster; see the module docstring for the rules."""
    watch = [] if evals is None else list(evals)
    if not all(isinstance(pair, (tuple, list)) and len(pair) == 2 and isinstance(pair[0], DMatrix)
               for pair in watch):
        raise TypeError("evals must be a sequence of (DMatrix, name) pairs")
    booster = Booster(params, [dtrain, *(dmat for dmat, _ in watch)], model_file=xgb_model)
    container = CallbackContainer(_default_callbacks(callbacks, verbose_eval, early_stopping_rounds, maximize),
                                  metric=custom_metric or feval, output_margin=callable(obj))

    def step(rnd: int) -> None:
        booster.update(dtrain, rnd, fobj=obj)

    trained, _ = _boost(booster, num_boost_round, container, step, dtrain, watch)
    if evals_result is not None:
        evals_result.update(container.history)
    return trained.reset()


class _Fold:
    """One cross-validation fold: its train and test matrices and booster."""

    def __init__(self, dtrain: DMatrix, dtest: DMatrix, params: Any) -> None:
        self.dtrain, self.dtest = dtrain, dtest
        self.booster = Booster(params, [dtrain, dtest])

    def evaluation(self, rnd: int, metric: Optional[Callable], output_margin: bool) -> str:
        return self.booster.eval_set([(self.dtrain, "train"), (self.dtest, "test")], rnd, metric, output_margin)


class _FoldSet:
    """The folds seen by the callbacks as one model: updates, parameters and
    attributes go to every fold, ``eval`` gives each fold's evaluation line,
    and best round, score and round count are read from the first fold."""

    def __init__(self, folds: List[_Fold]) -> None:
        self.folds = folds

    def update(self, rnd: int, obj: Optional[Callable]) -> None:
        for fold in self.folds:
            fold.booster.update(fold.dtrain, rnd, fobj=obj)

    def eval(self, rnd: int, metric: Optional[Callable], output_margin: bool) -> List[str]:
        return [fold.evaluation(rnd, metric, output_margin) for fold in self.folds]

    def set_param(self, params: Any, value: Any = None) -> None:
        for fold in self.folds:
            fold.booster.set_param(params, value)

    def set_attr(self, **kwargs: Any) -> None:
        for fold in self.folds:
            fold.booster.set_attr(**kwargs)

    def attr(self, key: str) -> Optional[str]:
        return self.folds[0].booster.attr(key)

    def num_boosted_rounds(self) -> int:
        return self.folds[0].booster.num_boosted_rounds()

    @property
    def best_iteration(self) -> int:
        return int(self.attr("best_iteration"))

    @property
    def best_score(self) -> float:
        return float(self.attr("best_score"))


def _fold_matrices(dall: DMatrix, nfold: int, seed: int, stratified: bool, shuffle: bool,
                   folds: Any, std_shuffle: Optional[str] = None) -> List[Tuple[DMatrix, DMatrix]]:
    if folds is None:
        train_handles = (ctypes.c_void_p * nfold)()
        test_handles = (ctypes.c_void_p * nfold)()
        # The fold shuffle draws like the column sample: the parameters'
        # std_shuffle, else the global config's (default libstdc++).
        with config_context(**({} if std_shuffle is None else {"std_shuffle": std_shuffle})):
            _check_call(_LIB.XGDMatrixBuildCVFolds(dall.handle, ctypes.c_int(nfold),
                                                   ctypes.c_uint(int(seed) & 0xFFFFFFFF),
                                                   ctypes.c_int(int(bool(shuffle))), ctypes.c_int(int(bool(stratified))),
                                                   train_handles, test_handles))
        return [(DMatrix(ctypes.c_void_p(train_handles[k])), DMatrix(ctypes.c_void_p(test_handles[k])))
                for k in range(nfold)]
    if hasattr(folds, "split"):  # a scikit-learn style splitter
        labels = dall.get_label()
        index_pairs = list(folds.split(X=labels, y=labels))
    else:
        index_pairs = [(pair[0], pair[1]) for pair in folds]
    return [(dall.slice(tr), dall.slice(te)) for tr, te in index_pairs]


def _metric_list(params: Any, metrics: Any) -> Tuple[Dict[str, Any], List[str]]:
    """Parameters without eval_metric, and the metrics to report: ``metrics``
    if given, else the parameters' eval_metric (one or a list; in a list of
    pairs, every eval_metric entry)."""
    if isinstance(params, dict):
        pairs = list(params.items())
    else:
        pairs = list(params)
    listed: List[str] = []
    for key, value in pairs:
        if key == "eval_metric":
            listed.extend(value if isinstance(value, (list, tuple)) else [value])
    rest = {key: value for key, value in pairs if key != "eval_metric"}
    chosen = [metrics] if isinstance(metrics, str) else list(metrics or [])
    return rest, chosen or listed


def cv(params: Any, dtrain: DMatrix, num_boost_round: int = 10, *, nfold: int = 3, stratified: bool = False,
       folds: Any = None, metrics: Sequence[str] = (), obj: Optional[Callable] = None, maximize: Optional[bool] = None,
       early_stopping_rounds: Optional[int] = None, fpreproc: Optional[Callable] = None, as_pandas: bool = True,
       verbose_eval: Any = None, show_stdv: bool = True, seed: int = 0,
       callbacks: Optional[Sequence[TrainingCallback]] = None, shuffle: bool = True,
       custom_metric: Optional[Callable] = None) -> Any:
    """Cross-validation; see the module docstring for the rules."""
    np.random.seed(seed)  # as the reference does: splitters that draw from numpy's global generator
    base, chosen = _metric_list(params, metrics)
    fold_list = []
    for fold_train, fold_test in _fold_matrices(dtrain, nfold, seed, stratified, shuffle, folds,
                                                base.get("std_shuffle")):
        fold_params = dict(base)
        if fpreproc is not None:
            fold_train, fold_test, fold_params = fpreproc(fold_train, fold_test, dict(base))
        fold_list.append(_Fold(fold_train, fold_test,
                               list(fold_params.items()) + [("eval_metric", m) for m in chosen]))
    model = _FoldSet(fold_list)
    container = CallbackContainer(_default_callbacks(callbacks, verbose_eval, early_stopping_rounds, maximize,
                                                     show_stdv=show_stdv),
                                  metric=custom_metric, is_cv=True)
    table: Dict[str, List[float]] = {}

    def step(rnd: int) -> None:
        model.update(rnd, obj)

    def record() -> None:
        for key, mean, std in container.aggregated_cv or []:
            table.setdefault(key + "-mean", []).append(mean)
            table.setdefault(key + "-std", []).append(std)

    _, stopped = _boost(model, num_boost_round, container, step, dtrain, None, record)
    if stopped:
        # Stopped by a callback (early stopping): keep the rounds up to the best.
        table = {key: values[: model.best_iteration + 1] for key, values in table.items()}
    if as_pandas:
        try:
            import pandas as pd
        except ImportError:
            return table
        return pd.DataFrame.from_dict(table)
    return table
