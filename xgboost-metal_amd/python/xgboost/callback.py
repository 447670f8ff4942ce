"""Training callbacks: the hooks ``train`` and ``cv`` call around every
boosting round.

The public classes keep the reference package's names, constructor
arguments and rules (python-package/xgboost/callback.py:50-640):

- ``TrainingCallback``: four hooks; ``before_iteration`` / ``after_iteration``
  return True to stop.
- ``CallbackContainer``: evaluates the watched matrices after each round and
  keeps the history ``{data name: {metric name: [score per round]}}`` (in
  ``cv``, each score is a ``(mean, std)`` pair over the folds).
- ``EarlyStopping``: stops after ``rounds`` rounds without improvement of one
  watched score.
- ``EvaluationMonitor``: prints ``[round]\\tdata-metric:score`` lines.
- ``LearningRateScheduler``: sets ``learning_rate`` after every round.
- ``TrainingCheckPoint``: saves the model every ``interval`` rounds.
"""
from __future__ import annotations

import os
import pickle
from abc import ABC
from collections.abc import Sequence as SequenceABC
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple, Union

import numpy as np

from .core import Booster, DMatrix

EvalsLog = Dict[str, Dict[str, Union[List[float], List[Tuple[float, float]]]]]

__all__ = ["TrainingCallback", "CallbackContainer", "LearningRateScheduler", "EarlyStopping", "EvaluationMonitor",
           "TrainingCheckPoint"]


class TrainingCallback(ABC):
    """Base class of training callbacks; every hook is optional.

    ``model`` is the Booster in ``train`` and the set of fold boosters in
    ``cv``; ``epoch`` counts the rounds of this call from 0; ``evals_log`` is
    the evaluation history so far.
    """

    EvalsLog = EvalsLog

    def __init__(self) -> None:
        pass

    def before_training(self, model: Any) -> Any:
        return model

    def after_training(self, model: Any) -> Any:
        return model

    def before_iteration(self, model: Any, epoch: int, evals_log: EvalsLog) -> bool:
        return False

    def after_iteration(self, model: Any, epoch: int, evals_log: EvalsLog) -> bool:
        return False


def _scores(line: str) -> List[Tuple[str, float]]:
    """("data-metric", value) pairs of one evaluation line
    ``[round]<TAB>data-metric:value<TAB>...``."""
    fields = line.strip().split("\t")[1:]
    pairs = []
    for field in fields:
        key, _, value = field.rpartition(":")
        pairs.append((key, float(value)))
    return pairs


def _fold_statistics(lines: Sequence[str]) -> List[Tuple[str, float, float]]:
    """Mean and (population) standard deviation of every ``data-metric`` over
    the folds' evaluation lines, keys in the order first met."""
    keys: List[str] = []
    values: Dict[str, List[float]] = {}
    for line in lines:
        for key, value in _scores(line):
            if key not in values:
                keys.append(key)
                values[key] = []
            values[key].append(value)
    return [(k, float(np.mean(values[k])), float(np.std(values[k]))) for k in keys]


class CallbackContainer:
    """Runs callbacks around the rounds and evaluates the watched matrices.

    ``metric`` is a custom metric ``f(predt, dmatrix) -> (name, value)``;
    ``output_margin`` hands it raw margins (a custom objective trains on
    margins); ``is_cv`` switches to fold statistics.
    """

    def __init__(self, callbacks: Sequence[TrainingCallback], metric: Optional[Callable] = None,
                 output_margin: bool = True, is_cv: bool = False) -> None:
        self.callbacks: List[TrainingCallback] = []
        for cb in callbacks:
            if not isinstance(cb, TrainingCallback):
                raise TypeError(f"callbacks must be TrainingCallback instances, got {type(cb).__name__}")
            if not any(cb is seen for seen in self.callbacks):
                self.callbacks.append(cb)
        if metric is not None and not callable(metric):
            raise TypeError("a custom metric must be callable; built-in metrics are chosen with the "
                            "eval_metric parameter")
        self.metric = metric
        self.history: EvalsLog = {}
        self._output_margin = output_margin
        self.is_cv = is_cv
        # cv: the last round's (data-metric, mean, std) triples.
        self.aggregated_cv: Optional[List[Tuple[str, float, float]]] = None

    def _each(self, hook: str, model: Any, *args: Any) -> bool:
        # The first callback that asks to stop ends the round: later ones are
        # not called for it.
        for cb in self.callbacks:
            if getattr(cb, hook)(model, *args):
                return True
        return False

    def _chain(self, hook: str, model: Any) -> Any:
        for cb in self.callbacks:
            model = getattr(cb, hook)(model)
            if not self.is_cv and not isinstance(model, Booster):
                raise TypeError(f"{type(cb).__name__}.{hook} must return the model")
        return model

    def before_training(self, model: Any) -> Any:
        return self._chain("before_training", model)

    def after_training(self, model: Any) -> Any:
        return self._chain("after_training", model)

    def before_iteration(self, model: Any, epoch: int, dtrain: DMatrix,
                         evals: Optional[List[Tuple[DMatrix, str]]]) -> bool:
        return self._each("before_iteration", model, epoch, self.history)

    def _record(self, key: str, score: Any) -> None:
        data, _, metric = key.partition("-")
        self.history.setdefault(data, {}).setdefault(metric, []).append(score)

    def after_iteration(self, model: Any, epoch: int, dtrain: DMatrix,
                        evals: Optional[List[Tuple[DMatrix, str]]]) -> bool:
        if self.is_cv:
            self.aggregated_cv = _fold_statistics(model.eval(epoch, self.metric, self._output_margin))
            for key, mean, std in self.aggregated_cv:
                self._record(key, (mean, std))
        elif evals:
            if any("-" in name for _, name in evals):
                raise ValueError("evaluation set names must not contain '-'")
            for key, value in _scores(model.eval_set(evals, epoch, self.metric, self._output_margin)):
                self._record(key, value)
        return self._each("after_iteration", model, epoch, self.history)


class LearningRateScheduler(TrainingCallback):
    """After round ``epoch``, sets ``learning_rate`` to ``learning_rates(epoch)``
    (a function of the round) or ``learning_rates[epoch]`` (a sequence), so
    round ``epoch + 1`` trains at that rate."""

    def __init__(self, learning_rates: Union[Callable[[int], float], Sequence[float]]) -> None:
        if callable(learning_rates):
            self._rate_of = learning_rates
        elif isinstance(learning_rates, SequenceABC):
            table = list(learning_rates)
            self._rate_of = table.__getitem__
        else:
            raise TypeError(f"learning_rates must be a function of the round or a sequence, "
                            f"not {type(learning_rates).__name__}")
        super().__init__()

    def after_iteration(self, model: Any, epoch: int, evals_log: EvalsLog) -> bool:
        model.set_param("learning_rate", self._rate_of(epoch))
        return False


def _higher_is_better(metric: str) -> bool:
    """Metrics named auc*, pre*, map* or ndcg* (AUC, AUC-PR, precision, MAP,
    NDCG and their @k forms) improve upwards, except mape; all others
    downwards."""
    return metric != "mape" and metric.startswith(("auc", "pre", "map", "ndcg"))


class EarlyStopping(TrainingCallback):
    """Stops training once the watched score has gone ``rounds`` rounds
    without improving.

    The watched score is ``metric_name`` of ``data_name``, by default the last
    metric of the last evaluation set.  A score improves when it beats the
    best so far by more than ``min_delta`` (upwards when ``maximize``,
    downwards otherwise; ``maximize=None`` decides from the metric's name).
    Each new best is stored in the model attributes ``best_iteration`` (rounds
    counted from the start of the model, continued training included) and
    ``best_score``.  With ``save_best`` the model returned by training ends at
    the best round (``train`` only).
    """

    def __init__(self, *, rounds: int, metric_name: Optional[str] = None, data_name: Optional[str] = None,
                 maximize: Optional[bool] = None, save_best: Optional[bool] = False, min_delta: float = 0.0) -> None:
        if min_delta < 0:
            raise ValueError("min_delta must not be negative")
        self.rounds = rounds
        self.metric_name = metric_name
        self.data = data_name
        self.maximize = maximize
        self.save_best = save_best
        self._min_delta = min_delta
        self._best: Optional[float] = None
        self._since_best = 0
        self._offset = 0
        super().__init__()

    def before_training(self, model: Any) -> Any:
        if self.save_best and not isinstance(model, Booster):
            raise ValueError("save_best needs a model to cut; cv returns none")
        self._offset = model.num_boosted_rounds()
        return model

    def _watched(self, evals_log: EvalsLog) -> Tuple[str, str]:
        if not evals_log:
            raise ValueError("early stopping needs at least one evaluation set")
        data = self.data or next(reversed(evals_log))
        if data not in evals_log:
            raise ValueError(f"no evaluation set named {data!r}")
        metrics = evals_log[data]
        metric = self.metric_name or next(reversed(metrics))
        if metric not in metrics:
            raise ValueError(f"no metric named {metric!r} in evaluation set {data!r}")
        return data, metric

    def after_iteration(self, model: Any, epoch: int, evals_log: EvalsLog) -> bool:
        data, metric = self._watched(evals_log)
        latest = evals_log[data][metric][-1]
        score = latest[0] if isinstance(latest, tuple) else latest  # cv: the fold mean
        if self.maximize is None:
            self.maximize = _higher_is_better(metric)
        if self._best is None:
            improved = True
        elif self.maximize:
            improved = score - self._min_delta > self._best
        else:
            improved = self._best - self._min_delta > score
        if improved:
            self._best = score
            self._since_best = 0
            model.set_attr(best_score=str(score), best_iteration=str(epoch + self._offset))
            return False
        self._since_best += 1
        return self._since_best >= self.rounds

    def after_training(self, model: Any) -> Any:
        if not self.save_best:
            return model
        best_iteration, best_score = model.best_iteration, model.best_score
        kept = model[: best_iteration + 1]
        kept.best_iteration = best_iteration
        kept.best_score = best_score
        return kept


class EvaluationMonitor(TrainingCallback):
    """Prints each round's scores as ``[round]\\tdata-metric:score`` (five
    decimals; ``+std`` in cv when ``show_stdv``) on rounds that are multiples of
    ``period``; the last round's line is printed at the end if its round was
    skipped."""

    def __init__(self, rank: int = 0, period: int = 1, show_stdv: bool = False,
                 logger: Callable[[str], None] = lambda msg: print(msg, end="")) -> None:
        if period <= 0:
            raise ValueError("period must be positive")
        self.printer_rank = rank
        self.period = period
        self.show_stdv = show_stdv
        self._logger = logger
        self._unprinted: Optional[str] = None
        super().__init__()

    def _line(self, epoch: int, evals_log: EvalsLog) -> str:
        parts = [f"[{epoch}]"]
        for data, metrics in evals_log.items():
            for metric, log in metrics.items():
                last = log[-1]
                if isinstance(last, tuple):
                    mean, std = last
                    text = f"{mean:.5f}+{std:.5f}" if self.show_stdv else f"{mean:.5f}"
                else:
                    text = f"{last:.5f}"
                parts.append(f"{data}-{metric}:{text}")
        return "\t".join(parts) + "\n"

    def after_iteration(self, model: Any, epoch: int, evals_log: EvalsLog) -> bool:
        if evals_log:
            line = self._line(epoch, evals_log)
            if epoch % self.period == 0:
                self._logger(line)
                self._unprinted = None
            else:
                self._unprinted = line
        return False

    def after_training(self, model: Any) -> Any:
        if self._unprinted is not None:
            self._logger(self._unprinted)
            self._unprinted = None
        return model


class TrainingCheckPoint(TrainingCallback):
    """Saves the model after every round whose number (counted from 0 in
    this call) is a positive multiple of ``interval``, to
    ``directory/name_<rounds in the model before training + round>.ubj``
    (``.pkl``, pickled, with ``as_pickle``)."""

    default_format = "ubj"

    def __init__(self, directory: Union[str, os.PathLike], name: str = "model", as_pickle: bool = False,
                 interval: int = 100) -> None:
        self._directory = os.fspath(directory)
        self._name = name
        self._as_pickle = as_pickle
        self._interval = interval
        self._offset = 0
        super().__init__()

    def before_training(self, model: Any) -> Any:
        self._offset = model.num_boosted_rounds()
        return model

    def after_iteration(self, model: Any, epoch: int, evals_log: EvalsLog) -> bool:
        if epoch > 0 and epoch % self._interval == 0:
            suffix = "pkl" if self._as_pickle else self.default_format
            path = os.path.join(self._directory, f"{self._name}_{epoch + self._offset}.{suffix}")
            if self._as_pickle:
                with open(path, "wb") as out:
                    pickle.dump(model, out)
            else:
                model.save_model(path)
        return False
