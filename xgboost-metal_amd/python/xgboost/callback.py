"""Training callbacks (reference python-package/xgboost/callback.py:50-640).

``train`` and ``cv`` drive a ``CallbackContainer``: it evaluates the watched
matrices after every round, records the scores in an ordered history
``{data_name: {metric_name: [score, ...]}}`` and asks each callback whether
to stop.  ``EarlyStopping``, ``EvaluationMonitor``, ``LearningRateScheduler``
and ``TrainingCheckPoint`` keep the upstream names, arguments and rules.
"""
from __future__ import annotations

import collections
import os
import pickle
from abc import ABC
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple, Union

import numpy as np

from .core import Booster, DMatrix, XGBoostError

EvalsLog = Dict[str, Dict[str, Union[List[float], List[Tuple[float, float]]]]]

__all__ = ["TrainingCallback", "CallbackContainer", "LearningRateScheduler", "EarlyStopping", "EvaluationMonitor",
           "TrainingCheckPoint"]


class TrainingCallback(ABC):
    """Base class: override any of the four hooks (reference callback.py:50).

    ``before_iteration`` and ``after_iteration`` return True to stop training.
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


def parse_eval_str(result: str) -> List[Tuple[str, float]]:
    """``"[3]\\ttrain-rmse:0.5\\tvalid-rmse:0.7"`` -> ``[("train-rmse", 0.5), ...]``."""
    out = []
    for item in result.split()[1:]:
        name, value = item.rsplit(":", 1)
        out.append((name, float(value)))
    return out


def aggregate_cv(results: List[str]) -> List[Tuple[str, float, float]]:
    """Mean and standard deviation of each ``data-metric`` over the folds'
    evaluation strings, in first-seen order (reference callback.py:99)."""
    scores: Dict[str, List[float]] = collections.OrderedDict()
    for line in results:
        for name, value in parse_eval_str(line):
            scores.setdefault(name, []).append(value)
    return [(name, float(np.mean(v)), float(np.std(v))) for name, v in scores.items()]


class CallbackContainer:
    """Runs a list of callbacks and keeps the evaluation history (reference callback.py:151)."""

    def __init__(self, callbacks: Sequence[TrainingCallback], metric: Optional[Callable] = None,
                 output_margin: bool = True, is_cv: bool = False) -> None:
        self.callbacks = list(dict.fromkeys(callbacks))
        for cb in self.callbacks:
            if not isinstance(cb, TrainingCallback):
                raise TypeError("callback must be an instance of `TrainingCallback`.")
        if metric is not None and not callable(metric):
            raise TypeError("metric must be callable object for monitoring.  For builtin metrics, passing them in "
                            "training parameter invokes monitor automatically.")
        self.metric = metric
        self.history: EvalsLog = collections.OrderedDict()
        self._output_margin = output_margin
        self.is_cv = is_cv
        self.aggregated_cv: Optional[List[Tuple[str, float, float]]] = None

    def before_training(self, model: Any) -> Any:
        for cb in self.callbacks:
            model = cb.before_training(model=model)
            if not self.is_cv and not isinstance(model, Booster):
                raise TypeError("before_training should return the model")
        return model

    def after_training(self, model: Any) -> Any:
        for cb in self.callbacks:
            model = cb.after_training(model=model)
            if not self.is_cv and not isinstance(model, Booster):
                raise TypeError("after_training should return the model")
        return model

    def before_iteration(self, model: Any, epoch: int, dtrain: DMatrix,
                         evals: Optional[List[Tuple[DMatrix, str]]]) -> bool:
        return any(cb.before_iteration(model, epoch, self.history) for cb in self.callbacks)

    def _update_history(self, scores: Sequence[Tuple], epoch: int) -> None:
        for item in scores:
            data_name, metric_name = item[0].split("-", 1)
            value = (item[1], item[2]) if self.is_cv else item[1]
            self.history.setdefault(data_name, collections.OrderedDict()).setdefault(metric_name, []).append(value)

    def after_iteration(self, model: Any, epoch: int, dtrain: DMatrix,
                        evals: Optional[List[Tuple[DMatrix, str]]]) -> bool:
        if self.is_cv:
            scores = aggregate_cv(model.eval(epoch, self.metric, self._output_margin))
            self.aggregated_cv = scores
            self._update_history(scores, epoch)
        else:
            evals = evals or []
            for _, name in evals:
                if "-" in name:
                    raise ValueError("Dataset name should not contain `-`")
            if evals:
                self._update_history(parse_eval_str(model.eval_set(evals, epoch, self.metric,
                                                                   self._output_margin)), epoch)
        return any(cb.after_iteration(model, epoch, self.history) for cb in self.callbacks)


class LearningRateScheduler(TrainingCallback):
    """Sets ``learning_rate`` after every round from a list or a function of the round (reference callback.py:274)."""

    def __init__(self, learning_rates: Union[Callable[[int], float], Sequence[float]]) -> None:
        if callable(learning_rates):
            self.learning_rates = learning_rates
        elif isinstance(learning_rates, collections.abc.Sequence):
            rates = list(learning_rates)
            self.learning_rates = lambda epoch: rates[epoch]
        else:
            raise TypeError(f"Invalid learning rates, expecting callable or sequence, got: {type(learning_rates)}")
        super().__init__()

    def after_iteration(self, model: Any, epoch: int, evals_log: EvalsLog) -> bool:
        model.set_param("learning_rate", self.learning_rates(epoch))
        return False


_MAXIMIZE_PREFIXES = ("auc", "aucpr", "pre", "pre@", "map", "ndcg", "auc@", "aucpr@", "map@", "ndcg@")


class EarlyStopping(TrainingCallback):
    """Stops when the watched score has not improved for ``rounds`` rounds (reference callback.py:313).

    The score is the last metric of the last evaluation matrix unless
    ``metric_name`` / ``data_name`` say otherwise; ``maximize=None`` picks
    maximisation for AUC-like metrics.  The best round and score are stored
    as the booster attributes ``best_iteration`` and ``best_score``;
    ``save_best`` returns the model cut after the best round.
    """

    def __init__(self, *, rounds: int, metric_name: Optional[str] = None, data_name: Optional[str] = None,
                 maximize: Optional[bool] = None, save_best: Optional[bool] = False, min_delta: float = 0.0) -> None:
        if min_delta < 0:
            raise ValueError("min_delta must be greater or equal to 0.")
        self.data = data_name
        self.metric_name = metric_name
        self.rounds = rounds
        self.save_best = save_best
        self.maximize = maximize
        self._min_delta = min_delta
        self.stopping_history: EvalsLog = {}
        self.best_scores: Dict[str, Dict[str, list]] = {}
        self.current_rounds = 0
        self.starting_round = 0
        super().__init__()

    def before_training(self, model: Any) -> Any:
        self.starting_round = model.num_boosted_rounds()
        if not isinstance(model, Booster) and self.save_best:
            raise ValueError("`save_best` is not applicable to the `cv` function as it doesn't return a model.")
        return model

    @staticmethod
    def _value(score: Any) -> float:
        return score[0] if isinstance(score, tuple) else score

    def _improved(self, new: Any, best: Any) -> bool:
        if self.maximize:
            return (self._value(new) - self._min_delta) > self._value(best)
        return (self._value(best) - self._min_delta) > self._value(new)

    def _update_rounds(self, score: Any, name: str, metric: str, model: Any, epoch: int) -> bool:
        if self.maximize is None:
            self.maximize = metric != "mape" and any(metric.startswith(p) for p in _MAXIMIZE_PREFIXES)
        if not self.stopping_history:
            self.current_rounds = 0
            self.stopping_history[name] = {metric: [score]}
            self.best_scores[name] = {metric: [score]}
            model.set_attr(best_score=str(self._value(score)), best_iteration=str(epoch))
        elif not self._improved(score, self.best_scores[name][metric][-1]):
            self.stopping_history[name][metric].append(score)
            self.current_rounds += 1
        else:
            self.stopping_history[name][metric].append(score)
            self.best_scores[name][metric].append(score)
            model.set_attr(best_score=str(self._value(score)), best_iteration=str(epoch))
            self.current_rounds = 0
        return self.current_rounds >= self.rounds

    def after_iteration(self, model: Any, epoch: int, evals_log: EvalsLog) -> bool:
        epoch += self.starting_round  # continued training counts from the loaded rounds
        if len(evals_log) < 1:
            raise ValueError("Must have at least 1 validation dataset for early stopping.")
        data_name = self.data if self.data else list(evals_log.keys())[-1]
        if data_name not in evals_log:
            raise ValueError(f"No dataset named: {data_name}")
        data_log = evals_log[data_name]
        metric_name = self.metric_name if self.metric_name else list(data_log.keys())[-1]
        if metric_name not in data_log:
            raise ValueError(f"No metric named: {metric_name}")
        return self._update_rounds(data_log[metric_name][-1], data_name, metric_name, model, epoch)

    def after_training(self, model: Any) -> Any:
        if not self.save_best:
            return model
        best_iteration, best_score = model.best_iteration, model.best_score
        model = model[: best_iteration + 1]
        model.best_iteration = best_iteration
        model.best_score = best_score
        return model


class EvaluationMonitor(TrainingCallback):
    """Prints ``[epoch]\\tdata-metric:score`` every ``period`` rounds (reference callback.py:513)."""

    def __init__(self, rank: int = 0, period: int = 1, show_stdv: bool = False,
                 logger: Callable[[str], None] = lambda msg: print(msg, end="")) -> None:
        if period <= 0:
            raise ValueError("period must be positive")
        self.printer_rank = rank
        self.show_stdv = show_stdv
        self.period = period
        self._logger = logger
        self._latest: Optional[str] = None
        super().__init__()

    def _fmt_metric(self, data: str, metric: str, score: float, std: Optional[float]) -> str:
        if std is not None and self.show_stdv:
            return f"\t{data}-{metric}:{score:.5f}+{std:.5f}"
        return f"\t{data}-{metric}:{score:.5f}"

    def after_iteration(self, model: Any, epoch: int, evals_log: EvalsLog) -> bool:
        if not evals_log:
            return False
        msg = f"[{epoch}]"
        for data, metrics in evals_log.items():
            for metric_name, log in metrics.items():
                last = log[-1]
                score, std = (last[0], last[1]) if isinstance(last, tuple) else (last, None)
                msg += self._fmt_metric(data, metric_name, score, std)
        msg += "\n"
        if epoch % self.period == 0 or self.period == 1:
            self._logger(msg)
            self._latest = None
        else:
            self._latest = msg
        return False

    def after_training(self, model: Any) -> Any:
        if self._latest is not None:
            self._logger(self._latest)
        return model


class TrainingCheckPoint(TrainingCallback):
    """Saves the model every ``interval`` rounds as ``name_<round>.ubj`` (reference callback.py:588)."""

    default_format = "ubj"

    def __init__(self, directory: Union[str, os.PathLike], name: str = "model", as_pickle: bool = False,
                 interval: int = 100) -> None:
        self._path = os.fspath(directory)
        self._name = name
        self._as_pickle = as_pickle
        self._iterations = interval
        self._epoch = 0
        self._start = 0
        super().__init__()

    def before_training(self, model: Any) -> Any:
        self._start = model.num_boosted_rounds()
        return model

    def after_iteration(self, model: Any, epoch: int, evals_log: EvalsLog) -> bool:
        if self._epoch == self._iterations:
            suffix = ".pkl" if self._as_pickle else f".{self.default_format}"
            path = os.path.join(self._path, f"{self._name}_{epoch + self._start}{suffix}")
            self._epoch = 0
            if self._as_pickle:
                with open(path, "wb") as fd:
                    pickle.dump(model, fd)
            else:
                model.save_model(path)
        self._epoch += 1
        return False
