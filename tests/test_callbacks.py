"""The callback rules of xgboost.callback on the CPU, with a stand-in model
(the same rules as the reference package's callback.py:151-640): early
stopping's improvement test, direction, counting and attributes; the
monitor's line format and period; the scheduler's rates; the checkpoint's
rounds; the container's history and stop semantics."""
import os

import pytest

import xgboost as xgb
from xgboost.callback import CallbackContainer, _fold_statistics, _scores


class Model:
    """Records what the callbacks do to a booster."""

    def __init__(self, rounds=0):
        self.attrs, self.params, self.saved, self.rounds = {}, [], [], rounds

    def set_attr(self, **kw):
        self.attrs.update(kw)

    def set_param(self, key, value=None):
        self.params.append((key, value))

    def num_boosted_rounds(self):
        return self.rounds

    def save_model(self, path):
        self.saved.append(os.path.basename(path))


def _run(cb, scores, name="valid", metric="rmse", model=None):
    model = model or Model()
    cb.before_training(model)
    log = {name: {metric: []}}
    for epoch, s in enumerate(scores):
        log[name][metric].append(s)
        if cb.after_iteration(model, epoch, log):
            return model, epoch
    return model, None


def test_early_stopping_minimises_and_counts():
    es = xgb.callback.EarlyStopping(rounds=2)
    model, stopped = _run(es, [5.0, 4.0, 4.0, 3.9, 4.1, 4.2])
    assert stopped == 5 and model.attrs == {"best_score": "3.9", "best_iteration": "3"}


def test_early_stopping_min_delta_and_maximize_inference():
    # 0.705 does not beat 0.70 by more than 0.01; auc is maximised.
    model, stopped = _run(xgb.callback.EarlyStopping(rounds=2, min_delta=0.01), [0.7, 0.705, 0.709],
                          metric="auc")
    assert stopped == 2 and model.attrs["best_iteration"] == "0"
    # mape is minimised although it starts with "map"; map@3 is maximised.
    assert _run(xgb.callback.EarlyStopping(rounds=1), [1.0, 2.0], metric="mape")[1] == 1
    assert _run(xgb.callback.EarlyStopping(rounds=1), [1.0, 2.0], metric="map@3")[1] is None
    with pytest.raises(ValueError):
        xgb.callback.EarlyStopping(rounds=1, min_delta=-1)


def test_early_stopping_continued_training_and_cv_pairs():
    # best_iteration counts the rounds the model already had.
    model, _ = _run(xgb.callback.EarlyStopping(rounds=3), [3.0, 2.0], model=Model(rounds=10))
    assert model.attrs["best_iteration"] == "11"
    # cv history holds (mean, std) pairs: the mean decides.
    model, stopped = _run(xgb.callback.EarlyStopping(rounds=1), [(2.0, 9.0), (1.0, 0.0), (1.5, 0.0)])
    assert stopped == 2 and model.attrs["best_score"] == "1.0"


def test_early_stopping_watched_set_and_errors():
    es = xgb.callback.EarlyStopping(rounds=1, data_name="train", metric_name="mae")
    model = Model()
    es.before_training(model)
    log = {"train": {"mae": [1.0], "rmse": [9.0]}, "valid": {"rmse": [0.1]}}
    es.after_iteration(model, 0, log)
    assert model.attrs["best_score"] == "1.0"
    with pytest.raises(ValueError):
        xgb.callback.EarlyStopping(rounds=1).after_iteration(Model(), 0, {})
    with pytest.raises(ValueError):
        xgb.callback.EarlyStopping(rounds=1, data_name="nope").after_iteration(Model(), 0, log)
    with pytest.raises(ValueError):
        xgb.callback.EarlyStopping(rounds=1, save_best=True).before_training(Model())


def test_monitor_lines_and_period():
    lines = []
    mon = xgb.callback.EvaluationMonitor(period=2, logger=lines.append)
    log = {"train": {"rmse": []}, "valid": {"rmse": []}}
    for epoch in range(5):
        log["train"]["rmse"].append(1.0 / (epoch + 1))
        log["valid"]["rmse"].append(2.0 / (epoch + 1))
        mon.after_iteration(None, epoch, log)
    mon.after_training(None)
    assert lines == ["[0]\ttrain-rmse:1.00000\tvalid-rmse:2.00000\n",
                     "[2]\ttrain-rmse:0.33333\tvalid-rmse:0.66667\n",
                     "[4]\ttrain-rmse:0.20000\tvalid-rmse:0.40000\n"]
    lines.clear()
    mon = xgb.callback.EvaluationMonitor(period=3, show_stdv=True, logger=lines.append)
    cvlog = {"test": {"mae": []}}
    for epoch in range(5):
        cvlog["test"]["mae"].append((1.5, 0.25))
        mon.after_iteration(None, epoch, cvlog)
    mon.after_training(None)
    assert lines == ["[0]\ttest-mae:1.50000+0.25000\n", "[3]\ttest-mae:1.50000+0.25000\n",
                     "[4]\ttest-mae:1.50000+0.25000\n"]


def test_scheduler_and_checkpoint(tmp_path):
    model = Model(rounds=4)
    sched = xgb.callback.LearningRateScheduler(lambda r: 0.5 / (r + 1))
    table = xgb.callback.LearningRateScheduler([0.3, 0.2])
    ckpt = xgb.callback.TrainingCheckPoint(tmp_path, name="m", interval=3)
    ckpt.before_training(model)
    for epoch in range(2):
        sched.after_iteration(model, epoch, {})
        table.after_iteration(model, epoch, {})
    for epoch in range(8):
        ckpt.after_iteration(model, epoch, {})
    assert model.params == [("learning_rate", 0.5), ("learning_rate", 0.3), ("learning_rate", 0.25),
                            ("learning_rate", 0.2)]
    assert model.saved == ["m_7.ubj", "m_10.ubj"]
    with pytest.raises(TypeError):
        xgb.callback.LearningRateScheduler(0.1)


def test_container_history_and_short_circuit():
    calls = []

    class Stop(xgb.callback.TrainingCallback):
        def after_iteration(self, model, epoch, evals_log):
            calls.append("stop")
            return True

    class Later(xgb.callback.TrainingCallback):
        def after_iteration(self, model, epoch, evals_log):
            calls.append("later")
            return False

    stop = Stop()
    c = CallbackContainer([stop, Later(), stop])
    assert len(c.callbacks) == 2  # the same callback object once

    class Evaluating(Model):
        def eval_set(self, evals, epoch, metric, margin):
            return f"[{epoch}]\ttrain-rmse:0.5\tvalid-rmse:0.75\tvalid-mae:0.25"

    assert c.after_iteration(Evaluating(), 0, None, [(None, "train"), (None, "valid")])
    assert calls == ["stop"]
    assert c.history == {"train": {"rmse": [0.5]}, "valid": {"rmse": [0.75], "mae": [0.25]}}
    with pytest.raises(ValueError):
        c.after_iteration(Evaluating(), 1, None, [(None, "a-b")])
    with pytest.raises(TypeError):
        CallbackContainer([object()])


def test_fold_statistics():
    lines = ["[0]\ttrain-rmse:1\ttest-rmse:3", "[0]\ttrain-rmse:2\ttest-rmse:5"]
    assert _scores(lines[0]) == [("train-rmse", 1.0), ("test-rmse", 3.0)]
    assert _fold_statistics(lines) == [("train-rmse", 1.5, 0.5), ("test-rmse", 4.0, 1.0)]
