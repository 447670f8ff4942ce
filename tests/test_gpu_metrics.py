"""Device metrics against the CPU oracle, and evaluation through training.

Bitwise for the metrics whose per-row loss is exactly rounded fp32
arithmetic (rmse, mae, error, mape, mphe: subtraction, product, IEEE
division and square root) and for unweighted AUC (integer sums); relative
tolerance 1e-6 for the losses built on log / pow / lgamma (device and libm
implementations differ in the last bits) and 1e-12 for weighted AUC and
PR-AUC (binary64 sums in a different order).
"""
import numpy as np
import pytest

import device_lib as D
import oracle_lib as O
import workloads as W

pytestmark = pytest.mark.gpu

KINDS = {"rmse": 0, "mae": 1, "rmsle": 2, "logloss": 3, "error": 6, "mape": 7, "mphe": 8, "poisson": 9,
         "gamma-deviance": 10, "tweedie": 11, "gamma-nloglik": 12}
EXACT = {"rmse", "mae", "error", "mape", "mphe"}


@pytest.mark.parametrize("kind", sorted(KINDS))
@pytest.mark.parametrize("rows", [1, 257, 70001, 1_000_003])
def test_metric_sum_matches_oracle(kind, rows):
    rng = np.random.default_rng(rows)
    if kind in ("logloss", "error"):
        pred = rng.uniform(0.01, 0.99, rows).astype(np.float32)
        y = (rng.random(rows) < pred).astype(np.float32)
    elif kind in ("rmse", "mae", "mphe"):
        pred, y = rng.normal(size=(2, rows)).astype(np.float32)
    else:
        pred, y = rng.uniform(0.2, 5.0, size=(2, rows)).astype(np.float32)
        if kind == "poisson":
            y = np.round(y * 2).astype(np.float32)
    w = rng.uniform(0.5, 2.0, rows).astype(np.float32)
    parameter = {"error": 0.5, "mphe": 1.5, "tweedie": 1.4}.get(kind, 0.0)
    for weights in (None, w):
        got = D.metric_sum(pred, y, KINDS[kind], weights, parameter)
        expect = O.metric_sum(pred, y, KINDS[kind], weights, parameter)
        if kind in EXACT:
            np.testing.assert_array_equal(got.view(np.uint32), expect.view(np.uint32),
                                          err_msg=f"{kind} rows={rows} weighted={weights is not None}")
        else:
            np.testing.assert_allclose(got, expect, rtol=1e-6)


@pytest.mark.parametrize("rows", [1, 2, 999, 300_000])
def test_auc_matches_oracle(rows):
    rng = np.random.default_rng(rows + 1)
    pred = np.round(rng.normal(size=rows), 2).astype(np.float32)  # ties
    y = (rng.random(rows) < 0.3).astype(np.float32)
    if rows >= 2:
        y[0], y[1] = 1, 0  # both classes present
    w = rng.uniform(0.2, 2.0, rows).astype(np.float32)
    got, expect = D.metric_auc(pred, y), O.metric_auc(pred, y)
    np.testing.assert_array_equal(got, expect)
    np.testing.assert_allclose(D.metric_auc(pred, y, weights=w), O.metric_auc(pred, y, weights=w), rtol=1e-12)
    for weights in (None, w):
        np.testing.assert_allclose(D.metric_auc(pred, y, pr=True, weights=weights),
                                   O.metric_auc(pred, y, pr=True, weights=weights), rtol=1e-12)


def _expected_line(iteration, evals, metrics):
    """The evaluation line from oracle metric values, printed as the
    reference prints a binary64 with 10 significant digits."""
    parts = [f"[{iteration}]"]
    for name, pred, y in evals:
        for m in metrics:
            if m in ("auc", "aucpr"):
                area, pos, neg = O.metric_auc(pred, y, pr=m == "aucpr")
                value = area / (pos * neg) if m == "auc" else area
            else:
                s = O.metric_sum(pred, y, KINDS[m], None, 0.5)
                value = float(s[0]) / float(s[1])
                if m == "rmse":
                    value = np.sqrt(value)
            parts.append(f"{name}-{m}:{value:.10g}")
    return "\t".join(parts)


def test_eval_lines_match_oracle_metrics(xgb):
    X, y = W.config1(rows=5000, cols=8)
    Xv, yv = W.config1(rows=1500, cols=8, seed=99)
    dtrain, dvalid = xgb.DMatrix(X, label=y), xgb.DMatrix(Xv, label=yv)
    bst = xgb.Booster({"max_depth": 4, "eval_metric": ["rmse", "mae"]}, [dtrain, dvalid])
    for i in range(3):
        bst.update(dtrain, i)
        line = bst.eval_set([(dtrain, "train"), (dvalid, "valid")], i)
        preds = [("train", bst.predict(dtrain), y), ("valid", bst.predict(dvalid), yv)]
        assert line == _expected_line(i, preds, ["rmse", "mae"])


def test_logistic_default_metric_and_auc(xgb):
    rng = np.random.default_rng(3)
    X = rng.normal(size=(4000, 6)).astype(np.float32)
    y = (X[:, 0] + 0.5 * rng.normal(size=4000) > 0).astype(np.float32)
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train({"objective": "binary:logistic", "max_depth": 3}, d, 2)
    p = bst.predict(d)
    assert bst.eval(d, "t", 1) == _expected_line(1, [("t", p, y)], ["logloss"])
    bst.set_param({"eval_metric": ["auc", "aucpr", "error"]})
    line = bst.eval(d, "t", 1)
    assert line == _expected_line(1, [("t", p, y)], ["logloss", "auc", "aucpr", "error"])


def test_early_stopping_and_history(xgb):
    X, y = W.config1(rows=3000, cols=8)
    Xv, yv = W.config1(rows=800, cols=8, seed=5)
    dtrain, dvalid = xgb.DMatrix(X, label=y), xgb.DMatrix(Xv, label=yv)
    history = {}
    bst = xgb.train({"max_depth": 6, "eta": 0.9, "eval_metric": "rmse"}, dtrain, 200,
                    evals=[(dtrain, "train"), (dvalid, "valid")], early_stopping_rounds=3, evals_result=history,
                    verbose_eval=False)
    valid = history["valid"]["rmse"]
    best = int(np.argmin(valid))
    assert bst.best_iteration == best and bst.best_score == pytest.approx(valid[best], rel=1e-9)
    assert len(valid) == best + 4 and bst.num_boosted_rounds() == best + 4
    assert len(history["train"]["rmse"]) == len(valid)
    # save_best keeps the rounds up to the best one.
    es = xgb.callback.EarlyStopping(rounds=3, save_best=True)
    cut = xgb.train({"max_depth": 6, "eta": 0.9}, dtrain, 200, evals=[(dvalid, "valid")], callbacks=[es],
                    verbose_eval=False)
    assert cut.num_boosted_rounds() == best + 1
    np.testing.assert_array_equal(cut.predict(dvalid), bst.predict(dvalid, iteration_range=(0, best + 1)))


def test_learning_rate_scheduler_and_custom_callback(xgb):
    X, y = W.config1(rows=2000, cols=6)
    d = xgb.DMatrix(X, label=y)
    seen = []

    class Record(xgb.callback.TrainingCallback):
        def after_iteration(self, model, epoch, evals_log):
            seen.append((epoch, model.num_boosted_rounds()))
            return epoch == 4  # stop after round 4

    rates = [0.3, 0.2, 0.1, 0.05, 0.02, 0.01]
    sched = xgb.train({"max_depth": 3}, d, 6, callbacks=[xgb.callback.LearningRateScheduler(rates), Record()])
    assert seen == [(i, i + 1) for i in range(5)] and sched.num_boosted_rounds() == 5
    # Round r is trained at the rate set after round r - 1 (the first at the default).
    manual = xgb.Booster({"max_depth": 3}, [d])
    for r in range(5):
        if r:
            manual.set_param("learning_rate", rates[r - 1])
        manual.update(d, r)
    np.testing.assert_array_equal(sched.predict(d), manual.predict(d))


def test_cv_folds_and_results(xgb):
    X, y = W.config1(rows=3000, cols=6)
    d = xgb.DMatrix(X, label=y)
    params = {"max_depth": 3, "eval_metric": "mae"}
    res = xgb.cv(params, d, num_boost_round=4, nfold=3, seed=7, as_pandas=False)
    assert list(res) == ["train-mae-mean", "train-mae-std", "test-mae-mean", "test-mae-std"]
    # Fold by fold through the public pieces: the folds' test MAE after round 4.
    folds = O.cv_folds(3000, 3, 7)
    maes = []
    for k in range(3):
        tr, te = np.flatnonzero(folds != k), np.flatnonzero(folds == k)
        b = xgb.train(params, xgb.DMatrix(X[tr], label=y[tr]), 4)
        s = O.metric_sum(b.predict(xgb.DMatrix(X[te])), y[te], KINDS["mae"])
        maes.append(float(f"{float(s[0]) / float(s[1]):.10g}"))
    assert res["test-mae-mean"][-1] == pytest.approx(np.mean(maes), rel=1e-12)
    assert res["test-mae-std"][-1] == pytest.approx(np.std(maes), rel=1e-9, abs=1e-12)
    early = xgb.cv({"max_depth": 6, "eta": 1.0}, d, 100, nfold=3, early_stopping_rounds=2, as_pandas=False)
    assert len(early["test-rmse-mean"]) < 100
