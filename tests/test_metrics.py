"""The oracle's evaluation metrics and CV folds, each pinned against an
independent computation (reference src/metrics.cpp:8-159,
kernels/boost.metal:2225-2295, kernels/radix_sort.metal.h:427-790,
src/c_api.cpp:1018-1110):

- elementwise metrics: float64 closed forms within fp32 tolerance, and exact
  integer sums where every fp32 partial sum is exact;
- ROC-AUC: exact pair counting (a positive ranked above a negative counts 1,
  a tie 1/2) with Fractions, and weighted pair sums;
- PR-AUC: numerical quadrature of precision along each step's straight line;
- CV folds: partition rules, and the shuffle against libstdc++'s std::shuffle
  (the fixture written by the real one, tests/test_shuffle.py).

The CPU oracle is test infrastructure; the library's folds are checked
against it here (no GPU needed), the device metrics in test_gpu_metrics.py.
"""
from fractions import Fraction

import numpy as np
import pytest
from scipy import integrate
from scipy.special import gammaln

import oracle_lib as O

KINDS = {"rmse": 0, "mae": 1, "rmsle": 2, "logloss": 3, "error": 6, "mape": 7, "mphe": 8, "poisson": 9,
         "gamma-deviance": 10, "tweedie": 11, "gamma-nloglik": 12}


def _inputs(rows, seed, positive=False, unit=False):
    rng = np.random.default_rng(seed)
    if unit:
        pred = rng.uniform(0.01, 0.99, rows).astype(np.float32)
        y = (rng.random(rows) < pred).astype(np.float32)
    elif positive:
        pred = rng.uniform(0.2, 5.0, rows).astype(np.float32)
        y = rng.uniform(0.2, 5.0, rows).astype(np.float32)
    else:
        pred = rng.normal(size=rows).astype(np.float32)
        y = rng.normal(size=rows).astype(np.float32)
    w = rng.uniform(0.5, 2.0, rows).astype(np.float32)
    return pred, y, w


def _loss64(kind, p, y, parameter):
    p, y = p.astype(np.float64), y.astype(np.float64)
    if kind == "rmse":
        return (p - y) ** 2
    if kind == "mae":
        return np.abs(p - y)
    if kind == "rmsle":
        return (np.log1p(p) - np.log1p(y)) ** 2
    if kind == "logloss":
        return -y * np.log(np.maximum(p, 1e-16)) - (1 - y) * np.log(np.maximum(1 - p, 1e-16))
    if kind == "error":
        return np.where(p > parameter, 1 - y, y)
    if kind == "mape":
        return np.abs((p - y) / y)
    if kind == "mphe":
        z = (p - y) / parameter
        return parameter ** 2 * (np.sqrt(1 + z * z) - 1)
    if kind == "poisson":
        return gammaln(y + 1) + p - y * np.log(np.maximum(p, 1e-16))
    if kind == "gamma-deviance":
        return 2 * (-np.log(y / p) + y / p - 1)
    if kind == "tweedie":
        return -y * p ** (1 - parameter) / (1 - parameter) + p ** (2 - parameter) / (2 - parameter)
    if kind == "gamma-nloglik":
        return y / p + np.log(p)
    raise KeyError(kind)


@pytest.mark.parametrize("kind", sorted(KINDS))
@pytest.mark.parametrize("rows", [1, 255, 256, 257, 70001])
def test_metric_sums_match_float64(kind, rows):
    positive = kind in ("rmsle", "mape", "poisson", "gamma-deviance", "tweedie", "gamma-nloglik")
    pred, y, w = _inputs(rows, rows, positive=positive, unit=kind in ("logloss", "error"))
    if kind == "poisson":
        y = np.round(y * 2).astype(np.float32)  # counts
    parameter = {"error": 0.5, "mphe": 1.5, "tweedie": 1.4}.get(kind, 0.0)
    for weights in (None, w):
        got = O.metric_sum(pred, y, KINDS[kind], weights, parameter)
        wt = np.ones(rows) if weights is None else weights.astype(np.float64)
        expect_num = float((wt * _loss64(kind, pred, y, parameter)).sum())
        np.testing.assert_allclose(got[1], wt.sum(), rtol=2e-6)
        np.testing.assert_allclose(got[0], expect_num, rtol=2e-5, atol=1e-6 * rows)


def test_metric_sum_exact_for_integer_losses():
    """Integer residuals keep every fp32 partial sum exact, so any order gives
    the exact total: a dropped or repeated row would show."""
    rng = np.random.default_rng(7)
    rows = 300_001  # > 256 * 256 rows: several blocks per reduce thread
    y = rng.integers(-3, 4, rows).astype(np.float32)
    pred = (y + rng.integers(-2, 3, rows)).astype(np.float32)
    got = O.metric_sum(pred, y, KINDS["rmse"])
    assert got[0] == float(((pred - y).astype(np.int64) ** 2).sum()) and got[1] == rows
    w = rng.integers(1, 4, rows).astype(np.float32)
    got = O.metric_sum(pred, y, KINDS["mae"], w)
    assert got[0] == float((np.abs(pred - y).astype(np.int64) * w.astype(np.int64)).sum())
    assert got[1] == float(w.astype(np.int64).sum())


def _pairs_auc(pred, y):
    pos = [p for p, l in zip(pred, y) if l == 1]
    neg = [p for p, l in zip(pred, y) if l == 0]
    wins = sum(Fraction(1) if a > b else Fraction(1, 2) if a == b else Fraction(0) for a in pos for b in neg)
    return wins, len(pos), len(neg)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_roc_auc_equals_pair_counting(seed):
    rng = np.random.default_rng(seed)
    rows = 400
    pred = np.round(rng.normal(size=rows), 1).astype(np.float32)  # many ties
    pred[:5] = 0.0
    pred[5:10] = -0.0  # +0 and -0 tie
    y = (rng.random(rows) < 0.4).astype(np.float32)
    area, pos, neg = O.metric_auc(pred, y)
    wins, npos, nneg = _pairs_auc(pred.tolist(), y.tolist())
    assert (pos, neg) == (npos, nneg)
    assert Fraction(area) == wins  # half-integers: exact in binary64


def test_weighted_roc_auc_equals_weighted_pairs():
    rng = np.random.default_rng(11)
    rows = 300
    pred = np.round(rng.normal(size=rows), 1).astype(np.float32)
    y = (rng.random(rows) < 0.5).astype(np.float32)
    w = rng.uniform(0.1, 3.0, rows).astype(np.float32)
    area, pos, neg = O.metric_auc(pred, y, weights=w)
    wp, wn = w[y == 1].astype(np.float64), w[y == 0].astype(np.float64)
    pp, pn = pred[y == 1][:, None], pred[y == 0][None, :]
    pairs = (wp[:, None] * wn[None, :] * np.where(pp > pn, 1.0, np.where(pp == pn, 0.5, 0.0))).sum()
    np.testing.assert_allclose(area, pairs, rtol=1e-12)
    np.testing.assert_allclose([pos, neg], [wp.sum(), wn.sum()], rtol=1e-12)


def _pr_quadrature(pred, y, w):
    order = np.argsort(-pred.astype(np.float64), kind="stable")
    keys = pred[order]
    tp = (y * w)[order].astype(np.float64)
    fp = ((1 - y) * w)[order].astype(np.float64)
    positives = tp.sum()
    area, TP, FP, i = 0.0, 0.0, 0.0, 0
    while i < len(keys):
        j = i
        while j < len(keys) and keys[j] == keys[i]:
            j += 1
        a, b = tp[i:j].sum(), fp[i:j].sum()
        if a > 0:
            def precision(t, TP=TP, FP=FP, a=a, b=b):
                return (TP + t * a) / (TP + FP + t * (a + b))
            area += a / positives * integrate.quad(precision, 0, 1, epsabs=1e-14, epsrel=1e-13)[0]
        TP, FP, i = TP + a, FP + b, j
    return area


@pytest.mark.parametrize("weighted", [False, True])
def test_pr_auc_equals_quadrature(weighted):
    rng = np.random.default_rng(5)
    rows = 200
    pred = np.round(rng.uniform(size=rows), 2).astype(np.float32)
    y = (rng.random(rows) < pred).astype(np.float32)
    w = rng.uniform(0.2, 2.0, rows).astype(np.float32) if weighted else np.ones(rows, np.float32)
    area, _, _ = O.metric_auc(pred, y, pr=True, weights=w if weighted else None)
    np.testing.assert_allclose(area, _pr_quadrature(pred, y, w), rtol=1e-10)


def test_auc_closed_forms():
    y = np.array([1, 1, 0, 0, 0], np.float32)
    perfect = np.array([0.9, 0.8, 0.3, 0.2, 0.1], np.float32)
    assert O.metric_auc(perfect, y)[0] == 6.0  # every one of 2 x 3 pairs
    assert O.metric_auc(perfect, y, pr=True)[0] == 1.0
    tied = np.full(5, 0.5, np.float32)
    assert O.metric_auc(tied, y)[0] == 3.0
    np.testing.assert_allclose(O.metric_auc(tied, y, pr=True)[0], 2 / 5, rtol=1e-15)


def test_cv_folds_partition_rules():
    rows, nfold = 103, 4
    plain = O.cv_folds(rows, nfold, 0, shuffle=False)
    sizes = [26, 26, 26, 25]  # the first rows % nfold folds one longer
    np.testing.assert_array_equal(plain, np.repeat(np.arange(nfold), sizes))
    shuffled = O.cv_folds(rows, nfold, 42)
    assert sorted(np.bincount(shuffled).tolist()) == sorted(sizes)
    y = (np.arange(rows) % 3 == 0).astype(np.float32)
    strat = O.cv_folds(rows, nfold, 42, stratified=True, labels=y)
    for k in range(nfold):
        ones = int(y[strat == k].sum())
        assert abs(ones - y.sum() / nfold) <= 1
    assert not np.array_equal(O.cv_folds(rows, nfold, 43), shuffled)


def test_cv_shuffle_follows_libstdcxx_draws():
    """Plain folds take consecutive chunks of the row order std::shuffle
    draws over mt19937(seed) (libstdc++, as an x86-64 build of
    src/c_api.cpp:1018-1110), the first rows % nfold folds one row longer;
    the order is taken from the fixture the real std::shuffle wrote."""
    import json
    from pathlib import Path
    fixture = json.loads((Path(__file__).parent / "golden" / "shuffle_libstdcxx.json").read_text())
    rows, nfold, seed = 101, 3, 42
    order = next(c["head"] for c in fixture["cases"] if c["n"] == rows and c["seed"] == seed)
    expect = np.zeros(rows, np.int32)
    pos = 0
    for k in range(nfold):
        chunk = rows // nfold + (1 if k < rows % nfold else 0)
        for _ in range(chunk):
            expect[order[pos]] = k
            pos += 1
    np.testing.assert_array_equal(O.cv_folds(rows, nfold, seed), expect)


@pytest.mark.parametrize("model", ["libstdc++", "libc++"])
@pytest.mark.parametrize("stratified", [False, True])
def test_library_cv_folds_match_oracle(xgb, stratified, model):
    """XGDMatrixBuildCVFolds: each fold's test rows are the oracle's, with the
    shuffle draws of the standard library the global config's std_shuffle
    names (the default libstdc++; libc++ as the reference's macOS builds)."""
    import ctypes
    rows, nfold, seed = 61, 5, 9
    X = np.arange(rows * 2, dtype=np.float32).reshape(rows, 2)
    y = (np.arange(rows) % 4 == 1).astype(np.float32)
    d = xgb.DMatrix(X, label=y)
    c_train = (ctypes.c_void_p * nfold)()
    c_test = (ctypes.c_void_p * nfold)()
    assert xgb.get_config()["std_shuffle"] == "libstdc++"
    with xgb.config_context(std_shuffle=model):
        assert xgb.get_config()["std_shuffle"] == model
        assert xgb.core._LIB.XGDMatrixBuildCVFolds(d.handle, nfold, ctypes.c_uint(seed), 1, int(stratified), c_train,
                                                   c_test) == 0
    assert xgb.get_config()["std_shuffle"] == "libstdc++"
    expect = O.cv_folds(rows, nfold, seed, stratified=stratified, labels=y, std_shuffle=model)
    if model != "libstdc++" and not stratified:
        assert not np.array_equal(expect, O.cv_folds(rows, nfold, seed))  # the two models draw differently
    for k in range(nfold):
        test = xgb.DMatrix(ctypes.c_void_p(c_test[k]))
        train = xgb.DMatrix(ctypes.c_void_p(c_train[k]))
        got_test = test.get_data().toarray()[:, 0] / 2
        got_train = train.get_data().toarray()[:, 0] / 2
        np.testing.assert_array_equal(got_test, np.flatnonzero(expect == k))
        np.testing.assert_array_equal(got_train, np.flatnonzero(expect != k))
        np.testing.assert_array_equal(test.get_label(), y[expect == k])
