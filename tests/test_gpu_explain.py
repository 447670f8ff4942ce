"""Leaf indices, feature contributions and their interactions on the GPU
(reference src/learner.cpp:455-560, prediction types 2 to 6), checked against
references computed here from the saved model JSON:

- leaf ids: a plain walk of every tree (value < threshold goes left, NaN
  follows default_left);
- approximate contributions: each split's feature credited with the change
  of the cover-weighted node mean along the row's path, in binary64;
- exact contributions: Shapley values by their definition, over every subset
  of the features, with the path-dependent value function TreeSHAP computes
  (a tree's expectation where the subset fixes a feature the walk follows the
  row, elsewhere the children are weighted by their cover), in binary64;
- exact interactions: the Shapley interaction index by its definition, and on
  the diagonal each feature's value less its interactions; approximate ones
  carry the approximate contributions on the diagonal.

The kernels compute in binary32, so contributions compare within 2e-5 of the
margin's scale; leaf ids are exact.  Local accuracy (contributions plus bias
equal the margin prediction) is checked on every case."""
import json
import math
from itertools import combinations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class _Tree:
    def __init__(self, t):
        self.left = np.array(t["left_children"], dtype=np.int64)
        self.right = np.array(t["right_children"], dtype=np.int64)
        self.feature = np.array(t["split_indices"], dtype=np.int64)
        self.cond = np.array(t["split_conditions"], dtype=np.float32)
        self.dleft = np.array(t["default_left"], dtype=bool)
        self.cover = np.array(t["sum_hessian"], dtype=np.float64)
        self.mean = np.zeros(len(self.left))
        for k in range(len(self.left) - 1, -1, -1):
            l, r = self.left[k], self.right[k]
            self.mean[k] = (float(self.cond[k]) if l < 0 else
                            (self.mean[l] * self.cover[l] + self.mean[r] * self.cover[r]) / self.cover[k])

    def child(self, k, x):
        v = x[self.feature[k]]
        go_left = self.dleft[k] if np.isnan(v) else v < self.cond[k]
        return self.left[k] if go_left else self.right[k]

    def leaf(self, x):
        k = 0
        while self.left[k] >= 0:
            k = self.child(k, x)
        return k

    def expect(self, x, subset, k=0):
        """E[tree | the features in `subset` fixed at x], path-dependent."""
        if self.left[k] < 0:
            return float(self.cond[k])
        if self.feature[k] in subset:
            return self.expect(x, subset, self.child(k, x))
        l, r = self.left[k], self.right[k]
        return (self.cover[l] * self.expect(x, subset, l) + self.cover[r] * self.expect(x, subset, r)) / self.cover[k]


def _trees(bst):
    model = json.loads(bytes(bst.save_raw("json")))
    return [_Tree(t) for t in model["learner"]["gradient_booster"]["model"]["trees"]]


def _shapley(trees, x, cols):
    phi = np.zeros(cols)
    for f in range(cols):
        others = [g for g in range(cols) if g != f]
        for size in range(cols):
            w = math.factorial(size) * math.factorial(cols - size - 1) / math.factorial(cols)
            for s in combinations(others, size):
                s = set(s)
                phi[f] += w * sum(t.expect(x, s | {f}) - t.expect(x, s) for t in trees)
    return phi


def _interactions(trees, x, cols):
    """SHAP interaction values by their definition: off the diagonal the
    Shapley interaction index over every subset of the other features, on it
    the feature's Shapley value less its interactions."""
    def f(s):
        return sum(t.expect(x, s) for t in trees)
    phi = _shapley(trees, x, cols)
    m = np.zeros((cols + 1, cols + 1))
    for i in range(cols):
        for j in range(cols):
            if i == j:
                continue
            others = [g for g in range(cols) if g not in (i, j)]
            for size in range(cols - 1):
                w = math.factorial(size) * math.factorial(cols - size - 2) / (2 * math.factorial(cols - 1))
                for s in combinations(others, size):
                    s = set(s)
                    m[i, j] += w * (f(s | {i, j}) - f(s | {i}) - f(s | {j}) + f(s))
        m[i, i] = phi[i] - sum(m[i, j] for j in range(cols) if j != i)
    return m


def _saabas(trees, x, cols):
    phi = np.zeros(cols + 1)
    for t in trees:
        k = 0
        phi[cols] += t.mean[0]
        while t.left[k] >= 0:
            nxt = t.child(k, x)
            phi[t.feature[k]] += t.mean[nxt] - t.mean[k]
            k = nxt
    return phi


def _data(rows=60, cols=5, seed=7, missing=0.15):
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(rows, cols)).astype(np.float32)
    y = (X[:, 0] * 1.5 - X[:, 1] + 0.5 * X[:, 2] * X[:, 3] + 0.1 * rng.normal(size=rows)).astype(np.float32)
    X[rng.random(X.shape) < missing] = np.nan
    return X, y


@pytest.mark.parametrize("objective", ["reg:squarederror", "binary:logistic"])
def test_leaf_and_contributions_match_definitions(xgb, objective):
    X, y = _data()
    if objective == "binary:logistic":
        y = (y > 0).astype(np.float32)
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train({"objective": objective, "max_depth": 3, "max_bin": 32, "eta": 0.5}, d, 4)
    trees = _trees(bst)
    margin = bst.predict(d, output_margin=True).astype(np.float64)
    scale = max(1.0, float(np.abs(margin).max()))

    leaf = bst.predict(d, pred_leaf=True)
    assert leaf.shape == (len(X), 4) and leaf.dtype == np.float32
    expect = np.array([[t.leaf(x) for t in trees] for x in X], dtype=np.float32)
    np.testing.assert_array_equal(leaf, expect)

    approx = bst.predict(d, pred_contribs=True, approx_contribs=True).astype(np.float64)
    assert approx.shape == (len(X), X.shape[1] + 1)
    base = margin - np.array([sum(float(t.cond[t.leaf(x)]) for t in trees) for x in X])
    for i, x in enumerate(X):
        ref = _saabas(trees, x, X.shape[1])
        ref[-1] += base[i]
        np.testing.assert_allclose(approx[i], ref, rtol=0, atol=2e-5 * scale)
    np.testing.assert_allclose(approx.sum(axis=1), margin, rtol=0, atol=2e-5 * scale)

    exact = bst.predict(d, pred_contribs=True).astype(np.float64)
    assert exact.shape == (len(X), X.shape[1] + 1)
    for i, x in enumerate(X[:20]):
        phi = _shapley(trees, x, X.shape[1])
        np.testing.assert_allclose(exact[i, :-1], phi, rtol=0, atol=2e-5 * scale)
        np.testing.assert_allclose(exact[i, -1], base[i] + sum(t.mean[0] for t in trees), rtol=0, atol=2e-5 * scale)
    np.testing.assert_allclose(exact.sum(axis=1), margin, rtol=0, atol=2e-5 * scale)


def test_contributions_csr_equal_dense_and_follow_base_margin(xgb):
    import scipy.sparse as sp
    X, y = _data(rows=80, cols=6, seed=11, missing=0.3)
    bst = xgb.train({"max_depth": 4, "max_bin": 64, "eta": 0.3}, xgb.DMatrix(X, label=y), 5)
    rows, cols = np.nonzero(~np.isnan(X))
    csr = sp.csr_matrix((X[rows, cols], (rows, cols)), shape=X.shape)
    dense, sparse = xgb.DMatrix(X), xgb.DMatrix(csr)
    for kw in ({"pred_leaf": True}, {"pred_contribs": True}, {"pred_contribs": True, "approx_contribs": True}):
        np.testing.assert_array_equal(bst.predict(dense, **kw), bst.predict(sparse, **kw))
    offset = np.linspace(-1.0, 1.0, len(X)).astype(np.float32)
    shifted = xgb.DMatrix(X, base_margin=offset)
    plain = bst.predict(dense, pred_contribs=True)
    moved = bst.predict(shifted, pred_contribs=True)
    np.testing.assert_array_equal(moved[:, :-1], plain[:, :-1])
    base = float(plain[0, -1]) - sum(t.mean[0] for t in _trees(bst))
    np.testing.assert_allclose(moved[:, -1] - plain[:, -1], offset - base, rtol=0, atol=1e-5)
    np.testing.assert_allclose(moved.sum(axis=1), bst.predict(shifted, output_margin=True), rtol=0, atol=1e-4)


def test_deep_trees_are_locally_accurate_and_shaped(xgb):
    X, y = _data(rows=300, cols=6, seed=3, missing=0.05)
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train({"max_depth": 9, "max_bin": 128, "eta": 0.3}, d, 6)
    margin = bst.predict(d, output_margin=True)
    exact = bst.predict(d, pred_contribs=True)
    np.testing.assert_allclose(exact.sum(axis=1), margin, rtol=0, atol=1e-4 * max(1.0, np.abs(margin).max()))
    trees = _trees(bst)
    for x, row in zip(X[:2], exact[:2]):
        np.testing.assert_allclose(row[:-1], _shapley(trees, x, X.shape[1]), rtol=0, atol=1e-4)
    # Rounds [0, 3) only.
    part = bst.predict(d, pred_contribs=True, iteration_range=(0, 3))
    np.testing.assert_allclose(part.sum(axis=1), bst.predict(d, output_margin=True, iteration_range=(0, 3)),
                               rtol=0, atol=1e-4)
    assert bst.predict(d, pred_leaf=True, strict_shape=True).shape == (len(X), 6, 1, 1)
    assert bst.predict(d, pred_contribs=True, strict_shape=True).shape == (len(X), 1, X.shape[1] + 1)
    assert bst.predict(d, pred_leaf=True, iteration_range=(0, 2)).shape == (len(X), 2)


def test_interactions_match_definitions(xgb):
    X, y = _data(rows=40, cols=5, seed=5)
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train({"max_depth": 3, "max_bin": 32, "eta": 0.5}, d, 3)
    trees = _trees(bst)
    margin = bst.predict(d, output_margin=True).astype(np.float64)
    scale = max(1.0, float(np.abs(margin).max()))
    exact = bst.predict(d, pred_interactions=True).astype(np.float64)
    assert exact.shape == (len(X), 6, 6)
    contribs = bst.predict(d, pred_contribs=True).astype(np.float64)
    for i, x in enumerate(X[:12]):
        ref = _interactions(trees, x, 5)
        np.testing.assert_allclose(exact[i, :5, :5], ref[:5, :5], rtol=0, atol=2e-5 * scale)
    np.testing.assert_allclose(exact[:, :5, :5].sum(axis=2), contribs[:, :5], rtol=0, atol=2e-5 * scale)
    np.testing.assert_allclose(exact[:, 5, 5], contribs[:, 5], rtol=0, atol=1e-6 * scale)
    np.testing.assert_array_equal(exact[:, 5, :5], 0.0)
    np.testing.assert_array_equal(exact[:, :5, 5], 0.0)
    np.testing.assert_allclose(exact.sum(axis=(1, 2)), margin, rtol=0, atol=2e-5 * scale)
    approx = bst.predict(d, pred_interactions=True, approx_contribs=True)
    saabas = bst.predict(d, pred_contribs=True, approx_contribs=True)
    assert approx.shape == (len(X), 6, 6)
    np.testing.assert_array_equal(np.diagonal(approx, axis1=1, axis2=2), saabas)
    off = approx.copy()
    off[:, np.arange(6), np.arange(6)] = 0.0
    np.testing.assert_array_equal(off, 0.0)
    assert bst.predict(d, pred_interactions=True, strict_shape=True).shape == (len(X), 1, 6, 6)


def test_nonzero_start_and_two_types_are_refused(xgb):
    X, y = _data(rows=40, cols=4)
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train({"max_depth": 2}, d, 3)
    assert bst.predict(d, pred_leaf=True, iteration_range=(0, 1)).shape == (len(X),)
    with pytest.raises(xgb.XGBoostError, match="only iteration end"):
        bst.predict(d, pred_contribs=True, iteration_range=(1, 3))
    with pytest.raises(ValueError, match="One type of prediction"):
        bst.predict(d, pred_leaf=True, pred_contribs=True)


def test_interpret_shap_values_split_the_bias(xgb):
    X, y = _data(rows=50, cols=4, seed=9)
    model = xgb.XGBRegressor(n_estimators=4, max_depth=3, max_bin=32)
    model.fit(X, y)
    values, bias = xgb.interpret.shap_values(model, X)
    contribs = model.get_booster().predict(xgb.DMatrix(X), pred_contribs=True)
    np.testing.assert_array_equal(values, contribs[:, :-1])
    np.testing.assert_array_equal(bias, contribs[:, -1])
    with pytest.raises(NotImplementedError):
        xgb.interpret.shap_values(model, X, X_background=X)
    with pytest.raises(ValueError):
        xgb.interpret.shap_values(model.get_booster(), xgb.DMatrix(X), missing=0.0)


def test_empty_matrix_and_untrained_model(xgb):
    X, y = _data(rows=30, cols=4)
    d = xgb.DMatrix(X, label=y)
    fresh = xgb.Booster({"max_depth": 2}, [d])
    contribs = fresh.predict(d, pred_contribs=True)
    assert contribs.shape == (30, 5)
    np.testing.assert_array_equal(contribs[:, :4], 0.0)
    np.testing.assert_allclose(contribs[:, 4], fresh.predict(d, output_margin=True), rtol=0, atol=1e-6)
    assert fresh.predict(d, pred_leaf=True).shape == (30, 0)
    bst = xgb.train({"max_depth": 2}, d, 2)
    empty = xgb.DMatrix(np.zeros((0, 4), dtype=np.float32))
    assert bst.predict(empty, pred_contribs=True).shape == (0, 5)
    assert bst.predict(empty, pred_interactions=True).shape == (0, 5, 5)
    assert bst.predict(empty, pred_leaf=True).size == 0


def test_estimator_apply_returns_leaf_ids(xgb):
    X, y = _data(rows=50, cols=4, seed=13)
    model = xgb.XGBRegressor(n_estimators=3, max_depth=3, max_bin=32)
    model.fit(X, y)
    leaves = model.apply(X)
    assert leaves.shape == (50, 3)
    np.testing.assert_array_equal(leaves, model.get_booster().predict(xgb.DMatrix(X), pred_leaf=True))
    trees = _trees(model.get_booster())
    np.testing.assert_array_equal(leaves, np.array([[t.leaf(x) for t in trees] for x in X], dtype=np.float32))


def test_classifier_apply(xgb):
    X, y = _data(rows=40, cols=4, seed=17)
    model = xgb.XGBClassifier(n_estimators=2, max_depth=2, max_bin=16)
    model.fit(X, (y > 0).astype(np.int64))
    np.testing.assert_array_equal(model.apply(X), model.get_booster().predict(xgb.DMatrix(X), pred_leaf=True))
