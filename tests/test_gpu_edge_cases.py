"""The reference's own edge-case constructions through the HIP path, against
the CPU oracle bit for bit: cuts, every tree field, training margins and a
fresh matrix's prediction.

- the engine test inputs of tests/test_gpu_tree.py:36-85 (regression, missing
  values with an all-missing column, cross-feature ties, a constant label,
  zero sample weights, signed zeros and subnormal features, +/-inf as the
  missing value) at depths 2, 6 and 10;
- adversarial gradients (tests/test_gradient_precision.py:14-36): a float32
  residual after cancelling 2^16 terms, and 257 float32-max gradients;
- root-sum constructions (tests/test_parent_statistics.py:24-47,
  tests/test_scalar_root_statistics.py:10-45): [2^40, -2^40, 3 * 2^-14]
  with Hessians [1, 2, 1], one or two features, missing values in either,
  from DMatrix and QuantileDMatrix (own cuts or a reference matrix's);
- partition edges (tests/test_partition_single_pass.py:65-130): row counts
  at tile boundaries 1 ... 4,099, one-sided tiles with empty children, and a
  full depth-10 frontier (left children 2 * arange(511) + 1), each with the
  stable and the atomic-claim partition;
- full trees beyond the reference's depths: depth 12, 14 and 16 (the
  deepest this engine takes), dense with either partition and CSR;
- the x86 form of the gain (no fused multiply-add) on both sides;
- device gradients and fixed-point scales against the oracle's directly;
- BASELINE config 4's own generator (128 columns, Bernoulli labels) with its
  own parameters.

The max_leaves = 1 variants of the reference's tests are absent: this engine
grows depthwise only and rejects max_leaves."""
import ctypes
import json

import numpy as np
import pytest

import device_lib as D
import oracle_lib as O
import workloads as W
from test_gpu_parity import _oracle_params, assert_trees_equal
from test_zz_no_alloc import MASS_WORDS, MgbGradParams

pytestmark = pytest.mark.gpu

TINY = np.nextafter(np.float32(0), np.float32(1))


def engine_inputs(case, rows=513):
    """The reference's engine test inputs (tests/test_gpu_tree.py:36-85):
    returns X, y, DMatrix keyword arguments and extra parameters."""
    rng = np.random.default_rng(82171)
    X = rng.normal(size=(rows, 7)).astype(np.float32)
    y = (X[:, 0] - X[:, 1] * X[:, 2] + X[:, 3] ** 2).astype(np.float32)
    meta = {}
    if case == "missing":
        X[::7, 0] = np.nan
        X[::11, 3] = np.nan
        X[:, 6] = np.nan
    elif case == "ties":
        X[:, 0] = np.arange(rows) % 4
        X[:, 1:] = X[:, :1]
        y = (X[:, 0] >= 2).astype(np.float32)
    elif case == "constant":
        y.fill(0)
    elif case == "weighted":
        meta["weight"] = rng.uniform(0.01, 3, rows).astype(np.float32)
        meta["weight"][::13] = 0
    elif case == "subnormal_features":
        X[:, 0] = np.resize(np.asarray([-4 * TINY, -TINY, -0.0, 0.0, TINY, 4 * TINY], np.float32), rows)
        y = (np.arange(rows) % 6 >= 3).astype(np.float32)
    elif case in ("positive_infinity_missing", "negative_infinity_missing"):
        inf = np.inf if case == "positive_infinity_missing" else -np.inf
        X[::9, 2] = inf
        meta["missing"] = inf
    return X, y, meta


def _oracle_view(X, meta):
    """The matrix the oracle sees: entries equal to `missing` become NaN."""
    if "missing" in meta:
        X = np.where(X == meta["missing"], np.float32(np.nan), X).astype(np.float32)
    return X


def assert_cuts_equal(d, ref):
    cut_ptr, cut_values = d.get_quantile_cut()
    np.testing.assert_array_equal(np.diff(cut_ptr), ref["cut_counts"])
    for f in range(len(ref["cut_counts"])):
        c = ref["cut_counts"][f]
        np.testing.assert_array_equal(cut_values[cut_ptr[f]:cut_ptr[f + 1]].view(np.uint32),
                                      ref["cuts"][f, :c].view(np.uint32), err_msg=f"feature {f} cuts")


def _fit_and_compare(xgb, X, y, meta, params, rounds, quantile=False, obj=None, grad=None, hess=None):
    weight = meta.get("weight")
    missing = meta.get("missing")
    extra = {"max_bin": params["max_bin"]} if quantile else {}
    constructor = xgb.QuantileDMatrix if quantile else xgb.DMatrix
    d = constructor(X, label=y, weight=weight, missing=missing, **extra)
    bst = xgb.train(params, d, rounds, obj=obj)
    ref = O.train(_oracle_view(X, meta), y, _oracle_params(params), rounds, weights=weight,
                  custom_grad=grad, custom_hess=hess)
    assert_cuts_equal(d, ref)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d, output_margin=True).view(np.uint32),
                                  ref["margin"].view(np.uint32))
    fresh = xgb.DMatrix(X, missing=missing)
    np.testing.assert_array_equal(bst.predict(fresh, output_margin=True).view(np.uint32),
                                  ref["margin"].view(np.uint32))
    return bst, ref


# ---------------------------------------------------------------------------
# Engine inputs at several depths (tests/test_partition_single_pass.py:55-61)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["regression", "missing", "ties", "constant", "weighted", "subnormal_features",
                                  "positive_infinity_missing", "negative_infinity_missing"])
@pytest.mark.parametrize("depth", [2, 6, 10])
def test_engine_inputs_match_oracle(xgb, case, depth):
    X, y, meta = engine_inputs(case)
    params = {"tree_method": "hist", "max_depth": depth, "max_bin": 32, "base_score": 0, "seed": 41}
    bst, ref = _fit_and_compare(xgb, X, y, meta, params, 3)
    if case == "subnormal_features":
        # Six values, five distinct ones (-0 == +0): four cuts and the tail
        # sentinel (the training matrix's cuts equal these, checked above).
        # Rows cycle -4t, -t, -0, +0, t, 4t, so every run of zeros starts at
        # -0: the zero cut is -0.0, and the root splits there.
        assert ref["cut_counts"][0] == 5
        np.testing.assert_array_equal(ref["cuts"][0, :4].view(np.uint32),
                                      np.asarray([-TINY, -0.0, TINY, 4 * TINY], np.float32).view(np.uint32))
        root = bst.trees_to_json()[0]
        assert root["split_indices"][0] == 0
        assert np.float32(root["split_conditions"][0]).view(np.uint32) == 0x80000000


@pytest.mark.parametrize("case", ["missing", "subnormal_features", "weighted"])
def test_engine_inputs_quantile_matrix(xgb, case):
    """The same inputs through QuantileDMatrix (cuts from the iterator path)."""
    X, y, meta = engine_inputs(case)
    params = {"tree_method": "hist", "max_depth": 6, "max_bin": 32, "base_score": 0, "seed": 41}
    _fit_and_compare(xgb, X, y, meta, params, 3, quantile=True)


# ---------------------------------------------------------------------------
# Adversarial gradients (tests/test_gradient_precision.py:14-36, one target)
# ---------------------------------------------------------------------------
GRADIENT_CASES = {
    # A float32 residual between two adjacent fixed-point units of a coarser
    # scale, after the cancelling terms.
    "cancelled-residual": np.asarray([2 ** 16, -2 ** 16, 6.118193027759844e-7], np.float32),
    # Every gradient finite while a float32 sum of them overflows.
    "finite-overflow": np.full(257, np.finfo(np.float32).max, np.float32),
}


@pytest.mark.parametrize("quantile", [False, True])
@pytest.mark.parametrize("case", sorted(GRADIENT_CASES))
def test_gradient_magnitude_precision(xgb, case, quantile):
    grad = GRADIENT_CASES[case]
    hess = np.ones_like(grad)
    X = np.zeros((len(grad), 1), np.float32)
    y = np.zeros(len(grad), np.float32)
    params = {"tree_method": "hist", "max_depth": 1, "max_bin": 4, "base_score": 0, "eta": 1, "lambda": 1,
              "min_child_weight": 1, "seed": 9}
    bst, ref = _fit_and_compare(xgb, X, y, {}, params, 1, quantile=quantile, obj=lambda p, m: (grad, hess),
                                grad=grad[None, :], hess=hess[None, :])
    root = np.float32(bst.trees_to_json()[0]["base_weights"][0])
    assert np.isfinite(root) and root != 0


# ---------------------------------------------------------------------------
# Root sums (tests/test_parent_statistics.py:24-47,
# tests/test_scalar_root_statistics.py:10-45)
# ---------------------------------------------------------------------------
ROOT_GRAD = np.asarray([2 ** 40, -2 ** 40, 3 * 2 ** -14], np.float32)
ROOT_HESS = np.asarray([1, 2, 1], np.float32)
ROOT_PARAMS = {"tree_method": "hist", "max_depth": 1, "max_bin": 4, "base_score": 0, "eta": 1, "lambda": 1,
               "min_child_weight": 1, "seed": 9}


# The reference's max_leaves = 1 variants keep the root a leaf; here an
# unreachable min_split_loss does (this engine rejects max_leaves).
STOPPED = {"gamma": 1e30}


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("quantile", [False, True])
def test_applied_parent_rounds_children(xgb, quantile, split):
    """Summing the three bins in order keeps the small last term; converting
    the large children to binary64 before adding rounds it away.  Only
    applying a split changes the stored parent weight."""
    X = np.arange(3, dtype=np.float32).reshape(-1, 1)
    y = np.zeros(3, np.float32)
    params = dict(ROOT_PARAMS) if split else dict(ROOT_PARAMS, **STOPPED)
    bst, _ = _fit_and_compare(xgb, X, y, {}, params, 1, quantile=quantile,
                              obj=lambda p, m: (ROOT_GRAD, ROOT_HESS), grad=ROOT_GRAD[None, :],
                              hess=ROOT_HESS[None, :])
    assert len(bst.trees_to_json()[0]["left_children"]) == (3 if split else 1)


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("matrix", ["raw", "quantile", "ref-dense", "ref-missing"])
@pytest.mark.parametrize("missing_feature", [None, 0, 1])
def test_root_density_and_bin_order(xgb, matrix, missing_feature, split):
    """A dense root sums feature 0's bins in bin order in binary64; a root
    with missing values uses the exact integer totals (the stopped root's
    weight differs between the two; tests/test_oracle.py pins that).  A
    reference matrix's density (ref-missing has a NaN, ref-dense none) must
    not replace the training matrix's own."""
    params = dict(ROOT_PARAMS) if split else dict(ROOT_PARAMS, **STOPPED)
    X = np.asarray([[0, 0], [1, 0], [0, 0]], np.float32)
    if missing_feature is not None:
        X[0, missing_feature] = np.nan
    y = np.zeros(3, np.float32)
    if matrix == "raw":
        d = xgb.DMatrix(X, label=y)
    else:
        options = {}
        if matrix.startswith("ref-"):
            ref_values = np.asarray([[0, 0], [1, 0], [0, 0]], np.float32)
            if matrix == "ref-missing":
                ref_values[2, 1] = np.nan
            options["ref"] = xgb.QuantileDMatrix(ref_values, max_bin=4)
        d = xgb.QuantileDMatrix(X, label=y, max_bin=4, **options)
    bst = xgb.train(params, d, 1, obj=lambda p, m: (ROOT_GRAD, ROOT_HESS))
    ref = O.train(X, y, _oracle_params(params), 1, custom_grad=ROOT_GRAD[None, :],
                  custom_hess=ROOT_HESS[None, :])
    assert_cuts_equal(d, ref)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(xgb.DMatrix(X), output_margin=True).view(np.uint32),
                                  ref["margin"].view(np.uint32))


# ---------------------------------------------------------------------------
# Partition edges (tests/test_partition_single_pass.py:65-130)
# ---------------------------------------------------------------------------
PARTITION_PARAMS = {"tree_method": "hist", "max_depth": 7, "max_bin": 32, "base_score": 0, "seed": 59}


@pytest.mark.parametrize("stable", [0, 1])
@pytest.mark.parametrize("rows", [1, 2, 255, 256, 257, 511, 513, 4099])
def test_tile_boundaries(xgb, rows, stable):
    """Partial final tiles, single-tile and many-tile parents."""
    X, y, meta = engine_inputs("missing", rows=rows)
    params = dict(PARTITION_PARAMS, hip_stable_partition=stable)
    _fit_and_compare(xgb, X, y, meta, params, 2)


@pytest.mark.parametrize("stable", [0, 1])
@pytest.mark.parametrize("side", ["left", "right"])
def test_one_sided_tiles_and_empty_children(xgb, side, stable):
    """Missing rows follow the default direction, so whole tiles feed one
    cursor, and with min_child_weight 0 a child can receive no rows."""
    rng = np.random.default_rng(19)
    X = rng.normal(size=(3000, 4)).astype(np.float32)
    X[:1800, 0] = np.nan
    y = np.where(np.isnan(X[:, 0]), 5.0 if side == "left" else -5.0, X[:, 0]).astype(np.float32)
    y += (0.1 * X[:, 1]).astype(np.float32)
    params = dict(PARTITION_PARAMS, max_depth=6, min_child_weight=0, hip_stable_partition=stable)
    _fit_and_compare(xgb, X, y, {}, params, 2)


def full_frontier_data(pruned=False):
    """Every 10-bit pattern once, y its value (tests/test_gpu_tree_deep.py:12-24):
    all ten bits useful in descending significance, a balanced full tree."""
    values = np.arange(1024, dtype=np.uint32)
    X = ((values[:, None] >> np.arange(10, dtype=np.uint32)) & 1).astype(np.float32)
    y = values.astype(np.float32)
    if pruned:
        constant_pairs = (values // 2) % 3 == 0
        y[constant_pairs] = (values[constant_pairs] // 2 * 2).astype(np.float32)
    return X, y


@pytest.mark.parametrize("stable", [0, 1])
@pytest.mark.parametrize("quantile,pruned", [(False, False), (True, False), (False, True), (True, True)])
def test_full_and_pruned_deep_frontiers(xgb, quantile, pruned, stable):
    X, y = full_frontier_data(pruned)
    params = {"tree_method": "hist", "max_depth": 10, "max_bin": 2, "min_child_weight": 1, "lambda": 0,
              "base_score": 0, "eta": 0.3, "seed": 71, "hip_stable_partition": stable}
    bst, _ = _fit_and_compare(xgb, X, y, {}, params, 1, quantile=quantile)
    left = np.asarray(bst.trees_to_json()[0]["left_children"])
    np.testing.assert_array_equal(left[:511], 2 * np.arange(511) + 1)
    expanded = np.count_nonzero(left[511:1023] >= 0)
    if pruned:
        assert 256 < expanded < 512
        assert len(left) == 1023 + 2 * expanded
    else:
        assert expanded == 512 and len(left) == 2047


def bit_patterns(bits):
    """Every `bits`-bit pattern once, y = sum over set bits j of 1 + j/64:
    each bit splits any node's rows in half with a gain of at least a
    quarter of its rows, the highest remaining bit strictly best, so the
    tree is full to depth `bits` (y = the pattern's value instead loses its
    last splits to binary32 cancellation against the parent's gain beyond
    depth 10)."""
    values = np.arange(1 << bits, dtype=np.uint32)
    X = ((values[:, None] >> np.arange(bits, dtype=np.uint32)) & 1).astype(np.float32)
    return X, (X @ (1 + np.arange(bits, dtype=np.float32) / 64)).astype(np.float32)


@pytest.mark.parametrize("stable", [0, 1])
@pytest.mark.parametrize("depth", [12, 14, 16])
def test_full_frontiers_beyond_depth_ten(xgb, depth, stable):
    """Every depth-bit pattern once: a full tree to the deepest depth the
    engine takes (16), whose last levels hold up to 2^15 nodes -- past the
    2,048 that a level's bookkeeping plans from the counting pass, so the
    separate planning launch takes those levels."""
    X, y = bit_patterns(depth)
    params = {"tree_method": "hist", "max_depth": depth, "max_bin": 2, "min_child_weight": 1, "lambda": 0,
              "base_score": 0, "eta": 0.3, "seed": 71, "hip_stable_partition": stable}
    bst, _ = _fit_and_compare(xgb, X, y, {}, params, 1)
    left = np.asarray(bst.trees_to_json()[0]["left_children"])
    internal = (1 << depth) - 1
    np.testing.assert_array_equal(left[:internal], 2 * np.arange(internal) + 1)
    assert len(left) == 2 * internal + 1


@pytest.mark.parametrize("depth", [12, 14])
def test_csr_full_frontiers_beyond_depth_ten(xgb, depth):
    """The same patterns as a CSR matrix whose zero bits are absent
    (missing): every split is present against missing, down to depth 14."""
    import scipy.sparse as sp
    X, y = bit_patterns(depth)
    csr = sp.csr_matrix(X)
    csr.eliminate_zeros()
    dense = np.where(X == 0, np.float32(np.nan), X).astype(np.float32)
    params = {"tree_method": "hist", "max_depth": depth, "max_bin": 2, "min_child_weight": 1, "lambda": 0,
              "base_score": 0, "eta": 0.3, "seed": 71}
    d = xgb.DMatrix(csr, label=y)
    bst = xgb.train(params, d, 1)
    ref = O.train(dense, y, _oracle_params(params), 1)
    assert_cuts_equal(d, ref)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d, output_margin=True).view(np.uint32),
                                  ref["margin"].view(np.uint32))
    left = np.asarray(bst.trees_to_json()[0]["left_children"])
    assert len(left) == 2 * ((1 << depth) - 1) + 1


@pytest.mark.parametrize("depth", [9, 10])
def test_deep_subnormal_leaves(xgb, depth):
    """eta = the smallest normal float32 and labels / 128: the leaves are
    subnormal (tests/test_gpu_tree_deep.py:100-113); the device keeps them
    (no flush to zero)."""
    X, y = full_frontier_data()
    y = (y * np.float32(1 / 128)).astype(np.float32)
    params = {"tree_method": "hist", "max_depth": depth, "max_bin": 2, "min_child_weight": 1, "lambda": 0,
              "base_score": 0, "eta": float(np.finfo(np.float32).tiny), "seed": 71}
    bst, _ = _fit_and_compare(xgb, X, y, {}, params, 1)
    tree = bst.trees_to_json()[0]
    leaves = np.asarray(tree["split_conditions"], np.float32)[np.asarray(tree["left_children"]) < 0]
    assert np.any((np.abs(leaves) > 0) & (np.abs(leaves) < np.finfo(np.float32).tiny))


# ---------------------------------------------------------------------------
# The gain without fused multiply-adds (fma_contract = 0) on both sides
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("config,rows,rounds", [(0, 20000, 10), (1, 20000, 10), (2, 30000, 5)])
def test_trees_match_oracle_without_contraction(xgb, config, rows, rounds):
    gen = {0: W.config0, 1: W.config1, 2: W.config2}[config]
    X, y = gen(rows=rows, cols={0: 32, 1: 32, 2: 64}[config])
    params = dict(W.CONFIG_PARAMS[config], fma_contract=0)
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, rounds)
    op = _oracle_params(params)
    op.fma_contract = 0
    ref = O.train(X, y, op, rounds)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), ref["margin"].view(np.uint32))


@pytest.mark.parametrize("label_scale,params", [
    (1.0, {"max_depth": 6, "max_bin": 64, "min_child_weight": 5}),
    (1e-2, {"max_depth": 5, "max_bin": 32, "lambda": 0.001, "min_child_weight": 0}),
    (1e18, {"max_depth": 5, "max_bin": 32, "min_child_weight": 2}),
    (1.0, {"max_depth": 5, "max_bin": 64, "alpha": 0.2, "min_child_weight": 3}),
    (1.0, {"max_depth": 5, "max_bin": 64, "max_delta_step": 0.4}),
])
def test_split_gain_without_contraction(xgb, label_scale, params):
    from test_gpu_parity import _tie_matrix
    X, y = _tie_matrix(3000, 11)
    y = (y * np.float32(label_scale)).astype(np.float32)
    params = dict(params, objective="reg:squarederror", tree_method="hist", eta=0.3, fma_contract=0)
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, 4)
    op = _oracle_params(params)
    op.fma_contract = 0
    ref = O.train(X, y, op, 4)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), ref["margin"].view(np.uint32))


def test_logistic_without_contraction(xgb):
    X, _ = W.config1(rows=20000, cols=12)
    s = np.nan_to_num(X[:, :4]).sum(axis=1)
    y = (np.random.default_rng(2).random(len(X)) < 1 / (1 + np.exp(-s))).astype(np.float32)
    params = {"objective": "binary:logistic", "tree_method": "hist", "max_depth": 6, "max_bin": 128, "eta": 0.3,
              "fma_contract": 0}
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, 5)
    op = _oracle_params(params)
    op.fma_contract = 0
    ref = O.train(X, y, op, 5)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d, output_margin=True).view(np.uint32), ref["margin"].view(np.uint32))


# ---------------------------------------------------------------------------
# Device gradients and scales against the oracle's, directly
# ---------------------------------------------------------------------------
def _device_gradients(objective, margin, labels, weights=None, scale_pos_weight=1.0):
    rows = len(labels)
    dm, dl = D.Device.of(np.ascontiguousarray(margin, np.float32)), D.Device.of(np.ascontiguousarray(labels, np.float32))
    dw = D.Device.of(np.ascontiguousarray(weights, np.float32)) if weights is not None else None
    grad, scales, mass = D.Device(rows * 8), D.Device(8), D.Device(MASS_WORDS * 8)
    gp = MgbGradParams(rows, objective, 0 if weights is None else 1, 0, scale_pos_weight, 1.0, 0.0, 0.0)
    D.check(D.lib().mgb_gradients(ctypes.byref(gp), dm.ptr, dl.ptr, dw.ptr if dw else None, grad.ptr, mass.ptr,
                                  scales.ptr))
    gh = grad.read(np.float32, rows * 2).reshape(rows, 2)
    return gh[:, 0].copy(), gh[:, 1].copy(), scales.read(np.float32, 2)


def _device_scales(grad, hess):
    rows = len(grad)
    gh = np.ascontiguousarray(np.stack([grad, hess], axis=1).astype(np.float32))
    dg, scales, mass = D.Device.of(gh), D.Device(8), D.Device(MASS_WORDS * 8)
    gp = MgbGradParams(rows, 0, 0, 0, 1.0, 1.0, 0.0, 0.0)
    D.check(D.lib().mgb_gradient_mass(ctypes.byref(gp), dg.ptr, mass.ptr, scales.ptr))
    return scales.read(np.float32, 2)


def _oracle_gradients(objective, margin, labels, weights=None, scale_pos_weight=1.0):
    rows = len(labels)
    g, h = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    O.lib().oracle_gradients(ctypes.c_int32(objective), O.ptr(np.ascontiguousarray(margin, np.float32)),
                             O.ptr(np.ascontiguousarray(labels, np.float32)), O.ptr(w), ctypes.c_uint32(rows),
                             ctypes.c_float(scale_pos_weight), O.ptr(g), O.ptr(h))
    return g, h


@pytest.mark.parametrize("objective,weighted,spw", [(0, False, 1.0), (0, True, 1.0), (1, False, 1.0),
                                                     (1, True, 3.0), (2, False, 1.0)])
def test_device_gradients_and_scales_match_oracle(objective, weighted, spw):
    rng = np.random.default_rng(31 + objective)
    rows = 300_001
    margin = rng.normal(0, 3, rows).astype(np.float32)
    margin[:6] = [0.0, -0.0, 88.0, -88.0, 1e-30, -104.0]
    labels = (rng.normal(size=rows).astype(np.float32) if objective == 0
              else (rng.random(rows) < 0.3).astype(np.float32))
    weights = rng.uniform(0, 3, rows).astype(np.float32) if weighted else None
    if weighted:
        weights[::17] = 0
    g, h, scales = _device_gradients(objective, margin, labels, weights, spw)
    og, oh = _oracle_gradients(objective, margin, labels, weights, spw)
    np.testing.assert_array_equal(g.view(np.uint32), og.view(np.uint32))
    np.testing.assert_array_equal(h.view(np.uint32), oh.view(np.uint32))
    assert scales[0] == np.float32(O.gradient_scale(og))
    assert scales[1] == np.float32(O.gradient_scale(oh))


@pytest.mark.parametrize("values", [
    [2.0 ** 16, -(2.0 ** 16), 6.118193027759844e-7],
    [np.finfo(np.float32).max] * 257,
    [2.0 ** -149, -(2.0 ** -149), 1e-40, 0.0],
    [0.0, -0.0],
    [1.0] * 100_000 + [2.0 ** -60],
])
def test_device_scales_of_adversarial_gradients(values):
    """The exact |g| mass (2^-149 units, no float rounding) and its scale for
    extreme magnitudes: the device equals the oracle, which equals an exact
    big-integer computation (tests/test_oracle.py)."""
    v = np.asarray(values, np.float32)
    scales = _device_scales(v, v[::-1].copy())
    assert scales[0] == np.float32(O.gradient_scale(v))
    assert scales[1] == np.float32(O.gradient_scale(v[::-1].copy()))


# ---------------------------------------------------------------------------
# BASELINE config 4's own generator
# ---------------------------------------------------------------------------
def test_config4_generator_matches_oracle(xgb):
    """Config 4's 128 columns (N(0,1), U(0,1), integers), its Bernoulli
    labels and its parameters (logistic, depth 10, 1,024 bins, subsample and
    colsample_bytree 0.8) at 200,000 rows, 5 rounds."""
    import os
    X, y = W.config4(rows=200_000)
    params = dict(W.CONFIG_PARAMS[4])
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, 5)
    op = _oracle_params(params)
    op.nthread = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    ref = O.train(X, y, op, 5)
    assert_cuts_equal(d, ref)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d, output_margin=True).view(np.uint32), ref["margin"].view(np.uint32))


# ---------------------------------------------------------------------------
# The reweighted logistic intercept (kernels/boost.metal:379-381): with
# scale_pos_weight != 1 the base score sums binary32 products y * w.
# ---------------------------------------------------------------------------
def _product_rule_rows(count):
    """Single (label, weight) rows whose base score differs between binary32
    and exact products (labels below 1, so scale_pos_weight scales no weight):
    the oracle with scale_pos_weight 2.5 takes binary32 products, with 1 exact
    ones."""
    rng = np.random.default_rng(2024)
    rows = []
    while len(rows) < count:
        y = np.float32(rng.uniform(0.05, 0.95))
        w = np.float32(rng.uniform(0.3, 7.0))
        if O.base_score([y], [w], objective=1, scale_pos_weight=2.5) != \
                O.base_score([y], [w], objective=1, scale_pos_weight=1.0):
            rows.append((y, w))
    return rows


def test_reweighted_logistic_base_score_matches_oracle(xgb):
    params = {"tree_method": "hist", "objective": "binary:logistic", "scale_pos_weight": 2.5, "max_depth": 2,
              "max_bin": 8, "eta": 0.5}
    X = np.asarray([[0.25, -1.0, 3.0]], np.float32)
    for y, w in _product_rule_rows(4):
        label = np.asarray([y], np.float32)
        bst, ref = _fit_and_compare(xgb, X, label, {"weight": np.asarray([w], np.float32)}, params, 2)
        model = json.loads(bst.save_raw("json"))
        text = model["learner"]["learner_model_param"]["base_score"]  # "[v]", nine significant digits
        got = np.float32(json.loads(text)[0] if text.startswith("[") else float(text))
        want = np.float32(O.base_score(label, [w], objective=1, scale_pos_weight=2.5))
        assert got.view(np.uint32) == want.view(np.uint32), (y, w)


@pytest.mark.parametrize("objective", ["binary:logistic", "binary:logitraw"])
def test_scale_pos_weight_training_matches_oracle(xgb, objective):
    """scale_pos_weight end to end: the positive rows' weights in the base
    score and in every round's gradients (kernels/boost.metal:566-570)."""
    X, y = W.config1(rows=6000, cols=8, seed=19)
    labels = (y > np.median(y)).astype(np.float32)
    weight = np.random.default_rng(5).uniform(0.2, 2.0, len(y)).astype(np.float32)
    params = {"tree_method": "hist", "objective": objective, "scale_pos_weight": 3.0, "max_depth": 5,
              "max_bin": 64, "eta": 0.3}
    _fit_and_compare(xgb, X, labels, {"weight": weight}, params, 5)



@pytest.mark.parametrize("objective,base_score", [("binary:logitraw", 0.3), ("binary:logitraw", -1.25),
                                                  ("binary:logistic", 0.3)])
def test_given_base_score_margin_matches_oracle(xgb, objective, base_score):
    """A given base_score is the logistic score's probability but logitraw's
    margin itself (src/objectives.cpp:17-31 score_margins)."""
    X, y = W.config1(rows=3000, cols=6, seed=23)
    labels = (y > 0).astype(np.float32)
    params = {"tree_method": "hist", "objective": objective, "base_score": base_score, "max_depth": 4,
              "max_bin": 32, "eta": 0.3}
    _fit_and_compare(xgb, X, labels, {}, params, 3)
