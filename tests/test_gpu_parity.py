"""GPU parity: the HIP path against the CPU oracle and the published known answers.

Kernel-level checks go through the kernel C ABI (include/mgb_kernels.h);
end-to-end checks go through the drop-in API (xgb.train -> C API).
"""
import ctypes
import hashlib

import numpy as np
import pytest

import device_lib as D
import oracle_lib as O
import workloads as W

pytestmark = pytest.mark.gpu


def _oracle_params(params, rounds_override=None):
    return O.make_params(objective=params.get("objective", "reg:squarederror"), max_depth=params["max_depth"],
                         max_bin=params["max_bin"], eta=float(np.float32(params.get("eta", 0.3))),
                         reg_lambda=float(params.get("lambda", 1.0)), reg_alpha=float(params.get("alpha", 0.0)),
                         min_child_weight=float(params.get("min_child_weight", 1.0)),
                         max_delta_step=float(params.get("max_delta_step", 0.0)),
                         min_split_loss=float(params.get("gamma", 0.0)),
                         scale_pos_weight=float(np.float32(params.get("scale_pos_weight", 1.0))),
                         base_score=params.get("base_score"),
                         subsample=float(params.get("subsample", 1.0)),
                         colsample_bytree=float(params.get("colsample_bytree", 1.0)),
                         seed=int(params.get("seed", 0)),
                         seed_per_iteration=int(params.get("seed_per_iteration", 0)),
                         std_shuffle=params.get("std_shuffle", "libstdc++"))


def assert_trees_equal(bst, oracle_result):
    trees = bst.trees_to_json()
    assert len(trees) == len(oracle_result["sizes"])
    for t, tree in enumerate(trees):
        n = int(oracle_result["sizes"][t])
        ref = oracle_result["trees"][t][:n]
        assert len(tree["left_children"]) == n, f"tree {t}: node count"
        np.testing.assert_array_equal(tree["left_children"], ref["left"], err_msg=f"tree {t} left")
        np.testing.assert_array_equal(tree["right_children"], ref["right"], err_msg=f"tree {t} right")
        feat = np.where(ref["feature"] < 0, 0, ref["feature"])
        np.testing.assert_array_equal(tree["split_indices"], feat, err_msg=f"tree {t} features")
        np.testing.assert_array_equal(tree["default_left"], ref["default_left"], err_msg=f"tree {t} default_left")
        cond = np.where(ref["left"] < 0, ref["leaf"], ref["threshold"]).astype(np.float32)
        got = np.asarray(tree["split_conditions"], np.float32)
        np.testing.assert_array_equal(got.view(np.uint32), cond.view(np.uint32), err_msg=f"tree {t} conditions")
        for name, field in [("base_weights", "base_weight"), ("sum_hessian", "cover"), ("loss_changes", "gain")]:
            got = np.asarray(tree[name], np.float32)
            np.testing.assert_array_equal(got.view(np.uint32), ref[field].astype(np.float32).view(np.uint32),
                                          err_msg=f"tree {t} {name}")


# ---------------------------------------------------------------------------
# Kernel level
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("missing", [False, True])
@pytest.mark.parametrize("max_bin", [16, 256])
def test_sketch_cuts_match_oracle(missing, max_bin):
    X, _ = W.config1(rows=30000, cols=8) if missing else W.config0(rows=30000, cols=8)
    X[:, 3] = np.round(X[:, 3] * 2)  # few distinct values, with long runs
    cuts, counts = D.sketch_cuts(X, max_bin)
    ocuts, ocounts, _ = O.sketch_cuts(X, max_bin)
    np.testing.assert_array_equal(counts, ocounts)
    for f in range(X.shape[1]):
        c = counts[f]
        np.testing.assert_array_equal(cuts[f, :c].view(np.uint32), ocuts[f, :c].view(np.uint32))


def test_sketch_cuts_weighted_match_oracle():
    X, _ = W.config0(rows=20000, cols=4)
    w = np.random.default_rng(3).uniform(0.1, 2.0, len(X)).astype(np.float32)
    cuts, counts = D.sketch_cuts(X, 256, w)
    ocuts, ocounts, _ = O.sketch_cuts(X, 256, w)
    np.testing.assert_array_equal(counts, ocounts)
    for f in range(X.shape[1]):
        np.testing.assert_array_equal(cuts[f, :counts[f]].view(np.uint32), ocuts[f, :counts[f]].view(np.uint32))


@pytest.mark.parametrize("group_entries", [1, 3 * 30000, 0])
def test_sketch_feature_groups_match_oracle(group_entries):
    # One feature per group, groups of three (3 + 3 + 2) and the default (one
    # group): the cuts do not depend on how the features are grouped.
    X, _ = W.config1(rows=30000, cols=8)
    X[:, 3] = np.round(X[:, 3] * 2)
    w = np.random.default_rng(5).uniform(0.1, 2.0, len(X)).astype(np.float32)
    D.check(D.lib().mgb_sketch_group_entries(ctypes.c_uint64(group_entries)))
    try:
        got = [D.sketch_cuts(X, 64), D.sketch_cuts(X, 64, w)]
    finally:
        D.check(D.lib().mgb_sketch_group_entries(ctypes.c_uint64(0)))
    for (cuts, counts), weights in zip(got, [None, w]):
        ocuts, ocounts, _ = O.sketch_cuts(X, 64, weights)
        np.testing.assert_array_equal(counts, ocounts)
        for f in range(X.shape[1]):
            np.testing.assert_array_equal(cuts[f, :counts[f]].view(np.uint32), ocuts[f, :counts[f]].view(np.uint32))


@pytest.mark.parametrize("bin_bytes,G,group_major,unit", [
    (1, 16, False, False), (1, 4, False, False), (2, 8, False, False), (1, 4, True, False), (2, 4, True, False),
    (1, 16, True, False), (1, 1, False, False), (1, 2, False, False), (2, 2, False, False), (2, 16, False, False),
    (1, 8, False, True), (2, 1, True, True), (2, 16, False, True), (1, 2, True, True)])
def test_bins_and_histogram_match_oracle(bin_bytes, G, group_major, unit):
    """Codes and histograms (the root's identity rows and a gathered row list)
    against brute-force integer sums, for every feature-group width with u8
    and u16 codes, row- and group-major layouts, explicit and unit Hessians:
    21 features leave a partial last group for every G above 1, and missing
    values go to the missing slot."""
    rng = np.random.default_rng(11)
    X, y = W.config1(rows=9000, cols=21)
    ocuts, ocounts, _ = O.sketch_cuts(X, 64)
    obins = O.quantize(X, ocuts, ocounts)
    m, dbins, bins, missing = D.quantize_bins(X, ocuts, ocounts, 64, bin_bytes, G, group_major=group_major)
    assert missing
    code = 0xFF if bin_bytes == 1 else 0xFFFF
    got = bins[:, :X.shape[1]].astype(np.int64)
    want = np.where(obins == 0xFFFF, code, obins).astype(np.int64)
    np.testing.assert_array_equal(got, want)
    grad = rng.normal(size=len(X)).astype(np.float32)
    hess = np.ones(len(X), np.float32) if unit else rng.uniform(0.1, 1.0, len(X)).astype(np.float32)
    sg, sh = O.gradient_scale(grad), O.gradient_scale(hess)
    qg = np.rint(grad.astype(np.float32) * np.float32(sg)).astype(np.int64)
    qh = np.rint(hess.astype(np.float32) * np.float32(sh)).astype(np.int64)
    for rows_list in [None, np.sort(rng.choice(len(X), 3001, replace=False)).astype(np.uint32)]:
        hist = D.histogram(m, dbins, rows_list, grad, hess, [sg, sh], G, unit=unit, rows_per_tile=1024)
        idx = np.arange(len(X)) if rows_list is None else rows_list.astype(np.int64)
        # Brute-force integer sums (mod 2^64) per (feature, bin); bin max_bin = missing.
        for f in range(X.shape[1]):
            b = obins[idx, f].astype(np.int64)
            b = np.where(b == 0xFFFF, 64, b)
            eg = np.zeros(65, np.uint64)
            eh = np.zeros(65, np.uint64)
            np.add.at(eg, b, qg[idx].astype(np.uint64))
            np.add.at(eh, b, qh[idx].astype(np.uint64))
            np.testing.assert_array_equal(hist[f, :, 0].astype(np.uint64), eg)
            np.testing.assert_array_equal(hist[f, :, 1].astype(np.uint64), eh)


def test_dense_u8_uses_all_256_codes():
    """A matrix without missing values keeps u8 codes for 256 bins: code 255 is
    a real bin, counted in bin 255 of the histogram, not in the missing slot."""
    X, _ = W.config0(rows=20000, cols=4)
    ocuts, ocounts, _ = O.sketch_cuts(X, 256)
    assert ocounts.max() == 256
    obins = O.quantize(X, ocuts, ocounts)
    m, dbins, bins, missing = D.quantize_bins(X, ocuts, ocounts, 256, 1, 4, dense=True)
    assert not missing
    np.testing.assert_array_equal(bins[:, :4], obins)
    grad = np.ones(len(X), np.float32)
    hist = D.histogram(m, dbins, None, grad, grad, [O.gradient_scale(grad)] * 2, 4)
    counts = hist[:, :, 1] // int(np.float32(O.gradient_scale(grad)))
    for f in range(4):
        np.testing.assert_array_equal(counts[f, :256], np.bincount(obins[:, f], minlength=256))
        assert counts[f, 256] == 0


# ---------------------------------------------------------------------------
# End to end through the drop-in API
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["dense100", "missing100", "dense262"])
def test_published_prediction_hashes(xgb, case):
    """Stock XGBoost 3.4.1 CPU hist predictions (published SHA-256), reproduced on the GPU."""
    spec = W.KNOWN_ANSWERS[case]
    X, y = W.known_answer_data(case)
    params = dict(W.KNOWN_PARAMS, max_depth=spec["depth"])
    bst = xgb.train(params, xgb.DMatrix(X, label=y), 100)
    pred = bst.predict(xgb.DMatrix(X, label=y))
    assert hashlib.sha256(pred.tobytes()).hexdigest() == spec["prediction_sha256"]
    # Prediction cache of the training matrix gives the same bytes.
    d = xgb.DMatrix(X, label=y)
    bst2 = xgb.train(params, d, 100)
    assert hashlib.sha256(bst2.predict(d).tobytes()).hexdigest() == spec["prediction_sha256"]


@pytest.mark.parametrize("config,rows,rounds", [(0, 20000, 10), (1, 20000, 10), (2, 30000, 5), (0, 100000, 20),
                                                 (1, 100000, 20)])
def test_trees_match_oracle(xgb, config, rows, rounds):
    gen = {0: W.config0, 1: W.config1, 2: W.config2}[config]
    X, y = gen(rows=rows, cols={0: 32, 1: 32, 2: 64}[config])
    params = W.CONFIG_PARAMS[config]
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, rounds)
    ref = O.train(X, y, _oracle_params(params), rounds)
    assert_trees_equal(bst, ref)
    pred = bst.predict(d)
    np.testing.assert_array_equal(pred.view(np.uint32), ref["margin"].view(np.uint32))
    cut_ptr, cut_values = d.get_quantile_cut()
    np.testing.assert_array_equal(np.diff(cut_ptr), ref["cut_counts"])
    for f in range(X.shape[1]):
        c = ref["cut_counts"][f]
        np.testing.assert_array_equal(cut_values[cut_ptr[f]:cut_ptr[f + 1]].view(np.uint32),
                                      ref["cuts"][f, :c].view(np.uint32))
    # A fresh matrix (no prediction cache) predicts the same bytes.
    np.testing.assert_array_equal(bst.predict(xgb.DMatrix(X)).view(np.uint32), ref["margin"].view(np.uint32))


@pytest.mark.parametrize("params", [
    {"max_depth": 5, "max_bin": 32, "eta": 0.5, "lambda": 0.5, "alpha": 0.3, "min_child_weight": 3},
    {"max_depth": 3, "max_bin": 2, "eta": 1.0, "lambda": 0.0, "min_child_weight": 0, "gamma": 0.5},
    {"max_depth": 7, "max_bin": 1024, "eta": 0.1, "max_delta_step": 0.7},
])
def test_regularisation_parity(xgb, params):
    X, y = W.config1(rows=15000, cols=12)
    params = dict(params, objective="reg:squarederror", tree_method="hist")
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, 6)
    ref = O.train(X, y, _oracle_params(params), 6)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), ref["margin"].view(np.uint32))


def _tie_matrix(rows, seed):
    """Columns that repeat or monotonically transform earlier ones (equal
    partitions, so equal gains across features) beside few-valued integer
    columns (many equal Hessian counts at bin edges)."""
    rng = np.random.default_rng(seed)
    base = rng.normal(size=(rows, 4)).astype(np.float32)
    ints = rng.integers(0, 6, size=(rows, 3)).astype(np.float32)
    X = np.concatenate([base, base[:, :2], 2.0 * base[:, 2:3] + 1.0, ints, ints[:, :1]], axis=1).astype(np.float32)
    y = (base[:, 0] - 0.5 * base[:, 1] + 0.3 * ints[:, 0] + 0.1 * rng.normal(size=rows)).astype(np.float32)
    return X, y


@pytest.mark.parametrize("label_scale,params", [
    (1.0, {"max_depth": 6, "max_bin": 64, "min_child_weight": 5}),
    (1.0, {"max_depth": 6, "max_bin": 256, "lambda": 0.0, "min_child_weight": 0}),
    (1e-2, {"max_depth": 5, "max_bin": 32, "lambda": 0.001, "min_child_weight": 0}),
    (1e12, {"max_depth": 5, "max_bin": 32}),
    (1e15, {"max_depth": 5, "max_bin": 32, "min_child_weight": 2}),
    (1e18, {"max_depth": 5, "max_bin": 32, "min_child_weight": 2}),
    (1.0, {"max_depth": 5, "max_bin": 64, "alpha": 0.2, "min_child_weight": 3}),
])
def test_split_gain_bounds_parity(xgb, label_scale, params):
    """The split kernel scores exactly only the candidates whose division-free
    gain bounds reach the node's best lower bound; equal gains across
    features, Hessian sums on the min_child_weight boundary, and gradient
    magnitudes near the ends of the float range must still pick the oracle's
    first strictly greater candidate."""
    X, y = _tie_matrix(3000, 11)
    y = (y * np.float32(label_scale)).astype(np.float32)
    params = dict(params, objective="reg:squarederror", tree_method="hist", eta=0.3)
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, 4)
    ref = O.train(X, y, _oracle_params(params), 4)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), ref["margin"].view(np.uint32))


def test_weighted_regression_parity(xgb):
    X, y = W.config0(rows=20000, cols=8)
    w = np.random.default_rng(144).uniform(0.1, 2.0, len(X)).astype(np.float32)
    params = {"max_depth": 6, "max_bin": 256, "eta": 0.3, "objective": "reg:squarederror"}
    d = xgb.DMatrix(X, label=y, weight=w)
    bst = xgb.train(params, d, 5)
    ref = O.train(X, y, _oracle_params(params), 5, weights=w)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), ref["margin"].view(np.uint32))


def test_logistic_parity(xgb):
    rng = np.random.default_rng(5)
    X, _ = W.config1(rows=30000, cols=16)
    s = np.nan_to_num(X[:, :4]).sum(axis=1)
    y = (rng.random(len(X)) < 1 / (1 + np.exp(-s))).astype(np.float32)
    params = {"objective": "binary:logistic", "max_depth": 6, "max_bin": 256, "eta": 0.1}
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, 10)
    ref = O.train(X, y, _oracle_params(params), 10)
    assert_trees_equal(bst, ref)
    margin = bst.predict(d, output_margin=True)
    np.testing.assert_array_equal(margin.view(np.uint32), ref["margin"].view(np.uint32))
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), O.sigmoid(ref["margin"]).view(np.uint32))


# ---------------------------------------------------------------------------
# CSR input (the sparse path: per-nonzero codes, atomics histogram, missing
# slots from node totals, row lookups in the partition and the predictor)
# ---------------------------------------------------------------------------
def _csr(indptr, indices, values, cols):
    import scipy.sparse as sp
    return sp.csr_matrix((values, indices, indptr), shape=(len(indptr) - 1, cols))


def test_csr_sketch_feature_groups_match_oracle(xgb):
    """The CSR sketch (from the column-major copy) over groups of a few
    hundred entries -- whole columns per group, so many groups -- gives the
    oracle's cuts, as the default single group does."""
    cols = 300
    indptr, indices, values, _ = W.config3(rows=12000, cols=cols, nnz=20, informative=40, seed=23)
    X = W.csr_to_dense(indptr, indices, values, cols)
    y = np.nan_to_num(X[:, :40]).sum(axis=1).astype(np.float32)
    params = {"objective": "reg:squarederror", "tree_method": "hist", "max_depth": 4, "max_bin": 256}
    ref = O.train(X, y, _oracle_params(params), 1)
    lib = xgb.core._LIB
    for entries in (2000, 0):
        assert lib.mgb_sketch_group_entries(ctypes.c_uint64(entries)) == 0
        try:
            d = xgb.DMatrix(_csr(indptr, indices, values, cols), label=y)
            bst = xgb.train(params, d, 1)
            cut_ptr, cut_values = d.get_quantile_cut()
        finally:
            lib.mgb_sketch_group_entries(ctypes.c_uint64(0))
        np.testing.assert_array_equal(np.diff(cut_ptr), ref["cut_counts"])
        for f in range(cols):
            c = ref["cut_counts"][f]
            np.testing.assert_array_equal(cut_values[cut_ptr[f]:cut_ptr[f + 1]].view(np.uint32),
                                          ref["cuts"][f, :c].view(np.uint32))
        assert_trees_equal(bst, ref)



@pytest.mark.parametrize("sparse", [True, False])
def test_features_beyond_65535_match_oracle(xgb, sparse):
    """66,000 features, the label carried by features 65,900 (in every row)
    and 100 (in half of them): past 65,535 features a node's best-split key
    holds the feature alone and the partition rebuilds the split from the
    feature's record, so trees splitting on feature 65,900 check that path,
    as CSR and as a dense matrix with the absent entries missing."""
    import scipy.sparse as sp
    rows, cols = 2000, 66000
    rng = np.random.default_rng(3)
    r = np.repeat(np.arange(rows), 6)
    c = rng.integers(0, cols, size=rows * 6)
    v = rng.normal(size=rows * 6).astype(np.float32)
    strong = rng.normal(size=rows).astype(np.float32)
    weak = rng.normal(size=rows).astype(np.float32)
    half = rng.random(rows) < 0.5
    r = np.concatenate([r, np.arange(rows), np.nonzero(half)[0]])
    c = np.concatenate([c, np.full(rows, 65900), np.full(half.sum(), 100)])
    v = np.concatenate([v, strong, weak[half]])
    csr = sp.csr_matrix((v, (r, c)), shape=(rows, cols))
    csr.sum_duplicates()
    csr.sort_indices()
    y = ((strong + 0.7 * np.where(half, weak, 0)) > 0).astype(np.float32)
    X = W.csr_to_dense(csr.indptr, csr.indices, csr.data.astype(np.float32), cols)
    params = {"objective": "binary:logistic", "tree_method": "hist", "max_depth": 4, "max_bin": 16, "eta": 0.3}
    d = xgb.DMatrix(csr if sparse else X, label=y)
    bst = xgb.train(params, d, 2)
    ref = O.train(X, y, _oracle_params(params), 2)
    assert 65900 in [int(n["feature"]) for n in ref["trees"][0][:ref["sizes"][0]]]
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d, output_margin=True).view(np.uint32), ref["margin"].view(np.uint32))


@pytest.mark.parametrize("group_entries", [0, 20000])
def test_csr_sketch_skewed_columns_match_oracle(xgb, group_entries):
    """One dense column among 2,000 nearly empty ones (0 to 3 entries each)
    and a half-dense one: the sketch's run passes take a work list of each
    column's blocks, so the skew costs no idle workgroups and no block table
    sized by the longest column.  Cuts and the first tree equal the oracle's
    with one group and with groups of about 20,000 entries (the dense
    columns then form groups of their own)."""
    rows, cols = 60000, 2002
    rng = np.random.default_rng(41)
    per_col = [np.arange(rows), np.sort(rng.choice(rows, rows // 2, replace=False))]
    per_col += [np.sort(rng.choice(rows, k, replace=False)) for k in rng.integers(0, 4, size=cols - 2)]
    r = np.concatenate(per_col)
    c = np.concatenate([np.full(len(v), j) for j, v in enumerate(per_col)])
    v = rng.normal(size=len(r)).astype(np.float32)
    v[c == 1] = np.round(v[c == 1] * 4)  # runs of equal values in the half-dense column
    import scipy.sparse as sp
    csr = sp.csr_matrix((v, (r, c)), shape=(rows, cols))
    csr.sort_indices()
    X = W.csr_to_dense(csr.indptr, csr.indices, csr.data, cols)
    y = (np.nan_to_num(X[:, 0]) + 0.5 * np.nan_to_num(X[:, 1])).astype(np.float32)
    params = {"objective": "reg:squarederror", "tree_method": "hist", "max_depth": 4, "max_bin": 64}
    ref = O.train(X, y, _oracle_params(params), 1)
    lib = xgb.core._LIB
    assert lib.mgb_sketch_group_entries(ctypes.c_uint64(group_entries)) == 0
    try:
        d = xgb.DMatrix(csr, label=y)
        bst = xgb.train(params, d, 1)
        cut_ptr, cut_values = d.get_quantile_cut()
    finally:
        lib.mgb_sketch_group_entries(ctypes.c_uint64(0))
    np.testing.assert_array_equal(np.diff(cut_ptr), ref["cut_counts"])
    for f in range(cols):
        k = ref["cut_counts"][f]
        np.testing.assert_array_equal(cut_values[cut_ptr[f]:cut_ptr[f + 1]].view(np.uint32),
                                      ref["cuts"][f, :k].view(np.uint32), err_msg=f"feature {f}")
    assert_trees_equal(bst, ref)


@pytest.mark.parametrize("max_bin,root_columns", [(64, 1), (256, 1), (1024, 1), (256, 0)])
def test_csr_regression_matches_oracle(xgb, max_bin, root_columns):
    """Squared error on a config-3 style CSR matrix: cuts, trees and margins
    bit-identical to the oracle run on the dense matrix with NaN at the
    absent entries (u8 codes, and u16 at 1024 bins)."""
    cols = 300
    indptr, indices, values, _ = W.config3(rows=12000, cols=cols, nnz=20, informative=40, seed=21)
    X = W.csr_to_dense(indptr, indices, values, cols)
    y = (np.nan_to_num(X[:, :40]).sum(axis=1) + 0.1 * np.random.default_rng(3).normal(size=len(X))).astype(np.float32)
    params = {"objective": "reg:squarederror", "tree_method": "hist", "max_depth": 6, "max_bin": max_bin, "eta": 0.3,
              "hip_csr_root_columns": root_columns}
    d = xgb.DMatrix(_csr(indptr, indices, values, cols), label=y)
    bst = xgb.train(params, d, 5)
    ref = O.train(X, y, _oracle_params(params), 5)
    cut_ptr, cut_values = d.get_quantile_cut()
    np.testing.assert_array_equal(np.diff(cut_ptr), ref["cut_counts"])
    for f in range(cols):
        c = ref["cut_counts"][f]
        np.testing.assert_array_equal(cut_values[cut_ptr[f]:cut_ptr[f + 1]].view(np.uint32),
                                      ref["cuts"][f, :c].view(np.uint32))
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), ref["margin"].view(np.uint32))
    # Fresh CSR and dense matrices predict the same bytes.
    np.testing.assert_array_equal(bst.predict(xgb.DMatrix(_csr(indptr, indices, values, cols))).view(np.uint32),
                                  ref["margin"].view(np.uint32))
    np.testing.assert_array_equal(bst.predict(xgb.DMatrix(X)).view(np.uint32), ref["margin"].view(np.uint32))


def test_config3_logistic_matches_oracle(xgb):
    """BASELINE config 3's own workload at 50,000 rows: CSR, the full 2,000
    features with 20 nonzeros a row, its Bernoulli(sigmoid) labels and its
    parameters (binary:logistic, depth 8, 256 bins, eta 0.1), 5 rounds.
    Cuts, every tree, the training margins and the probabilities are
    bit-identical to the oracle run on the dense matrix with NaN at the
    absent entries."""
    cols = 2000
    indptr, indices, values, y = W.config3(rows=50000, cols=cols)
    X = W.csr_to_dense(indptr, indices, values, cols)
    params = dict(W.CONFIG_PARAMS[3])
    d = xgb.DMatrix(_csr(indptr, indices, values, cols), label=y)
    bst = xgb.train(params, d, 5)
    ref = O.train(X, y, _oracle_params(params), 5)
    cut_ptr, cut_values = d.get_quantile_cut()
    np.testing.assert_array_equal(np.diff(cut_ptr), ref["cut_counts"])
    for f in range(cols):
        c = ref["cut_counts"][f]
        np.testing.assert_array_equal(cut_values[cut_ptr[f]:cut_ptr[f + 1]].view(np.uint32),
                                      ref["cuts"][f, :c].view(np.uint32))
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d, output_margin=True).view(np.uint32), ref["margin"].view(np.uint32))
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), O.sigmoid(ref["margin"]).view(np.uint32))


def test_csr_logistic_weighted_equals_dense(xgb):
    """binary:logistic with sample weights, explicit NaN entries, an empty
    column, a row with every column and sampling: the CSR path grows the same
    trees, bit for bit, as the dense path on the same matrix (both on the
    device), and the dense path is pinned to the oracle elsewhere."""
    cols = 200
    indptr, indices, values, y = W.config3(rows=15000, cols=cols, nnz=12, informative=30, seed=33)
    values = values.copy()
    values[::97] = np.nan                       # explicit missing entries
    keep = indices != 7                          # column 7 has no entries at all
    counts = np.add.reduceat(keep, indptr[:-1])
    indices, values = indices[keep], values[keep]
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    # Row 0 holds every column.
    full_idx = np.arange(cols, dtype=np.int32)
    full_val = np.random.default_rng(8).lognormal(size=cols).astype(np.float32)
    indices = np.concatenate([full_idx, indices[indptr[1]:]])
    values = np.concatenate([full_val, values[indptr[1]:]])
    indptr = np.concatenate([[0], indptr[1:] - indptr[1] + cols]).astype(np.int64)
    X = W.csr_to_dense(indptr, indices, values, cols)
    w = np.random.default_rng(9).uniform(0.2, 2.0, len(y)).astype(np.float32)
    params = {"objective": "binary:logistic", "tree_method": "hist", "max_depth": 7, "max_bin": 128, "eta": 0.2,
              "subsample": 0.8, "colsample_bytree": 0.7, "seed": 5}
    ds = xgb.DMatrix(_csr(indptr, indices, values, cols), label=y, weight=w)
    dd = xgb.DMatrix(X, label=y, weight=w)
    bs = xgb.train(params, ds, 6)
    bd = xgb.train(params, dd, 6)
    assert bs.trees_to_json() == bd.trees_to_json()
    np.testing.assert_array_equal(bs.predict(ds, output_margin=True).view(np.uint32),
                                  bd.predict(dd, output_margin=True).view(np.uint32))
    np.testing.assert_array_equal(bs.predict(dd).view(np.uint32), bd.predict(ds).view(np.uint32))


def test_custom_objective_known_answer(xgb):
    """Negative Hessians and 2^40 cancellation across a depth-3 tree: leaf base
    weights [1, 3, -1, -3] (reference tests/test_histogram_present.py:66-81)."""
    X = np.repeat(np.asarray([[0, 0, np.nan], [0, 1, np.nan], [1, 0, np.nan], [1, 1, np.nan]], np.float32), 3, axis=0)
    grad = np.asarray([[2.0**40, -(2.0**40), f] for f in [-1, -3, 1, 3]], np.float32).ravel()
    hess = np.tile(np.asarray([-1, 1, 1], np.float32), 4)
    params = {"max_depth": 3, "eta": 1, "lambda": 0, "min_child_weight": 0, "max_bin": 4}
    d = xgb.DMatrix(X, label=np.zeros(len(X), np.float32))
    bst = xgb.train(params, d, 1, obj=lambda p, m: (grad, hess))
    tree = bst.trees_to_json()[0]
    assert len(tree["base_weights"]) == 7
    np.testing.assert_array_equal(np.asarray(tree["base_weights"][3:], np.float32), [1, 3, -1, -3])
    ref = O.train(X, np.zeros(len(X), np.float32), _oracle_params(dict(params, base_score=0.5)), 1,
                  custom_grad=grad[None, :], custom_hess=hess[None, :])
    assert_trees_equal(bst, ref)


def test_model_roundtrip(xgb, tmp_path):
    X, y = W.config1(rows=5000, cols=6)
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train({"max_depth": 4, "max_bin": 64}, d, 5)
    pred = bst.predict(d)
    for name in ["m.json", "m.ubj"]:
        bst.save_model(tmp_path / name)
        loaded = xgb.Booster(model_file=tmp_path / name)
        np.testing.assert_array_equal(loaded.predict(xgb.DMatrix(X)).view(np.uint32), pred.view(np.uint32))
    import pickle
    clone = pickle.loads(pickle.dumps(bst))
    np.testing.assert_array_equal(clone.predict(xgb.DMatrix(X)).view(np.uint32), pred.view(np.uint32))


def test_sklearn_estimators(xgb):
    X, y = W.config0(rows=4000, cols=5)
    reg = xgb.XGBRegressor(n_estimators=10, max_depth=4, tree_method="hist").fit(X, y)
    assert reg.score(X, y) > 0.5
    cls = xgb.XGBClassifier(n_estimators=10, max_depth=3).fit(X, (y > 0).astype(int))
    assert cls.score(X, (y > 0).astype(int)) > 0.7
    assert cls.predict_proba(X).shape == (len(X), 2)


@pytest.mark.parametrize("params", [
    {"max_depth": 6, "max_bin": 256, "subsample": 0.8},
    {"max_depth": 5, "max_bin": 64, "colsample_bytree": 0.5, "seed": 7},
    {"max_depth": 6, "max_bin": 128, "subsample": 0.6, "colsample_bytree": 0.8, "seed": 42},
])
def test_sampling_parity(xgb, params):
    """Row sampling (one engine draw per round, dropped rows carry (0, 0)) and
    per-tree column sampling give the oracle's trees and margins bit for bit."""
    X, y = W.config1(rows=30000, cols=24)
    full = dict(params, objective="reg:squarederror", tree_method="hist")
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(full, d, 8)
    ref = O.train(X, y, _oracle_params(full), 8)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), ref["margin"].view(np.uint32))


def _config4_small(rows=40000, seed=5):
    """The config-4 column recipe at a small size: N(0,1), U(0,1) and integer
    columns, labels from a logistic model of the first 16 columns."""
    rng = np.random.default_rng(seed)
    X = np.empty((rows, 32), np.float32)
    X[:, :16] = rng.normal(size=(rows, 16))
    X[:, 16:24] = rng.random((rows, 8))
    X[:, 24:] = rng.integers(0, 1000, size=(rows, 8))
    w = rng.normal(size=16).astype(np.float32)
    y = (X[:, :16] @ w + 0.3 * rng.normal(size=rows) > 0).astype(np.float32)
    return X, y


@pytest.mark.parametrize("group,shuffle", [(0, "libstdc++"), (4, "libstdc++"), (0, "libc++")])
def test_sampled_1024_bins_depth10_parity(xgb, group, shuffle):
    """1024 bins (u16 codes; 8 features per histogram workgroup by the LDS
    rule, or 4 on request), depth 10, subsample 0.8 and colsample_bytree 0.8,
    with the column sample drawn by libstdc++'s std::shuffle (the default) or
    libc++'s: bit-identical trees and margins."""
    X, y = _config4_small()
    params = {"objective": "reg:squarederror", "tree_method": "hist", "max_depth": 10, "max_bin": 1024, "eta": 0.1,
              "subsample": 0.8, "colsample_bytree": 0.8, "hip_histogram_features": group, "std_shuffle": shuffle}
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, 5)
    ref = O.train(X, y, _oracle_params(params), 5)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), ref["margin"].view(np.uint32))


@pytest.mark.parametrize("quantile", [False, True])
def test_weighted_million_root_literal(xgb, quantile):
    """The reference's literal 2915099116 (tests/test_scalar_root_statistics.py:
    66-80) from a DMatrix and a QuantileDMatrix: the root's base weight of a
    weighted 1,000,000-row depth-1 tree, and the whole tree and margins equal
    the oracle's."""
    X, y, weight = W.weighted_million()
    params = dict(W.WEIGHTED_MILLION_PARAMS)
    d = (xgb.QuantileDMatrix(X, label=y, weight=weight, max_bin=256) if quantile
         else xgb.DMatrix(X, label=y, weight=weight))
    bst = xgb.train(params, d, 1)
    root = np.float32(bst.trees_to_json()[0]["base_weights"][0])
    assert int(root.view(np.uint32)) == W.WEIGHTED_MILLION_ROOT_BITS
    ref = O.train(X, y, _oracle_params(params), 1, weights=weight)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(xgb.DMatrix(X)).view(np.uint32), ref["margin"].view(np.uint32))


@pytest.mark.parametrize("quantile", [False, True])
def test_weighted_4096_bin_root_literal(xgb, quantile):
    """The reference's literal 2990026907 (tests/test_parent_statistics.py:55-68)
    at max_bin 4096 from a DMatrix and a QuantileDMatrix: the root's base weight
    of a weighted depth-1 tree; cuts, tree and margins equal the oracle's."""
    X, y, weight = W.weighted_benchmark()
    params = dict(W.WEIGHTED_BENCHMARK_PARAMS)
    d = (xgb.QuantileDMatrix(X, label=y, weight=weight, max_bin=4096) if quantile
         else xgb.DMatrix(X, label=y, weight=weight))
    bst = xgb.train(params, d, 1)
    root = np.float32(bst.trees_to_json()[0]["base_weights"][0])
    assert int(root.view(np.uint32)) == W.WEIGHTED_BENCHMARK_ROOT_BITS
    ref = O.train(X, y, _oracle_params(params), 1, weights=weight)
    cut_ptr, cut_values = d.get_quantile_cut()
    np.testing.assert_array_equal(np.diff(cut_ptr), ref["cut_counts"])
    for f in range(X.shape[1]):
        np.testing.assert_array_equal(cut_values[cut_ptr[f]:cut_ptr[f + 1]].view(np.uint32),
                                      ref["cuts"][f, :ref["cut_counts"][f]].view(np.uint32))
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(xgb.DMatrix(X)).view(np.uint32), ref["margin"].view(np.uint32))


@pytest.mark.parametrize("max_bin,missing", [(2048, True), (4096, False), (4096, True)])
def test_large_bin_counts_match_oracle(xgb, max_bin, missing):
    """More than 1024 bins (u16 codes, one or two features per histogram
    group, 16 waves per split item): cuts, trees and margins of a depth-6
    model with and without missing values equal the oracle's."""
    X, y = W.config1(rows=30000, cols=12) if missing else W.config0(rows=30000, cols=12)
    params = {"tree_method": "hist", "max_depth": 6, "max_bin": max_bin, "eta": 0.3}
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, 3)
    ref = O.train(X, y, _oracle_params(params), 3)
    cut_ptr, _ = d.get_quantile_cut()
    np.testing.assert_array_equal(np.diff(cut_ptr), ref["cut_counts"])
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), ref["margin"].view(np.uint32))


def test_seed_per_iteration_queued_equals_stepwise_and_oracle(xgb):
    """seed_per_iteration reseeds the engine with seed * 127 + the number of
    rounds already boosted (src/learner.cpp:668), counting rounds still
    queued on the device: rounds queued without a host wait, rounds read back
    one at a time and the oracle grow the same sampled trees."""
    X, y = W.config0(rows=12000, cols=16)
    params = {"tree_method": "hist", "max_depth": 5, "max_bin": 64, "eta": 0.3, "subsample": 0.7,
              "colsample_bytree": 0.6, "seed": 5, "seed_per_iteration": 1}
    d = xgb.DMatrix(X, label=y)
    queued = xgb.train(params, d, 6)
    stepwise = xgb.Booster(params, [d])
    for i in range(6):
        stepwise.update(d, i)
        stepwise.predict(d)  # reads the model back after every round
    ref = O.train(X, y, _oracle_params(params), 6)
    assert_trees_equal(queued, ref)
    assert_trees_equal(stepwise, ref)
    np.testing.assert_array_equal(queued.predict(d).view(np.uint32), ref["margin"].view(np.uint32))
    # Reseeding matters: without it the same seed draws other samples.
    plain = O.train(X, y, _oracle_params(dict(params, seed_per_iteration=0)), 6)
    assert not np.array_equal(plain["margin"], ref["margin"])


def test_sampled_logistic_parity(xgb):
    """The config-4 objective and sampling at a small size: every tree and
    the training margins bit-identical to the oracle."""
    X, y = _config4_small()
    params = {"objective": "binary:logistic", "tree_method": "hist", "max_depth": 10, "max_bin": 1024, "eta": 0.1,
              "subsample": 0.8, "colsample_bytree": 0.8}
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, 5)
    ref = O.train(X, y, _oracle_params(params), 5)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d, output_margin=True).view(np.uint32), ref["margin"].view(np.uint32))


def test_sampling_stream_survives_pickle(xgb):
    """A pickled booster continues the engine's stream: training 3 + 3 rounds
    across a pickle equals 6 rounds in one go."""
    import pickle
    X, y = W.config0(rows=8000, cols=10)
    params = {"tree_method": "hist", "max_depth": 4, "max_bin": 64, "subsample": 0.7, "colsample_bytree": 0.6,
              "seed": 3}
    d = xgb.DMatrix(X, label=y)
    whole = xgb.train(params, d, 6)
    half = xgb.train(params, d, 3)
    half = pickle.loads(pickle.dumps(half))
    resumed = xgb.train(params, d, 3, xgb_model=half)
    np.testing.assert_array_equal(resumed.predict(d).view(np.uint32), whole.predict(d).view(np.uint32))


@pytest.mark.parametrize("layout,columns,column_levels", [("row", 1, 2), ("group", 1, 2), ("row", 0, 0),
                                                           ("group", 0, 0), ("row", 1, 16), ("row", 1, 0)])
@pytest.mark.parametrize("max_bin", [64, 1024])
def test_bin_layouts_give_identical_trees(xgb, layout, columns, column_levels, max_bin):
    """Row-major and group-major bin matrices (forced either way), with the
    row partition reading the column-major copy of the codes or the bin
    matrix itself, and histograms of the first column_levels levels read from
    the column-major copy, grow the oracle's trees, with missing values and
    u8 or u16 codes (40 features: a partial last feature group)."""
    X, y = W.config1(rows=20000, cols=40)
    params = {"tree_method": "hist", "max_depth": 6, "max_bin": max_bin, "hip_bin_layout": layout,
              "hip_partition_columns": columns, "hip_histogram_column_levels": column_levels}
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, 4)
    ref = O.train(X, y, _oracle_params(params), 4)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), ref["margin"].view(np.uint32))


@pytest.mark.parametrize("case", ["dense", "missing", "logistic", "csr", "sampled"])
def test_monotone_constraints_match_oracle(xgb, case):
    """Monotone constraints (src/tree.cpp:15-26, :1083-1086;
    kernels/boost.metal:902-920): node weight bounds, clamped weights, the
    left/right order on constrained features and the children's midpoint
    bounds give trees and training margins bit-identical to the oracle's,
    dense, with missing values, logistic, CSR and with row and column
    sampling (the oracle is pinned by the monotonicity of its predictions)."""
    mono = [1, 0, -1, 0, 0, 0, 1]
    cols = len(mono)
    rng = np.random.default_rng(17)
    if case == "csr":
        cols = 40
        mono = mono + [0] * (cols - len(mono))
        indptr, indices, values, _ = W.config3(rows=12000, cols=cols, nnz=12, informative=10, seed=5)
        X = W.csr_to_dense(indptr, indices, values, cols)
    else:
        X, _ = W.config1(rows=20000, cols=cols) if case == "missing" else W.config0(rows=20000, cols=cols)
    Z = np.nan_to_num(X)
    y = (np.sin(2 * Z[:, 0]) + Z[:, 0] - np.cos(2 * Z[:, 2]) - Z[:, 2] + Z[:, 6] + 0.3 * Z[:, 1]
         + 0.2 * rng.normal(size=len(X))).astype(np.float32)
    params = {"tree_method": "hist", "max_depth": 6, "max_bin": 64, "eta": 0.3,
              "monotone_constraints": "(" + ",".join(map(str, mono)) + ")"}
    if case == "logistic":
        params["objective"] = "binary:logistic"
        y = (y > np.median(y)).astype(np.float32)
    if case == "sampled":
        params.update(subsample=0.8, colsample_bytree=0.7, seed=9)
    d = xgb.DMatrix(_csr(indptr, indices, values, cols) if case == "csr" else X, label=y)
    bst = xgb.train(params, d, 6)
    op = _oracle_params(params)
    oracle_params = O.make_params(objective=params.get("objective", "reg:squarederror"), max_depth=6, max_bin=64,
                                  eta=float(np.float32(0.3)), subsample=op.subsample,
                                  colsample_bytree=op.colsample_bytree, seed=op.seed, monotone=mono)
    ref = O.train(X, y, oracle_params, 6)
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d, output_margin=True).view(np.uint32), ref["margin"].view(np.uint32))
    # The constraints bind: the same data trains other trees without them.
    free = xgb.train(dict(params, monotone_constraints="()"), d, 6)
    assert free.trees_to_json() != bst.trees_to_json()


def _tie_columns(rows, seed):
    """Columns whose batches hold ties the merge order decides: integer values
    (many equal values in separate runs), zeros of both signs in separate
    runs, and one with thousands of distinct values (more runs a batch)."""
    rng = np.random.default_rng(seed)
    X = np.empty((rows, 4), np.float32)
    signed_zero = np.where(rng.random(rows) < 0.5, np.float32(-0.0), np.float32(0.0))
    X[:, 0] = rng.integers(-3, 4, rows)
    X[:, 1] = np.where(rng.random(rows) < 0.5, signed_zero, rng.choice(np.float32([-1.0, 1.0]), rows))
    X[:, 2] = rng.integers(-2500, 2500, rows)
    X[:, 3] = np.where(rng.random(rows) < 0.3, signed_zero, X[:, 2])
    return X


@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("rows,max_bin", [(20000, 256), (200000, 1024)])
def test_sketch_ties_follow_std_sort(weighted, rows, max_bin):
    """Equal values in different runs are merged in the order libstdc++'s
    std::sort leaves them (the oracle's restatement, pinned by
    tests/golden/sort_ties_libstdcxx.json): which zero represents a mixed
    +0/-0 group and, with weights, the order a group's weights are added in.
    Batches of up to 8,000 runs are re-sorted in LDS, longer ones (1,024
    bins) in device memory.  Cuts bit for bit against the oracle."""
    X = _tie_columns(rows, 5)
    w = np.random.default_rng(6).uniform(0.1, 3.0, rows).astype(np.float32) if weighted else None
    cuts, counts = D.sketch_cuts(X, max_bin, w)
    ocuts, ocounts, _ = O.sketch_cuts(X, max_bin, w)
    np.testing.assert_array_equal(counts, ocounts)
    for f in range(X.shape[1]):
        np.testing.assert_array_equal(cuts[f, :counts[f]].view(np.uint32), ocuts[f, :counts[f]].view(np.uint32),
                                      err_msg=f"feature {f}")


def test_sketch_ties_train_like_oracle(xgb):
    """The tie columns through training: weighted regression, depth 6, cuts,
    trees and margins equal the oracle's."""
    X = _tie_columns(30000, 8)
    rng = np.random.default_rng(9)
    y = (X[:, 0] + 0.001 * X[:, 2] + np.signbit(X[:, 1]) + 0.1 * rng.normal(size=len(X))).astype(np.float32)
    w = rng.uniform(0.1, 3.0, len(X)).astype(np.float32)
    params = {"objective": "reg:squarederror", "tree_method": "hist", "max_depth": 6, "max_bin": 64}
    d = xgb.DMatrix(X, label=y, weight=w)
    bst = xgb.train(params, d, 4)
    ref = O.train(X, y, _oracle_params(params), 4, weights=w)
    cut_ptr, cut_values = d.get_quantile_cut()
    np.testing.assert_array_equal(np.diff(cut_ptr), ref["cut_counts"])
    for f in range(X.shape[1]):
        np.testing.assert_array_equal(cut_values[cut_ptr[f]:cut_ptr[f + 1]].view(np.uint32),
                                      ref["cuts"][f, :ref["cut_counts"][f]].view(np.uint32))
    assert_trees_equal(bst, ref)
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), ref["margin"].view(np.uint32))
