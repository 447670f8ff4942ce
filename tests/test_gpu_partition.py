"""The row partition (reference kernels/boost.metal:1316-1614, stable variant
:1550-1614).  With shape.stable_partition each child keeps its parent's row
order: from the root's rows [0, N) in order, every node's segment of a
level's row list is ascending, so the list has at most one ascending run per
node.  With tiles claiming their ranges by atomics the order inside a child
follows arrival; the trees, leaves and margins are the same either way
(histograms are exact integer sums), through the C ABI and through training
on dense, missing-value, CSR and subsampled matrices."""
import ctypes
import json

import numpy as np
import pytest

import device_lib as D
import workloads as W
from test_zz_no_alloc import NODE_BYTES, MASS_WORDS, MgbGradParams, MgbSplitParams

pytestmark = pytest.mark.gpu


def _problem(rows, cols, max_bin, depth, weighted, seed):
    X, y = W.config0(rows=rows, cols=cols, seed=seed)
    cuts, counts = D.sketch_cuts(X, max_bin)
    m, dbins, _, _ = D.quantize_bins(X, cuts, counts, max_bin, 1, 4, dense=True)
    w = np.random.default_rng(seed + 1).uniform(0.5, 2.0, rows).astype(np.float32) if weighted else None
    keep = [D.Device(rows * 4), D.Device.of(y), D.Device.of(w) if weighted else None, D.Device(MASS_WORDS * 8)]
    grad, scales = D.Device(rows * 8), D.Device(8)
    gp = MgbGradParams(rows, 0, 1 if weighted else 0, 0, 1.0, 1.0, 0.0, 0.0)
    D.check(D.lib().mgb_gradients(ctypes.byref(gp), keep[0].ptr, keep[1].ptr, keep[2].ptr if keep[2] else None,
                                  grad.ptr, keep[3].ptr, scales.ptr))
    return dict(m=m, bins=dbins, cuts=D.Device.of(np.ascontiguousarray(cuts, np.float32)),
                counts=D.Device.of(np.ascontiguousarray(counts, np.uint32)), grad=grad, scales=scales, keep=keep,
                rows=rows, cols=cols, max_bin=max_bin, depth=depth, weighted=weighted)


def _grow(p, stable, rows_per_tile=2048):
    shape = D.MgbTreeShape(p["rows"], p["cols"], p["max_bin"], p["depth"], rows_per_tile, 4,
                           0 if p["weighted"] else 1, 1, 0, 0, 0, 0, 1 if stable else 0)
    sp = MgbSplitParams(1.0, 0.0, 1.0, 0.0, 0.0, 0.3, p["depth"], 1)
    max_nodes = (2 << p["depth"]) - 1
    nodes, count, margin = D.Device(max_nodes * NODE_BYTES), D.Device(8), D.Device(p["rows"] * 4)
    ws_bytes = D.lib().mgb_tree_workspace_bytes(ctypes.byref(shape))
    ws = D.Device(ws_bytes)
    D.check(D.lib().mgb_grow_tree(ctypes.byref(shape), ctypes.byref(p["m"]), p["bins"].ptr, None, p["cuts"].ptr,
                                  p["counts"].ptr, p["grad"].ptr, p["scales"].ptr, ctypes.byref(sp), None, None,
                                  ws.ptr, ctypes.c_size_t(ws_bytes), margin.ptr, nodes.ptr, count.ptr))
    D.check(D.lib().mgb_synchronize())
    n = int(count.read(np.uint32, 1)[0])
    records = nodes.read(np.int32, n * NODE_BYTES // 4).reshape(n, NODE_BYTES // 4)
    last = np.zeros(p["rows"], np.uint32)
    D.check(D.lib().mgb_tree_row_list(ctypes.byref(shape), ws.ptr, ctypes.c_uint32(p["depth"] - 1),
                                      last.ctypes.data_as(ctypes.c_void_p)))
    return records, margin.read(np.uint32, p["rows"]), last


def _runs(v):
    return 1 + int(np.count_nonzero(np.diff(v.astype(np.int64)) < 0))


def _splits_to_last_level(records, depth):
    """Every node above the last level splits (so the last level's row list
    holds every row, none left behind by an early leaf)."""
    level, frontier = 0, [0]
    while level < depth - 1:
        nxt = []
        for i in frontier:
            if records[i, 0] < 0:
                return False
            nxt += [int(records[i, 0]), int(records[i, 1])]
        frontier, level = nxt, level + 1
    return True


@pytest.mark.parametrize("rows,depth,weighted,tile", [(40000, 5, False, 2048), (40000, 6, True, 2048),
                                                      (5000, 4, False, 64), (131072, 7, False, 4096)])
def test_stable_partition_keeps_row_order(rows, depth, weighted, tile):
    p = _problem(rows, 12, 64, depth, weighted, seed=rows + depth)
    rec_s, margin_s, last_s = _grow(p, stable=True, rows_per_tile=tile)
    rec_a, margin_a, last_a = _grow(p, stable=False, rows_per_tile=tile)
    np.testing.assert_array_equal(rec_s, rec_a)
    np.testing.assert_array_equal(margin_s, margin_a)
    assert _splits_to_last_level(rec_s, depth)
    for last in (last_s, last_a):
        np.testing.assert_array_equal(np.sort(last), np.arange(rows, dtype=np.uint32))
    # One ascending run per node of the last level at most.
    assert _runs(last_s) <= 2 ** (depth - 1)
    # The same list twice: the stable order is a function of the tree alone.
    assert np.array_equal(_grow(p, stable=True, rows_per_tile=tile)[2], last_s)


def _trees(bst):
    return json.loads(bst.save_raw("json"))["learner"]["gradient_booster"]["model"]["trees"]


def _same_with_both_partitions(xgb, dtrain, params, rounds):
    stable = xgb.train(dict(params, hip_stable_partition=1), dtrain, rounds)
    claims = xgb.train(dict(params, hip_stable_partition=0), dtrain, rounds)
    assert _trees(stable) == _trees(claims)
    np.testing.assert_array_equal(stable.predict(dtrain, output_margin=True).view(np.uint32),
                                  claims.predict(dtrain, output_margin=True).view(np.uint32))


@pytest.mark.parametrize("rows,depth", [(3000, 1), (3000, 2), (9000, 2), (20000, 3)])
def test_partition_modes_small_grids(xgb, rows, depth):
    """Shallow trees on few rows: the last level's partition grid has fewer
    than 8 workgroups (or just 8 and more), so the stable partition's margin
    updates run in task order or by row range; both modes give the same
    trees and bit-identical margins."""
    X, y = W.config1(rows=rows, cols=12)
    _same_with_both_partitions(xgb, xgb.DMatrix(X, label=y), {"max_depth": depth, "max_bin": 64}, 3)


def test_partition_modes_train_identical_models(xgb):
    X, y = W.config1(rows=30000, cols=16)
    _same_with_both_partitions(xgb, xgb.DMatrix(X, label=y), {"max_depth": 7, "max_bin": 128}, 5)
    X, y = W.config0(rows=20000, cols=10)
    yb = (y > np.median(y)).astype(np.float32)
    _same_with_both_partitions(xgb, xgb.DMatrix(X, label=yb),
                               {"max_depth": 6, "max_bin": 64, "objective": "binary:logistic", "subsample": 0.7,
                                "colsample_bytree": 0.8, "seed": 5}, 5)
    indptr, indices, values, yc = W.config3(rows=20000, cols=300, nnz=12, informative=40)
    import scipy.sparse as sps
    csr = sps.csr_matrix((values, indices, indptr), shape=(20000, 300))
    _same_with_both_partitions(xgb, xgb.DMatrix(csr, label=yc),
                               {"max_depth": 6, "max_bin": 64, "objective": "binary:logistic", "eta": 0.1}, 4)
