"""mgb_grow_tree_noalloc (the allocation-free tree entry point) against
mgb_grow_tree with a caller-allocated workspace, through the C ABI: two
calls in a row, the second on a smaller input (fewer rows and features,
fewer bins, shallower, unit Hessians after a weighted first call), give
bit-identical node records, node counts and margins; shapes above the static
scratch and calls under per-kernel timing are refused before any device
work."""
import ctypes

import numpy as np
import pytest

import device_lib as D
import workloads as W

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20
NODE_BYTES = 40  # MgbTreeNode: 10 x 4 bytes


class MgbGradParams(ctypes.Structure):
    _fields_ = [("rows", ctypes.c_uint32), ("objective", ctypes.c_uint32), ("has_weight", ctypes.c_uint32),
                ("sample_seed", ctypes.c_uint32), ("scale_pos_weight", ctypes.c_float), ("subsample", ctypes.c_float),
                ("padding1", ctypes.c_float), ("padding2", ctypes.c_float)]


class MgbSplitParams(ctypes.Structure):
    _fields_ = [("reg_lambda", ctypes.c_float), ("reg_alpha", ctypes.c_float), ("min_child_weight", ctypes.c_float),
                ("max_delta_step", ctypes.c_float), ("min_split_loss", ctypes.c_float), ("eta", ctypes.c_float),
                ("max_depth", ctypes.c_uint32), ("fma_contract", ctypes.c_uint32), ("inject_status", ctypes.c_uint32),
                ("padding", ctypes.c_uint32)]


MASS_WORDS = 5640  # MGB_MASS_WORDS


def _problem(rows, cols, max_bin, depth, G, weighted, seed):
    X, y = W.config0(rows=rows, cols=cols, seed=seed)
    cuts, counts = D.sketch_cuts(X, max_bin)
    m, dbins, _, any_missing = D.quantize_bins(X, cuts, counts, max_bin, 1, G, dense=True)
    assert not any_missing
    w = np.random.default_rng(seed + 1).uniform(0.5, 2.0, rows).astype(np.float32) if weighted else None
    d_margin0 = D.Device(rows * 4)
    d_labels = D.Device.of(y)
    d_w = D.Device.of(w) if weighted else None
    d_grad = D.Device(rows * 8)
    d_mass = D.Device(MASS_WORDS * 8)
    d_scales = D.Device(8)
    gp = MgbGradParams(rows, 0, 1 if weighted else 0, 0, 1.0, 1.0, 0.0, 0.0)
    D.check(D.lib().mgb_gradients(ctypes.byref(gp), d_margin0.ptr, d_labels.ptr, d_w.ptr if d_w else None,
                                  d_grad.ptr, d_mass.ptr, d_scales.ptr))
    shape = D.MgbTreeShape(rows, cols, max_bin, depth, 2048, G, 0 if weighted else 1, 1, 0, 0, 0, 0)
    sp = MgbSplitParams(1.0, 0.0, 1.0, 0.0, 0.0, 0.3, depth, 1)
    return dict(shape=shape, m=m, bins=dbins, cuts=D.Device.of(np.ascontiguousarray(cuts, np.float32)),
                counts=D.Device.of(np.ascontiguousarray(counts, np.uint32)), grad=d_grad, scales=d_scales, sp=sp,
                keep=(d_margin0, d_labels, d_w, d_mass), rows=rows, depth=depth)


def _grow(p, noalloc):
    max_nodes = (2 << p["depth"]) - 1
    nodes = D.Device(max_nodes * NODE_BYTES)
    count = D.Device(8)  # node count, tree status
    margin = D.Device(p["rows"] * 4)
    args_head = (ctypes.byref(p["shape"]), ctypes.byref(p["m"]), p["bins"].ptr, None, p["cuts"].ptr,
                 p["counts"].ptr, p["grad"].ptr, p["scales"].ptr, ctypes.byref(p["sp"]), None, None)
    if noalloc:
        D.check(D.lib().mgb_grow_tree_noalloc(*args_head, margin.ptr, nodes.ptr, count.ptr))
    else:
        ws_bytes = D.lib().mgb_tree_workspace_bytes(ctypes.byref(p["shape"]))
        ws = D.Device(ws_bytes)
        D.check(D.lib().mgb_grow_tree(*args_head, ws.ptr, ctypes.c_size_t(ws_bytes), margin.ptr, nodes.ptr,
                                      count.ptr))
    D.check(D.lib().mgb_synchronize())
    n = int(count.read(np.uint32, 1)[0])
    assert 1 <= n <= max_nodes
    return n, nodes.read(np.uint8, n * NODE_BYTES), margin.read(np.uint32, p["rows"])


def _assert_same(p):
    want = _grow(p, noalloc=False)
    got = _grow(p, noalloc=True)
    assert got[0] == want[0]
    np.testing.assert_array_equal(got[1], want[1])
    np.testing.assert_array_equal(got[2], want[2])
    return want[0]


def test_noalloc_equals_workspace_entry_point_twice():
    first = _problem(rows=30000, cols=16, max_bin=64, depth=6, G=4, weighted=True, seed=11)
    assert D.lib().mgb_tree_workspace_bytes(ctypes.byref(first["shape"])) <= SCRATCH_BYTES
    assert _assert_same(first) > 31  # a real tree, not a stump
    second = _problem(rows=9000, cols=12, max_bin=32, depth=4, G=4, weighted=False, seed=12)
    assert _assert_same(second) > 7


def test_noalloc_refuses_large_shape_and_timing():
    L = D.lib()
    # A config-2 shape needs a 115 MiB workspace: refused on the host (checked
    # here first, so no kernel is ever launched with these null pointers).
    big = D.MgbTreeShape(262144, 64, 256, 8, 4096, 8, 1, 1, 0, 0, 0, 0)
    assert L.mgb_tree_workspace_bytes(ctypes.byref(big)) > SCRATCH_BYTES
    m = D.MgbMatrix(262144, 64, 64, 1, 256, 256, 0xFFFFFFFF, 8, 8)
    sp = MgbSplitParams(1.0, 0.0, 1.0, 0.0, 0.0, 0.3, 8, 1)
    rc = L.mgb_grow_tree_noalloc(ctypes.byref(big), ctypes.byref(m), None, None, None, None, None, None,
                                 ctypes.byref(sp), None, None, None, None, None)
    assert rc == -1
    assert b"allocation-free scratch" in L.mgb_last_error()
    # Per-kernel timing creates events: refused while it is on.
    p = _problem(rows=4000, cols=8, max_bin=16, depth=3, G=4, weighted=False, seed=13)
    D.check(L.mgb_profile_enable(1))
    try:
        rc = L.mgb_grow_tree_noalloc(ctypes.byref(p["shape"]), ctypes.byref(p["m"]), p["bins"].ptr, None,
                                     p["cuts"].ptr, p["counts"].ptr, p["grad"].ptr, p["scales"].ptr,
                                     ctypes.byref(p["sp"]), None, None, D.Device(4000 * 4).ptr,
                                     D.Device(15 * NODE_BYTES).ptr, D.Device(8).ptr)
    finally:
        D.check(L.mgb_profile_enable(0))
    assert rc == -1
    assert b"timing" in L.mgb_last_error()
