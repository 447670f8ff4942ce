"""The C-ABI library builds, loads without a GPU, and exports every entry
point declared in include/*.h; the Python package imports over it."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "xgboost-metal_amd" / "python" / "xgboost" / "lib" / "libxgboost.so"


def declared_functions(header):
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:XGB_DLL\s+)?(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s+\**([A-Za-z_][A-Za-z0-9_]*)\s*\(",
                       text, flags=re.M)
    return sorted(set(n for n in names if n not in ("if", "return")))


@pytest.mark.parametrize("header", sorted((ROOT / "include").glob("*.h")), ids=lambda p: p.name)
def test_exports_every_declared_symbol(header):
    lib = ctypes.CDLL(str(LIB))
    names = declared_functions(header)
    assert len(names) > 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"{header.name}: not exported: {missing}"


def test_version_and_error_without_gpu():
    lib = ctypes.CDLL(str(LIB))
    major, minor, patch = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    lib.XGBoostVersion(ctypes.byref(major), ctypes.byref(minor), ctypes.byref(patch))
    assert (major.value, minor.value, patch.value) == (3, 5, 0)
    lib.XGBGetLastError.restype = ctypes.c_char_p
    # A null handle is rejected with a message, not a crash.
    out = ctypes.c_uint64()
    assert lib.XGDMatrixNumRow(None, ctypes.byref(out)) == -1
    assert b"null" in lib.XGBGetLastError()


def test_package_imports(xgb):
    assert xgb.__version__ == "3.5.0-dev"
    info = xgb.build_info()
    assert info["USE_HIP"] is True and info["HIP_ARCH"] == "gfx950"


def test_dmatrix_host_side(xgb):
    import numpy as np
    X = np.arange(12, dtype=np.float32).reshape(4, 3)
    X[1, 2] = -999
    d = xgb.DMatrix(X, label=[1, 2, 3, 4], missing=-999, feature_names=["a", "b", "c"])
    assert d.num_row() == 4 and d.num_col() == 3 and d.num_nonmissing() == 11
    np.testing.assert_array_equal(d.get_label(), [1, 2, 3, 4])
    assert d.feature_names == ["a", "b", "c"]
    import scipy.sparse as sp
    csr = sp.csr_matrix(np.asarray([[0, 1.5], [2.0, 0]], np.float32))
    d2 = xgb.DMatrix(csr)
    assert d2.num_row() == 2 and d2.num_col() == 2 and d2.num_nonmissing() == 2


def test_csr_ingest_sorts_rows_and_rejects_repeats(xgb):
    """CSR rows arrive in any column order (sorted on ingest); a stored entry
    equal to `missing` is missing; a repeated column in a row is an error."""
    import numpy as np
    import scipy.sparse as sp
    indptr = np.array([0, 3, 5, 5])
    indices = np.array([2, 0, 1, 1, 0])
    data = np.array([1.0, 2.0, -1.0, 4.0, 5.0], np.float32)
    d = xgb.DMatrix(sp.csr_matrix((data, indices, indptr), shape=(3, 3)), missing=-1.0)
    assert d.num_row() == 3 and d.num_col() == 3 and d.num_nonmissing() == 4
    dup = sp.csr_matrix((np.ones(3, np.float32), np.array([1, 0, 1]), np.array([0, 3])), shape=(1, 3))
    with pytest.raises(xgb.XGBoostError, match="repeats a column"):
        xgb.DMatrix(dup)


def test_unsupported_parameters_fail_loudly(xgb):
    import numpy as np
    b = xgb.Booster({"tree_method": "exact"})
    d = xgb.DMatrix(np.zeros((4, 2), np.float32), label=np.zeros(4))
    with pytest.raises(xgb.XGBoostError, match="hist"):
        b.update(d, 0)


NODE = [("left", "<i4"), ("right", "<i4"), ("parent", "<i4"), ("feature", "<i4"), ("threshold", "<f4"),
        ("leaf", "<f4"), ("cover", "<f4"), ("gain", "<f4"), ("default_left", "<u4"), ("base_weight", "<f4")]


def _validate(nodes, status=0, max_nodes=15, cols=4, count=None):
    import numpy as np
    lib = ctypes.CDLL(str(LIB))
    lib.mgb_last_error.restype = ctypes.c_char_p
    nodes = np.ascontiguousarray(nodes)
    rc = lib.mgb_validate_tree(nodes.ctypes.data_as(ctypes.c_void_p), ctypes.c_uint32(len(nodes) if count is None else count),
                               ctypes.c_uint32(status), ctypes.c_uint32(max_nodes), ctypes.c_uint32(cols))
    return rc, lib.mgb_last_error().decode()


def _depth2_tree():
    """Root splits (children 1, 2); node 1 splits (children 3, 4); node 2 is a
    leaf: the node-id order the tree driver emits."""
    import numpy as np
    t = np.zeros(5, dtype=np.dtype(NODE))
    t["left"], t["right"], t["feature"] = -1, -1, -1
    t["parent"] = [-1, 0, 0, 1, 1]
    t[0]["left"], t[0]["right"], t[0]["feature"] = 1, 2, 3
    t[1]["left"], t[1]["right"], t[1]["feature"] = 3, 4, 0
    return t


def _put(t, i, field, value):
    t[field][i] = value


def test_validate_tree_accepts_driver_order():
    assert _validate(_depth2_tree())[0] == 0


@pytest.mark.parametrize("corrupt,message", [
    (lambda t: _put(t, 1, "left", 5), "not the next unused ids"),
    (lambda t: _put(t, 3, "parent", 0), "do not name it as their parent"),
    (lambda t: _put(t, 0, "feature", 4), "splits on feature 4 of 4"),
    (lambda t: _put(t, 2, "feature", 1), "is a leaf with split feature"),
    (lambda t: _put(t, 2, "left", 5), "has one child"),
    (lambda t: _put(t, 0, "parent", 3), "node 0 is not a root"),
    (lambda t: _put(t, 4, "default_left", 7), "default_left 7"),
])
def test_validate_tree_rejects_corrupt_records(corrupt, message):
    """The checks the learner runs on every queued round's records before it
    publishes the tree (a refused round raises XGBoostError naming it)."""
    t = _depth2_tree()
    corrupt(t)
    rc, err = _validate(t)
    assert rc == -1 and message in err


def test_validate_tree_rejects_counts_and_status():
    t = _depth2_tree()
    rc, err = _validate(t, count=4)  # node 1's children end beyond the count
    assert rc == -1 and "beyond the node count" in err
    rc, err = _validate(t, max_nodes=3)
    assert rc == -1 and "outside [1, 3]" in err
    rc, err = _validate(t, status=2)
    assert rc == -1 and "status 0x2" in err and "capacity" in err
    rc, err = _validate(t, status=0x18)
    assert rc == -1 and "more rows than its parent" in err and "unknown bits" in err


@pytest.mark.parametrize("quantile", [False, True])
@pytest.mark.parametrize("params", [
    {"max_depth": 2, "max_bin": 32, "base_score": 0, "seed": 41},
    {"max_depth": 10, "max_bin": 32, "seed": 41},
    {"max_depth": 6, "max_bin": 64, "objective": "binary:logistic"},
])
def test_empty_matrix_training_matches_oracle(xgb, quantile, params):
    """Training on a matrix without rows (the reference's 'empty' engine case,
    tests/test_gpu_tree.py:51-52) needs no device work: every feature's cuts
    are the empty summary's sentinel 1e-5, the base score is the weighted
    mean of no labels (0 for squared error, 0.5 for logistic) unless given,
    and every round's tree is one leaf of weight 0 -- as the oracle trains
    it.  Prediction on the empty matrix is empty."""
    import numpy as np
    import oracle_lib as O
    from test_gpu_parity import _oracle_params, assert_trees_equal
    X, y = np.zeros((0, 7), np.float32), np.zeros(0, np.float32)
    params = dict(params, tree_method="hist")
    d = xgb.QuantileDMatrix(X, label=y, max_bin=params["max_bin"]) if quantile else xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, 3)
    ref = O.train(X, y, _oracle_params(params), 3)
    assert_trees_equal(bst, ref)
    cut_ptr, cut_values = d.get_quantile_cut()
    np.testing.assert_array_equal(np.diff(cut_ptr), ref["cut_counts"])
    np.testing.assert_array_equal(cut_values, np.full(7, 1e-5, np.float32))
    assert bst.predict(d).shape == (0,)
    import json
    stored = json.loads(bst.save_raw("json"))["learner"]["learner_model_param"]["base_score"]
    assert np.float32(float(stored.strip("[]"))) == np.float32(ref["base_score"])


def test_device_tie_sort_follows_libstdcxx():
    """The sketch kernel's tie sort (run on the host through its test hook,
    the same code the device runs for a batch with ties the merge order
    decides) leaves every case of tests/golden/sort_ties_libstdcxx.json in
    the order this image's libstdc++ std::sort does.  Class k becomes the
    order key of the non-negative binary32 value whose bits are k, so the
    values increase with the class (up to 2^30 classes)."""
    import json
    import numpy as np
    from test_oracle import _sort_fixture_keys
    lib = ctypes.CDLL(str(LIB))
    fixture = json.loads((ROOT / "tests" / "golden" / "sort_ties_libstdcxx.json").read_text())
    for case in fixture["cases"]:
        n = case["n"]
        cls = _sort_fixture_keys(case["pattern"], n, case["k"], case["seed"]).astype(np.uint32)
        keys = (cls | np.uint32(0x80000000)).astype(np.uint32)  # order keys of increasing non-negative values
        order = np.zeros(max(n, 1), np.uint32)
        assert lib.mgb_tie_sort_order(keys.ctypes.data_as(ctypes.c_void_p), ctypes.c_uint32(n),
                                      order.ctypes.data_as(ctypes.c_void_p)) == 0
        order = order[:n].astype(np.uint64)
        checksum = int((order * (2 * np.arange(n, dtype=np.uint64) + 1)).sum(dtype=np.uint64))
        assert checksum == case["checksum"], case
        assert order[:len(case["order"])].tolist() == case["order"], case


@pytest.mark.parametrize("sparse", [False, True])
def test_grow_tree_rejects_rows_from_two_to_the_31(sparse):
    """Both tree drivers refuse 2^31 rows or more before any device work (row
    positions in the kernels are 32-bit and run past a task's end); the check
    is host-side, so it runs without a GPU."""
    import device_lib as D
    lib = D.lib()
    shape = D.MgbTreeShape(rows=1 << 31, cols=4, max_bin=16, max_depth=3, rows_per_tile=1024,
                           features_per_group=4, sparse=1 if sparse else 0)
    if sparse:
        class Csr(ctypes.Structure):
            _fields_ = [("rows", ctypes.c_uint32), ("cols", ctypes.c_uint32), ("max_bin", ctypes.c_uint32),
                        ("cut_stride", ctypes.c_uint32), ("bin_bytes", ctypes.c_uint32),
                        ("missing_code", ctypes.c_uint32), ("nnz", ctypes.c_uint64)]
        m = Csr(rows=1 << 31, cols=4, max_bin=16, cut_stride=16, bin_bytes=1, missing_code=255, nnz=0)
        rc = lib.mgb_grow_tree_csr(ctypes.byref(shape), ctypes.byref(m), *([None] * 18))
    else:
        m = D.MgbMatrix(rows=1 << 31, cols=4, row_stride=4, bin_bytes=1, max_bin=16, cut_stride=16,
                        missing_code=255, group_features=4, group_stride=4)
        rc = lib.mgb_grow_tree(ctypes.byref(shape), ctypes.byref(m), *([None] * 14))
    assert rc == -1
    assert "below 2^31" in lib.mgb_last_error().decode()


def test_explain_entry_points_validate_on_the_host():
    """The leaf and contribution entry points refuse null buffers and trees
    deeper than exact TreeSHAP's limit before any device work, and return at
    once for an empty matrix (no GPU needed)."""
    import device_lib as D
    lib = D.lib()
    one = ctypes.c_uint32(1)
    assert lib.mgb_predict_leaf(None, None, None, ctypes.c_uint32(0), one, None, None, one, None) == 0
    assert lib.mgb_predict_leaf(None, None, None, one, one, None, None, one, None) == -1
    assert "null argument" in lib.mgb_last_error().decode()
    buf = ctypes.create_string_buffer(64)
    args = [buf, None, None, one, one, buf, buf, buf, one, ctypes.c_uint32(17), ctypes.c_uint32(0),
            ctypes.c_uint32(0), None, ctypes.c_float(0.0), buf]
    assert lib.mgb_predict_contribs(*args) == -1
    assert "depth at most 16" in lib.mgb_last_error().decode()
    args[1] = buf  # CSR offsets without column ids
    args[10] = ctypes.c_uint32(1)
    assert lib.mgb_predict_contribs(*args) == -1
    assert "null argument" in lib.mgb_last_error().decode()
