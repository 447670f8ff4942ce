"""Host-side C API and Python surface beyond training (no GPU needed):
iterator-fed matrices, CSC/COO input, row slices, model dumps, feature
importance, model slicing and the entry points this engine rejects.

The C entry points follow the reference's src/c_api.cpp (file:line in each
test); the dump formats follow src/model.cpp:334-428."""
import ctypes
import json
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "xgboost-metal_amd" / "python" / "xgboost" / "lib" / "libxgboost.so"


def test_exports_every_entry_point_the_reference_package_binds():
    """All names the reference's Python package calls through `_LIB`
    (fixture written by tests/golden/make_c_api_symbols.py)."""
    names = (ROOT / "tests" / "golden" / "reference_c_api_symbols.txt").read_text().split()
    assert len(names) >= 90
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing


def _iter_class(xgb):
    class Batches(xgb.DataIter):
        def __init__(self, parts, **kwargs):
            self.parts = parts
            self.i = 0
            super().__init__(**kwargs)

        def next(self, input_data):
            if self.i == len(self.parts):
                return False
            input_data(**self.parts[self.i])
            self.i += 1
            return True

        def reset(self):
            self.i = 0

    return Batches


def _data(rows=120, cols=6, seed=0):
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(rows, cols)).astype(np.float32)
    X[rng.random(X.shape) < 0.2] = np.nan
    y = rng.normal(size=rows).astype(np.float32)
    w = rng.uniform(0.5, 2, size=rows).astype(np.float32)
    return X, y, w


def _dense_of(d):
    csr = d.get_data()
    out = np.full(csr.shape, np.nan, np.float32)
    for r in range(csr.shape[0]):
        lo, hi = csr.indptr[r], csr.indptr[r + 1]
        out[r, csr.indices[lo:hi]] = csr.data[lo:hi]
    return out


def test_iterator_batches_concatenate_in_order(xgb):
    """XGDMatrixCreateFromCallback (src/c_api.cpp:222): the batches in order,
    their labels and weights with them; dense and CSR batches mix."""
    import scipy.sparse as sp
    X, y, w = _data()
    Batches = _iter_class(xgb)
    parts = [dict(data=X[:50], label=y[:50], weight=w[:50]), dict(data=X[50:90], label=y[50:90], weight=w[50:90]),
             dict(data=X[90:], label=y[90:], weight=w[90:])]
    d = xgb.DMatrix(Batches(parts))
    assert d.num_row() == 120 and d.num_col() == 6
    np.testing.assert_array_equal(d.get_label(), y)
    np.testing.assert_array_equal(d.get_weight(), w)
    np.testing.assert_array_equal(_dense_of(d), X)
    assert d.num_nonmissing() == int(np.isfinite(X).sum())
    # A CSR batch: absent entries are missing, like NaN in a dense batch.
    Xz = np.where(np.isnan(X), 0, X)
    first = sp.csr_matrix(Xz[:50])
    mixed = xgb.DMatrix(Batches([dict(data=first, label=y[:50]), dict(data=X[50:], label=y[50:])]))
    expect = X.copy()
    expect[:50][Xz[:50] == 0] = np.nan
    np.testing.assert_array_equal(_dense_of(mixed), expect)


def test_iterator_errors(xgb):
    """Exceptions in the callbacks surface after the C call; external memory
    and meta info on only some batches are rejected."""
    X, y, _ = _data(40)
    Batches = _iter_class(xgb)

    class Failing(Batches):
        def next(self, input_data):
            raise RuntimeError("batch source failed")

    with pytest.raises(RuntimeError, match="batch source failed"):
        xgb.DMatrix(Failing([]))
    with pytest.raises(xgb.XGBoostError, match="cache_prefix"):
        xgb.DMatrix(Batches([dict(data=X)], cache_prefix="/tmp/cache"))
    with pytest.raises(xgb.XGBoostError, match="others do not"):
        xgb.DMatrix(Batches([dict(data=X[:20], label=y[:20]), dict(data=X[20:])]))
    with pytest.raises(xgb.XGBoostError, match="differ in their number of features"):
        xgb.DMatrix(Batches([dict(data=X[:20]), dict(data=X[20:, :3])]))


def test_quantile_iterator_and_ref(xgb):
    """XGQuantileDMatrixCreateFromCallback (src/c_api.cpp:225-239): batches,
    max_bin and a reference matrix."""
    X, y, _ = _data(80)
    Batches = _iter_class(xgb)
    q = xgb.QuantileDMatrix(Batches([dict(data=X[:30], label=y[:30]), dict(data=X[30:], label=y[30:])]), max_bin=32)
    assert q.num_row() == 80 and q.max_bin == 32
    np.testing.assert_array_equal(q.get_label(), y)
    ev = xgb.QuantileDMatrix(X[:10], y[:10], ref=q, max_bin=32)
    assert ev.num_row() == 10
    np.testing.assert_array_equal(ev.get_label(), y[:10])
    with pytest.raises(xgb.XGBoostError, match="max_bin"):
        xgb.QuantileDMatrix(Batches([dict(data=X)]), max_bin=1)


def _raw_interface(a):
    return json.dumps({"data": [a.ctypes.data, True], "shape": list(a.shape), "typestr": a.dtype.str,
                       "version": 3}).encode()


def test_csc_and_coo_equal_csr(xgb):
    """XGDMatrixCreateFromCSC / FromCOO (src/c_api.cpp:201-206) hold the same
    entries as the CSR of the same matrix."""
    import scipy.sparse as sp
    rng = np.random.default_rng(3)
    dense = rng.normal(size=(30, 7)).astype(np.float32)
    dense[rng.random(dense.shape) < 0.6] = 0
    csr = sp.csr_matrix(dense)
    ref = _dense_of(xgb.DMatrix(csr))
    lib = xgb.core._LIB
    csc = sp.csc_matrix(dense)
    cp, ri, dv = (np.ascontiguousarray(csc.indptr, np.int64), np.ascontiguousarray(csc.indices, np.int32),
                  np.ascontiguousarray(csc.data, np.float32))
    h = ctypes.c_void_p()
    assert lib.XGDMatrixCreateFromCSC(_raw_interface(cp), _raw_interface(ri), _raw_interface(dv),
                                      ctypes.c_uint64(30), b'{"missing": NaN}', ctypes.byref(h)) == 0
    np.testing.assert_array_equal(_dense_of(xgb.DMatrix(h)), ref)
    coo = sp.coo_matrix(dense)
    perm = rng.permutation(coo.nnz)  # any entry order
    r, c, v = (np.ascontiguousarray(coo.row[perm], np.int32), np.ascontiguousarray(coo.col[perm], np.int32),
               np.ascontiguousarray(coo.data[perm], np.float32))
    h2 = ctypes.c_void_p()
    assert lib.XGDMatrixCreateFromCOO(_raw_interface(r), _raw_interface(c), _raw_interface(v), ctypes.c_uint64(30),
                                      ctypes.c_uint64(7), b"{}", ctypes.byref(h2)) == 0
    np.testing.assert_array_equal(_dense_of(xgb.DMatrix(h2)), ref)


def test_slice_keeps_rows_and_meta(xgb):
    """XGDMatrixSliceDMatrixEx (src/c_api.cpp:294, src/data.cpp:1451)."""
    import scipy.sparse as sp
    X, y, w = _data(50)
    margin = np.arange(50, dtype=np.float32)
    idx = [7, 3, 3, 49, 0]
    for data in (X, sp.csr_matrix(np.nan_to_num(X))):
        d = xgb.DMatrix(data, label=y, weight=w, base_margin=margin, feature_names=[f"c{i}" for i in range(6)])
        s = d.slice(idx)
        assert s.num_row() == 5 and s.num_col() == 6
        np.testing.assert_array_equal(s.get_label(), y[idx])
        np.testing.assert_array_equal(s.get_weight(), w[idx])
        np.testing.assert_array_equal(s.get_base_margin(), margin[idx])
        np.testing.assert_array_equal(_dense_of(s), _dense_of(d)[idx])
        assert s.feature_names == d.feature_names
    with pytest.raises(xgb.XGBoostError, match="out of range"):
        xgb.DMatrix(X).slice([50])


# A hand-written two-feature model in XGBoost's JSON model format.
def _tree(left, right, parent, feature, cond, gain, cover, default_left):
    n = len(left)
    return {"left_children": left, "right_children": right, "parents": parent, "split_indices": feature,
            "split_conditions": cond, "loss_changes": gain, "sum_hessian": cover, "base_weights": [0.0] * n,
            "default_left": default_left, "split_type": [0] * n, "categories": [], "categories_nodes": [],
            "categories_segments": [], "categories_sizes": [], "id": 0,
            "tree_param": {"num_nodes": str(n), "num_deleted": "0", "num_feature": "3", "size_leaf_vector": "1"}}


MAX = 2147483647
TREES = [
    _tree([1, -1, -1], [2, -1, -1], [MAX, 0, 0], [1, 0, 0], [0.5, 0.1, -0.3], [12.5, 0, 0], [10, 4, 6], [1, 0, 0]),
    _tree([1, -1, 3, -1, -1], [2, -1, 4, -1, -1], [MAX, 0, 0, 2, 2], [0, 0, 2, 0, 0],
          [1e-05, 0.25, 1e20, -3.0, 2.0], [2.0, 0, 4.0, 0, 0], [8, 3, 5, 2, 3], [0, 0, 1, 0, 0]),
    _tree([1, -1, -1], [2, -1, -1], [MAX, 0, 0], [1, 0, 0], [-1.5, 0.5, 0.75], [3.0, 0, 0], [6, 1, 5], [0, 0, 0]),
]


def _model(attributes=None):
    return {"version": [3, 5, 0], "learner": {
        "attributes": attributes or {}, "feature_names": [], "feature_types": [],
        "gradient_booster": {"name": "gbtree", "model": {"trees": TREES, "tree_info": [0, 0, 0],
                                                         "gbtree_model_param": {"num_trees": "3"}}},
        "learner_model_param": {"base_score": "[5E-1]", "num_class": "0", "num_feature": "3", "num_target": "1"},
        "objective": {"name": "reg:squarederror", "reg_loss_param": {}}}}


def _booster(xgb, **attributes):
    b = xgb.Booster()
    b.load_model(bytearray(json.dumps(_model(attributes)).encode()))
    return b


def test_text_and_dot_dumps(xgb):
    """XGBoosterDumpModelEx text and dot formats (src/model.cpp:401-424):
    floats with 9 significant digits, one tab per depth level."""
    b = _booster(xgb)
    text = b.get_dump()
    assert text[0] == "0:[f1<0.5] yes=1,no=2,missing=1\n\t1:leaf=0.100000001\n\t2:leaf=-0.300000012\n"
    assert text[1] == ("0:[f0<9.99999975e-06] yes=1,no=2,missing=2\n\t1:leaf=0.25\n"
                       "\t2:[f2<1.00000002e+20] yes=3,no=4,missing=3\n\t\t3:leaf=-3\n\t\t4:leaf=2\n")
    stats = b.get_dump(with_stats=True)[0]
    assert stats == ("0:[f1<0.5] yes=1,no=2,missing=1,gain=12.5,cover=10\n"
                     "\t1:leaf=0.100000001,cover=4\n\t2:leaf=-0.300000012,cover=6\n")
    dot = b.get_dump(dump_format="dot")[2]
    assert dot == ('digraph {\n    graph [ rankdir=TB ]\n    0 [ label="f1<-1.5" ]\n'
                   '    0 -> 1 [ label="yes" ]\n    0 -> 2 [ label="no, missing" ]\n'
                   '    1 [ label="leaf=0.5" ]\n    2 [ label="leaf=0.75" ]\n}\n')
    named = xgb.core._LIB
    names = (ctypes.c_char_p * 3)(b"age", b"height", b"zone")
    types = (ctypes.c_char_p * 3)(b"q", b"q", b"q")
    n = ctypes.c_uint64()
    out = ctypes.POINTER(ctypes.c_char_p)()
    assert named.XGBoosterDumpModelExWithFeatures(b.handle, 3, names, types, 0, b"text", ctypes.byref(n),
                                                  ctypes.byref(out)) == 0
    assert out[0].decode().startswith("0:[height<0.5]")
    with pytest.raises(xgb.XGBoostError, match="format"):
        b.get_dump(dump_format="yaml")


def test_json_dump_layout_and_values(xgb):
    """JSON dump (src/model.cpp:381-399): sorted keys, indent 2, each float as
    the shortest decimal of its double, so json.loads gives back the model's
    float32 values exactly and Python's own writer reproduces the text."""
    b = _booster(xgb)
    for stats in (False, True):
        for i, text in enumerate(b.get_dump(dump_format="json", with_stats=stats)):
            parsed = json.loads(text)
            assert text == json.dumps(parsed, indent=2, sort_keys=True)
            tree = TREES[i]

            def walk(node, depth):
                nid = node["nodeid"]
                if stats:
                    assert node["cover"] == float(np.float32(tree["sum_hessian"][nid]))
                if tree["left_children"][nid] < 0:
                    assert node["leaf"] == float(np.float32(tree["split_conditions"][nid]))
                    return
                assert node["depth"] == depth
                assert node["split"] == f"f{tree['split_indices'][nid]}"
                assert node["split_condition"] == float(np.float32(tree["split_conditions"][nid]))
                assert node["yes"] == tree["left_children"][nid] and node["no"] == tree["right_children"][nid]
                assert node["missing"] == (node["yes"] if tree["default_left"][nid] else node["no"])
                if stats:
                    assert node["gain"] == float(np.float32(tree["loss_changes"][nid]))
                walk(node["children"][0], depth + 1)
                walk(node["children"][1], depth + 1)

            walk(parsed, 0)
    second = b.get_dump(dump_format="json")[1]
    for literal in ('"split_condition": 9.999999747378752e-06', '"split_condition": 1.0000000200408773e+20',
                    '"leaf": -3.0', '"leaf": 0.25'):
        assert literal in second


def test_feature_scores(xgb, tmp_path):
    """XGBoosterFeatureScore (src/c_api.cpp:571-597) over the split nodes."""
    b = _booster(xgb)
    # Splits: f1 (gain 12.5, cover 10), f0 (2, 8), f2 (4, 5), f1 (3, 6).
    assert b.get_score() == {"f0": 1.0, "f1": 2.0, "f2": 1.0}
    assert b.get_fscore() == b.get_score()
    assert b.get_score(importance_type="total_gain") == {"f0": 2.0, "f1": 15.5, "f2": 4.0}
    assert b.get_score(importance_type="gain") == {"f0": 2.0, "f1": 7.75, "f2": 4.0}
    assert b.get_score(importance_type="total_cover") == {"f0": 8.0, "f1": 16.0, "f2": 5.0}
    assert b.get_score(importance_type="cover") == {"f0": 8.0, "f1": 8.0, "f2": 5.0}
    with pytest.raises(xgb.XGBoostError, match="importance"):
        b.get_score(importance_type="shap")
    fmap = tmp_path / "fmap.txt"
    fmap.write_text("0 age q\n1 height q\n2 zone q\n")
    assert b.get_score(fmap=str(fmap)) == {"age": 1.0, "height": 2.0, "zone": 1.0}
    assert b.get_dump(fmap=str(fmap))[0].startswith("0:[height<0.5]")
    reg = xgb.XGBRegressor()
    reg._Booster = b
    np.testing.assert_allclose(reg.feature_importances_, np.array([2.0, 7.75, 4.0]) / 13.75, rtol=1e-6)


def test_booster_slicing(xgb):
    """XGBoosterSlice (src/c_api.cpp:503-506, src/model.cpp:430-454)."""
    b = _booster(xgb, best_iteration="2", best_score="0.5", note="kept")
    trees = lambda m: json.loads(m.save_raw("json"))["learner"]["gradient_booster"]["model"]["trees"]
    full = trees(b)
    assert len(full) == 3
    for sl, picked in ((slice(1, 3), [1, 2]), (slice(0, 3, 2), [0, 2]), (slice(None), [0, 1, 2]), (2, [2])):
        part = b[sl]
        assert part.num_boosted_rounds() == len(picked)
        got = trees(part)
        for t, i in zip(got, picked):
            assert t["left_children"] == full[i]["left_children"]
            assert t["split_conditions"] == full[i]["split_conditions"]
    assert b[0:2].attributes() == {"note": "kept"}
    assert [t.num_boosted_rounds() for t in b] == [1, 1, 1]
    with pytest.raises(IndexError):
        b[3]
    with pytest.raises(IndexError):
        b[0:5]
    with pytest.raises(ValueError):
        b[2:1]
    with pytest.raises(xgb.XGBoostError, match="Invalid"):
        b[0:2:0]


def test_rejected_and_single_process_entry_points(xgb, tmp_path):
    """Inputs and modes outside this engine return an error, never a crash;
    the communicator is the one-process identity (src/c_api.cpp:599-615)."""
    lib = xgb.core._LIB
    h = ctypes.c_void_p()
    for call in (lambda: lib.XGDMatrixCreateFromURI(b'{"uri": "x.csv"}', ctypes.byref(h)),
                 lambda: lib.XGDMatrixCreateFromCudaArrayInterface(b"{}", b"{}", ctypes.byref(h)),
                 lambda: lib.XGDMatrixCreateFromDLPack(None, 0, ctypes.c_float(0), ctypes.byref(h)),
                 lambda: lib.XGExtMemQuantileDMatrixCreateFromCallback(None, None, None, None, None, b"{}",
                                                                       ctypes.byref(h)),
                 lambda: lib.XGTrackerCreate(b"{}", ctypes.byref(h))):
        assert call() == -1
        assert b"not supported" in lib.XGBGetLastError()
    X, _, _ = _data(10)
    with pytest.raises(xgb.XGBoostError, match="not supported"):
        xgb.DMatrix(X).save_binary(str(tmp_path / "m.buffer"))
    assert lib.XGCommunicatorInit(b"{}") == 0
    assert lib.XGCommunicatorGetRank() == 0 and lib.XGCommunicatorGetWorldSize() == 1
    assert lib.XGCommunicatorIsDistributed() == 0
    assert lib.XGCommunicatorInit(b'{"dmlc_communicator": "rabit"}') == -1
    buf = (ctypes.c_float * 3)(1, 2, 3)
    assert lib.XGCommunicatorAllreduce(buf, ctypes.c_size_t(3), 2, 2) == 0
    assert list(buf) == [1, 2, 3]
    assert lib.XGCommunicatorFinalize() == 0
    out = ctypes.c_void_p(1)
    d = xgb.DMatrix(X)
    assert lib.XGDMatrixGetCategories(d.handle, b"{}", ctypes.byref(out)) == 0 and out.value is None
    z = ctypes.c_int(7)
    assert lib.XGDMatrixWasZeroCopied(d.handle, ctypes.byref(z)) == 0 and z.value == 0


def test_get_info_ref(xgb):
    """XGDMatrixGetInfoRef returns an array interface of the stored field
    (src/c_api.cpp:255-268)."""
    X, y, _ = _data(12)
    d = xgb.DMatrix(X, label=y)
    lib = xgb.core._LIB
    out = ctypes.c_char_p()
    assert lib.XGDMatrixGetInfoRef(d.handle, b"label", ctypes.byref(out)) == 0
    inter = json.loads(out.value)
    assert inter["shape"] == [12] and inter["typestr"] == "<f4"
    got = np.ctypeslib.as_array((ctypes.c_float * 12).from_address(inter["data"][0]))
    np.testing.assert_array_equal(got, y)
