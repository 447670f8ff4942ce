"""GPU checks of the API surface around training: iterator-fed matrices train
the same trees as one matrix, a `ref` matrix shares its cuts, in-place
prediction equals DMatrix prediction, and model slices predict like
iteration ranges (reference src/c_api.cpp:222-239, :503-518)."""
import ctypes
import json

import numpy as np
import pytest

import workloads as W

pytestmark = pytest.mark.gpu

PARAMS = {"tree_method": "hist", "max_depth": 5, "max_bin": 64, "eta": 0.3, "objective": "reg:squarederror"}


def _batches(xgb):
    class Batches(xgb.DataIter):
        def __init__(self, parts):
            self.parts = parts
            self.i = 0
            super().__init__()

        def next(self, input_data):
            if self.i == len(self.parts):
                return False
            input_data(**self.parts[self.i])
            self.i += 1
            return True

        def reset(self):
            self.i = 0

    return Batches


def _trees(bst):
    return json.loads(bst.save_raw("json"))["learner"]["gradient_booster"]["model"]["trees"]


def test_iterator_matrices_train_like_one_matrix(xgb):
    X, y = W.config1(rows=6000, cols=10)
    Batches = _batches(xgb)
    splits = [0, 1500, 4000, 6000]
    parts = [dict(data=X[a:b], label=y[a:b]) for a, b in zip(splits, splits[1:])]
    whole = xgb.train(PARAMS, xgb.DMatrix(X, label=y), 8)
    it = xgb.train(PARAMS, xgb.DMatrix(Batches(parts)), 8)
    assert _trees(it) == _trees(whole)
    q_whole = xgb.train(PARAMS, xgb.QuantileDMatrix(X, label=y, max_bin=64), 8)
    q_it = xgb.train(PARAMS, xgb.QuantileDMatrix(Batches(parts), max_bin=64), 8)
    assert _trees(q_it) == _trees(q_whole) == _trees(whole)


def test_ref_matrix_shares_cuts(xgb):
    X, y = W.config1(rows=5000, cols=8)
    train = xgb.QuantileDMatrix(X, label=y, max_bin=32)
    xgb.train({**PARAMS, "max_bin": 32}, train, 2)
    sub = X[:700] * 0.5  # a different distribution: its own sketch would differ
    ev = xgb.QuantileDMatrix(sub, label=y[:700], ref=train, max_bin=32)
    own = xgb.QuantileDMatrix(sub, label=y[:700], max_bin=32)
    bst = xgb.train({**PARAMS, "max_bin": 32}, ev, 1)
    ip_ref, cut_ref = train.get_quantile_cut()
    ip_ev, cut_ev = ev.get_quantile_cut()
    np.testing.assert_array_equal(ip_ev, ip_ref)
    np.testing.assert_array_equal(cut_ev.view(np.uint32), cut_ref.view(np.uint32))
    xgb.train({**PARAMS, "max_bin": 32}, own, 1)
    _, cut_own = own.get_quantile_cut()
    assert cut_own.shape != cut_ref.shape or not np.array_equal(cut_own, cut_ref)
    assert bst.num_boosted_rounds() == 1


def test_inplace_predict_equals_dmatrix_predict(xgb):
    import scipy.sparse as sp
    X, y = W.config1(rows=3000, cols=12)
    bst = xgb.train(PARAMS, xgb.DMatrix(X, label=y), 10)
    d = xgb.DMatrix(X)
    for kind, margin in (("value", False), ("margin", True)):
        expect = bst.predict(d, output_margin=margin)
        np.testing.assert_array_equal(bst.inplace_predict(X, predict_type=kind), expect)
    np.testing.assert_array_equal(bst.inplace_predict(X, iteration_range=(2, 7)),
                                  bst.predict(d, iteration_range=(2, 7)))
    Xs = np.where(np.isnan(X), 0, X)
    Xs[np.abs(Xs) < 0.5] = 0
    ds = xgb.DMatrix(sp.csr_matrix(Xs))
    np.testing.assert_array_equal(bst.inplace_predict(sp.csr_matrix(Xs)), bst.predict(ds))
    # `missing` applies to in-place input as to a DMatrix.
    Xm = np.where(np.isnan(X), -999.0, X).astype(np.float32)
    np.testing.assert_array_equal(bst.inplace_predict(Xm, missing=-999.0), bst.predict(d))


def test_model_slices_predict_like_iteration_ranges(xgb):
    X, y = W.config1(rows=2000, cols=6)
    bst = xgb.train(PARAMS, xgb.DMatrix(X, label=y), 9)
    d = xgb.DMatrix(X)
    for a, b in ((0, 3), (3, 9), (4, 5)):
        np.testing.assert_array_equal(bst[a:b].predict(d), bst.predict(d, iteration_range=(a, b)))
    # A stepped slice holds rounds 0, 3 and 6: its margin is the base margin
    # plus those three trees.
    base = float(json.loads(bst.save_raw("json"))["learner"]["learner_model_param"]["base_score"].strip("[]"))
    single = [bst[r:r + 1].predict(d, output_margin=True).astype(np.float64) - base for r in (0, 3, 6)]
    np.testing.assert_allclose(bst[0:9:3].predict(d, output_margin=True), base + sum(single), rtol=1e-6, atol=1e-6)


def test_predict_to_buffer(xgb):
    X, y = W.config1(rows=500, cols=5)
    bst = xgb.train(PARAMS, xgb.DMatrix(X, label=y), 3)
    d = xgb.DMatrix(X)
    lib = xgb.core._LIB
    buf = np.zeros(500, np.float32)
    shape = ctypes.POINTER(ctypes.c_uint64)()
    dims = ctypes.c_uint64()
    cfg = json.dumps({"type": 0, "training": False, "iteration_begin": 0, "iteration_end": 0,
                      "strict_shape": False}).encode()
    assert lib.XGBoosterPredictToBuffer(bst.handle, d.handle, cfg, buf.ctypes.data_as(ctypes.c_void_p),
                                        ctypes.c_uint64(500), ctypes.byref(shape), ctypes.byref(dims)) == 0
    assert dims.value == 1 and shape[0] == 500
    np.testing.assert_array_equal(buf, bst.predict(d))
    small = np.zeros(10, np.float32)
    assert lib.XGBoosterPredictToBuffer(bst.handle, d.handle, cfg, small.ctypes.data_as(ctypes.c_void_p),
                                        ctypes.c_uint64(10), ctypes.byref(shape), ctypes.byref(dims)) == -1
    assert b"capacity" in lib.XGBGetLastError()
    assert not small.any()


def test_queued_rounds_equal_drained_rounds(xgb):
    """Rounds queued without host synchronisation (trees copied back only when
    the model is read, or when 64 are pending) give the same model as rounds
    read back one at a time, with parameter and attribute calls in between."""
    X, y = W.config1(rows=4000, cols=10)
    d = xgb.DMatrix(X, label=y)
    params = {"max_depth": 5, "max_bin": 64, "subsample": 0.8, "colsample_bytree": 0.7, "seed": 3}
    queued = xgb.Booster(params, [d])
    stepwise = xgb.Booster(params, [d])
    for i in range(70):  # more than one queue's worth
        queued.update(d, i)
        queued.set_attr(note=str(i))
        if i == 30:
            queued.set_param("learning_rate", 0.1)
        stepwise.update(d, i)
        assert stepwise.num_boosted_rounds() == i + 1
        if i == 30:
            stepwise.set_param("learning_rate", 0.1)
    assert queued.num_boosted_rounds() == 70
    assert _trees(queued) == _trees(stepwise)
    np.testing.assert_array_equal(queued.predict(d), stepwise.predict(d))
    profiled = xgb.Booster(dict(params, hip_profile=1), [d])  # profiled rounds stay synchronous
    for i in range(5):
        profiled.update(d, i)
    assert _trees(profiled) == _trees(stepwise[:5])


@pytest.mark.parametrize("max_bin,missing", [(64, False), (1000, True)])
def test_compacted_sampled_rows_equal_full_row_list(xgb, max_bin, missing):
    """A subsample's dropped rows leave the row list before the root and get
    their leaves from a walk of the finished tree: the trees and the training
    margins (the cached margins the next round's gradients read) equal those
    of the full row list, u8 and u16 codes, with and without missing values."""
    rng = np.random.default_rng(max_bin)
    X = rng.normal(size=(30000, 12)).astype(np.float32)
    if missing:
        X[rng.random(X.shape) < 0.1] = np.nan
    y = (np.nan_to_num(X[:, 0]) + 0.3 * rng.normal(size=30000) > 0).astype(np.float32)
    d = xgb.DMatrix(X, label=y)
    params = {"objective": "binary:logistic", "max_depth": 6, "max_bin": max_bin, "subsample": 0.6,
              "colsample_bytree": 0.8, "seed": 11}
    compact = xgb.train(params, d, 6)
    full = xgb.train(dict(params, hip_compact_sampled=0), d, 6)
    assert _trees(compact) == _trees(full)
    # The training margins: the cache of the training matrix against a fresh
    # prediction of the same rows.
    fresh = xgb.DMatrix(X)
    for bst in (compact, full):
        np.testing.assert_array_equal(bst.predict(d, output_margin=True), bst.predict(fresh, output_margin=True))


@pytest.mark.parametrize("subsample,max_depth", [(1e-3, 4), (0.5, 1), (0.9, 2)])
def test_compacted_rows_edge_cases(xgb, subsample, max_depth):
    """Compaction when a round keeps a handful of rows (or none), and when the
    root is also the last level (its partition reads the compacted list):
    trees and training margins equal the full row list's."""
    import oracle_lib as O
    X, y = W.config0(rows=3000, cols=6)
    d = xgb.DMatrix(X, label=y)
    params = {"max_depth": max_depth, "max_bin": 32, "subsample": subsample, "seed": 4}
    compact = xgb.train(params, d, 4)
    full = xgb.train(dict(params, hip_compact_sampled=0), d, 4)
    assert _trees(compact) == _trees(full)
    np.testing.assert_array_equal(compact.predict(d, output_margin=True), full.predict(d, output_margin=True))
    ref = O.train(X, y, O.make_params(max_depth=max_depth, max_bin=32, subsample=subsample, seed=4), 4)
    np.testing.assert_array_equal(compact.predict(d, output_margin=True).view(np.uint32), ref["margin"].view(np.uint32))


def test_monotone_constraints_parameter_errors(xgb):
    """monotone_constraints as the reference parses it (src/tree.cpp:15-26):
    "(..)" or "[..]" lists of -1, 0, 1, at most one entry per feature; anything
    else fails with the reference's messages, and all zeros is unconstrained."""
    X, y = W.config0(rows=2000, cols=4)
    d = xgb.DMatrix(X, label=y)
    base = {"max_depth": 3, "max_bin": 32}
    for bad, message in [("(2,0)", "must be -1, 0 or 1"), ("(1,0,0,0,1)", "more entries than features"),
                         ("(1,x)", "list of -1, 0 or 1"), ("(0.5)", "list of -1, 0 or 1")]:
        with pytest.raises(xgb.core.XGBoostError, match=message.replace("(", r"\(")):
            xgb.train(dict(base, monotone_constraints=bad), d, 1)
    free = xgb.train(base, d, 3)
    for same in ["()", "[]", "(0,0)", "[0, 0, 0, 0]"]:
        assert _trees(xgb.train(dict(base, monotone_constraints=same), d, 3)) == _trees(free)
    short = xgb.train(dict(base, monotone_constraints="(1)"), d, 3)
    longer = xgb.train(dict(base, monotone_constraints="[1,0,0,0]"), d, 3)
    assert _trees(short) == _trees(longer)


def test_monotone_constraints_by_feature_name(xgb):
    """A dict of feature names maps to the positional constraint list."""
    X, y = W.config0(rows=2000, cols=4)
    names = ["a", "b", "c", "d"]
    d = xgb.DMatrix(X, label=y, feature_names=names)
    base = {"max_depth": 3, "max_bin": 32}
    by_name = xgb.train(dict(base, monotone_constraints={"c": -1, "a": 1}), d, 3)
    by_position = xgb.train(dict(base, monotone_constraints="(1,0,-1,0)"), d, 3)
    assert _trees(by_name) == _trees(by_position)
    with pytest.raises(ValueError, match="not a subset"):
        xgb.train(dict(base, monotone_constraints={"z": 1}), d, 1)


def test_device_status_refuses_round_and_rolls_back(xgb):
    """A round whose tree the device flags is refused when the model is read
    (src/learner.cpp:36-61 retire_round, src/tree.cpp:1664-1665): the status
    word is set from the test parameter hip_inject_tree_status while every
    kernel runs normally; XGBoostError names the round, the rounds queued
    after it are dropped with it, and the model keeps the earlier rounds.
    The training margins are rebuilt from the kept trees, so predictions and
    further rounds equal those of a model that never saw the refused round."""
    X, y = W.config1(rows=5000, cols=8)
    params = {"tree_method": "hist", "max_depth": 4, "max_bin": 32}
    d = xgb.DMatrix(X, label=y)
    clean3 = xgb.train(params, d, 3)
    clean4 = xgb.train(params, d, 4)
    bst = xgb.Booster(params, [d])
    for i in range(3):
        bst.update(d, i)
    bst.set_param({"hip_inject_tree_status": 2})
    bst.update(d, 3)
    bst.set_param({"hip_inject_tree_status": 0})
    bst.update(d, 4)
    with pytest.raises(xgb.XGBoostError, match=r"round 3: the device tree is invalid: .*0x2 .*capacity.*1 later"):
        bst.predict(d)
    assert bst.num_boosted_rounds() == 3
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), clean3.predict(d).view(np.uint32))
    bst.update(d, 3)
    assert bst.num_boosted_rounds() == 4
    assert _trees(bst) == _trees(clean4)
    np.testing.assert_array_equal(bst.predict(d).view(np.uint32), clean4.predict(d).view(np.uint32))
