"""GPU checks of the runtime under the training path: the allocator hands
freed device buffers out again (no two live buffers overlap, and nothing a
kernel computes depends on what a reused buffer held), and the ring of
queued rounds drains when it fills in the middle of training with the same
trees as draining every round (reference src/learner.cpp:25-35 round
buffers, :36-61 retire_round)."""
import ctypes
import json

import numpy as np
import pytest
import scipy.sparse as sp

import device_lib as D
import workloads as W

pytestmark = pytest.mark.gpu


def _fill(dev, seed):
    pattern = np.random.default_rng(seed).integers(0, 256, dev.nbytes, dtype=np.uint8)
    D.check(D.lib().mgb_memcpy_h2d(dev.ptr, pattern.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(dev.nbytes)))
    return pattern


def test_kept_buffers_never_overlap():
    # Sizes around the allocator's granules (256 bytes up to 1 MiB, then
    # 2 MiB): freed blocks are handed out again to requests of about their size.
    sizes = [16, 255, 256, 4096, 65536, (1 << 20) - 8, (1 << 20) + 8, 3 << 20, (5 << 20) + 1]
    live = {}
    for round_ in range(4):
        for k, n in enumerate(sizes):
            dev = D.Device(n)
            live[(round_, k)] = (dev, _fill(dev, 1000 * round_ + k))
        # Free every other buffer of this round, so the next round reuses them.
        for k in range(0, len(sizes), 2):
            del live[(round_, k)]
    for (round_, k), (dev, pattern) in live.items():
        got = dev.read(np.uint8, dev.nbytes)
        assert np.array_equal(got, pattern), (round_, k)


def test_free_refuses_a_pointer_it_did_not_hand_out():
    dev = D.Device(4096)
    lib = D.lib()
    lib.mgb_last_error.restype = ctypes.c_char_p
    inside = ctypes.c_void_p(dev.ptr.value + 256)
    assert lib.mgb_free(inside) == -1
    assert b"not a buffer from mgb_malloc" in lib.mgb_last_error()
    assert dev.read(np.uint8, 16).shape == (16,)  # the buffer itself is still live


def _predict_bits(xgb, X, y, params, rounds):
    d = xgb.DMatrix(X, label=y)
    bst = xgb.train(params, d, rounds)
    return bst.predict(d).view(np.uint32)


def test_training_does_not_depend_on_reused_memory(xgb):
    params = {"tree_method": "hist", "max_depth": 6, "max_bin": 64, "eta": 0.3, "objective": "reg:squarederror"}
    X, y = W.config2(rows=20000, cols=16)
    first = _predict_bits(xgb, X, y, params, 10)
    # Other shapes, depths, bin widths, sampling, a logistic objective and a
    # CSR matrix leave differently filled buffers behind for the allocator.
    for seed, (rows, cols, depth, max_bin) in enumerate([(30000, 24, 8, 256), (5000, 8, 3, 16), (12000, 40, 10, 1024)]):
        Xo, yo = W.config2(rows=rows, cols=cols, seed=seed + 7)
        other = dict(params, max_depth=depth, max_bin=max_bin, subsample=0.7, colsample_bytree=0.6, seed=seed)
        _predict_bits(xgb, Xo, yo, other, 6)
    indptr, indices, values, yl = W.config3(rows=4000, cols=300, informative=40)
    csr = sp.csr_matrix((values, indices, indptr), shape=(4000, 300))
    xgb.train({"tree_method": "hist", "max_depth": 5, "objective": "binary:logistic"}, xgb.DMatrix(csr, label=yl), 4)
    again = _predict_bits(xgb, X, y, params, 10)
    assert np.array_equal(first, again)


def test_full_ring_drains_like_every_round(xgb):
    # Depth 2 trees take 512-byte slots: the ring holds 1,024 rounds, so the
    # 1,025th drains the queue in the middle of training.
    X, y = W.config1(rows=600, cols=4)
    params = {"tree_method": "hist", "max_depth": 2, "max_bin": 16, "eta": 0.05, "objective": "reg:squarederror"}
    d = xgb.DMatrix(X, label=y)
    rounds = 1100
    queued = xgb.Booster(params, [d])
    for i in range(rounds):
        queued.update(d, i)
    stepwise = xgb.Booster(params, [d])
    for i in range(rounds):
        stepwise.update(d, i)
        assert stepwise.num_boosted_rounds() == i + 1  # drains this round
    assert queued.num_boosted_rounds() == rounds
    t_queued = json.loads(queued.save_raw("json"))["learner"]["gradient_booster"]["model"]["trees"]
    t_step = json.loads(stepwise.save_raw("json"))["learner"]["gradient_booster"]["model"]["trees"]
    assert t_queued == t_step
    assert np.array_equal(queued.predict(d).view(np.uint32), stepwise.predict(d).view(np.uint32))
