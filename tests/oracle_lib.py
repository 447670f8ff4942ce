"""ctypes binding of the CPU oracle (oracle/libhist_oracle.so).

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this module.
"""
import ctypes
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
LIB_PATH = ROOT / "oracle" / "_build" / "libhist_oracle.so"


class OracleParams(ctypes.Structure):
    _fields_ = [("objective", ctypes.c_int32), ("max_depth", ctypes.c_int32), ("max_bin", ctypes.c_int32),
                ("fma_contract", ctypes.c_int32), ("eta", ctypes.c_float), ("reg_lambda", ctypes.c_float),
                ("reg_alpha", ctypes.c_float), ("min_child_weight", ctypes.c_float),
                ("max_delta_step", ctypes.c_float), ("min_split_loss", ctypes.c_float),
                ("scale_pos_weight", ctypes.c_float), ("base_score", ctypes.c_float),
                ("has_base_score", ctypes.c_int32), ("nthread", ctypes.c_int32),
                ("subsample", ctypes.c_float), ("colsample_bytree", ctypes.c_float), ("seed", ctypes.c_uint32),
                ("monotone", ctypes.c_void_p), ("std_shuffle", ctypes.c_int32),
                ("seed_per_iteration", ctypes.c_int32)]


NODE_DTYPE = np.dtype([("left", "<i4"), ("right", "<i4"), ("parent", "<i4"), ("feature", "<i4"),
                       ("threshold", "<f4"), ("leaf", "<f4"), ("cover", "<f4"), ("gain", "<f4"),
                       ("default_left", "<u4"), ("base_weight", "<f4")])

SPLIT_DTYPE = np.dtype([("gain", "<f4"), ("threshold", "<f4"), ("left_weight", "<f4"), ("right_weight", "<f4"),
                        ("left_h", "<f4"), ("right_h", "<f4"), ("parent_weight", "<f4"), ("total_g", "<f4"),
                        ("total_h", "<f4"), ("feature", "<i4"), ("default_left", "<u4"), ("bin", "<u4"),
                        ("left_g", "<i8"), ("left_hs", "<i8"), ("right_g", "<i8"), ("right_hs", "<i8")])

OBJECTIVES = {"reg:squarederror": 0, "binary:logistic": 1, "binary:logitraw": 2}
SHUFFLE_MODELS = {"libstdc++": 0, "libc++": 1}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            import subprocess
            subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.oracle_max_nodes.restype = ctypes.c_uint32
        _lib.oracle_sketch_budget.restype = ctypes.c_uint32
        _lib.oracle_gradient_scale.restype = ctypes.c_float
        _lib.oracle_base_score.restype = ctypes.c_float
        _lib.oracle_base_margin.restype = ctypes.c_float
        _lib.oracle_weight.restype = ctypes.c_float
        _lib.oracle_weight.argtypes = [ctypes.c_double, ctypes.c_double, ctypes.POINTER(OracleParams)]
        _lib.oracle_sigmoid.restype = ctypes.c_float
        _lib.oracle_sigmoid.argtypes = [ctypes.c_float]
        _lib.oracle_gain.restype = ctypes.c_float
        _lib.oracle_gain.argtypes = [ctypes.c_double, ctypes.c_double, ctypes.c_float, ctypes.POINTER(OracleParams)]
    return _lib


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def make_params(objective="reg:squarederror", max_depth=6, max_bin=256, eta=0.3, reg_lambda=1.0, reg_alpha=0.0,
                min_child_weight=1.0, max_delta_step=0.0, min_split_loss=0.0, scale_pos_weight=1.0,
                base_score=None, fma_contract=1, nthread=0, subsample=1.0, colsample_bytree=1.0, seed=0,
                monotone=None, std_shuffle="libstdc++", seed_per_iteration=0):
    """monotone: one -1/0/1 per feature, or None.  std_shuffle: the standard
    library whose std::shuffle draws the column sample ("libstdc++" or
    "libc++")."""
    mono = None if monotone is None else np.ascontiguousarray(monotone, np.int32)
    p = OracleParams(OBJECTIVES[objective], max_depth, max_bin, fma_contract, eta, reg_lambda, reg_alpha,
                     min_child_weight, max_delta_step, min_split_loss, scale_pos_weight,
                     0.0 if base_score is None else base_score, 0 if base_score is None else 1, nthread,
                     subsample, colsample_bytree, seed, None if mono is None else mono.ctypes.data,
                     SHUFFLE_MODELS[std_shuffle], int(seed_per_iteration))
    p._monotone = mono  # keeps the array alive while the parameters are
    return p


def sketch_cuts(X, max_bin, weights=None):
    X = np.ascontiguousarray(X, np.float32)
    rows, cols = X.shape
    cuts = np.zeros((cols, max_bin), np.float32)
    counts = np.zeros(cols, np.uint32)
    minima = np.zeros(cols, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    lib().oracle_sketch_cuts(ptr(X), ctypes.c_uint32(rows), ctypes.c_uint32(cols), ptr(w), ctypes.c_uint32(max_bin),
                             ptr(cuts), ptr(counts), ptr(minima))
    return cuts, counts, minima


def quantize(X, cuts, counts):
    X = np.ascontiguousarray(X, np.float32)
    rows, cols = X.shape
    bins = np.zeros((rows, cols), np.uint16)
    lib().oracle_quantize(ptr(X), ctypes.c_uint32(rows), ctypes.c_uint32(cols), ptr(np.ascontiguousarray(cuts)),
                          ptr(np.ascontiguousarray(counts, np.uint32)), ctypes.c_uint32(cuts.shape[1]), ptr(bins))
    return bins


def gradient_scale(values):
    v = np.ascontiguousarray(values, np.float32)
    return float(lib().oracle_gradient_scale(ptr(v), ctypes.c_uint32(len(v))))


def base_score(labels, weights=None, objective=0, scale_pos_weight=1.0):
    y = np.ascontiguousarray(labels, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    return float(lib().oracle_base_score(ctypes.c_int32(objective), ptr(y), ptr(w) if w is not None else None,
                                         ctypes.c_uint32(len(y)), ctypes.c_float(scale_pos_weight)))


def train(X, y, params, rounds, weights=None, custom_grad=None, custom_hess=None):
    X = np.ascontiguousarray(X, np.float32)
    y = np.ascontiguousarray(y, np.float32)
    rows, cols = X.shape
    max_nodes = lib().oracle_max_nodes(params.max_depth)
    trees = np.zeros((rounds, max_nodes), NODE_DTYPE)
    sizes = np.zeros(rounds, np.uint32)
    margin = np.zeros(rows, np.float32)
    base = ctypes.c_float(0)
    cuts = np.zeros((cols, params.max_bin), np.float32)
    counts = np.zeros(cols, np.uint32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    cg = None if custom_grad is None else np.ascontiguousarray(custom_grad, np.float32)
    ch = None if custom_hess is None else np.ascontiguousarray(custom_hess, np.float32)
    rc = lib().oracle_train(ptr(X), ctypes.c_uint32(rows), ctypes.c_uint32(cols), ptr(y), ptr(w),
                            ctypes.byref(params), ctypes.c_uint32(rounds), ptr(cg), ptr(ch), ptr(trees), ptr(sizes),
                            ptr(margin), ctypes.byref(base), ptr(cuts), ptr(counts))
    if rc != 0:
        raise RuntimeError("oracle_train failed")
    return {"trees": trees, "sizes": sizes, "margin": margin, "base_score": base.value, "cuts": cuts,
            "cut_counts": counts}


def sigmoid(margin):
    """binary:logistic's prediction transform (upstream XGBoost's Sigmoid
    over the host libm's expf)."""
    margin = np.ascontiguousarray(margin, np.float32)
    out = np.empty_like(margin)
    lib().oracle_sigmoid_array(ptr(margin), ptr(out), ctypes.c_uint64(margin.size))
    return out


def predict_margin(X, result, base_margin):
    X = np.ascontiguousarray(X, np.float32)
    rows, cols = X.shape
    out = np.zeros(rows, np.float32)
    trees = result["trees"]
    lib().oracle_predict_margin(ptr(X), ctypes.c_uint32(rows), ctypes.c_uint32(cols), ptr(trees),
                                ptr(result["sizes"]), ctypes.c_uint32(trees.shape[0]),
                                ctypes.c_uint32(trees.shape[1]), ctypes.c_float(base_margin), ptr(out))
    return out


class OracleMT(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint32 * 624), ("next", ctypes.c_uint32)]


def mt_outputs(seed, count):
    """First `count` outputs of the oracle's MT19937 seeded with `seed`."""
    g = OracleMT()
    lib().oracle_mt_seed(ctypes.byref(g), ctypes.c_uint32(seed))
    lib().oracle_mt_next.restype = ctypes.c_uint32
    return np.array([lib().oracle_mt_next(ctypes.byref(g)) for _ in range(count)], np.uint32)


def sample_rows(seed, rows, subsample):
    """Keep mask of uniform row sampling for one round."""
    f = lib().oracle_sample_row
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float]
    return np.array([f(seed, r, subsample) for r in range(rows)], bool)


def sample_columns(n, fraction, seed, std_shuffle="libstdc++"):
    out = np.zeros(max(n, 1), np.uint32)
    f = lib().oracle_sample_columns
    f.restype = ctypes.c_uint32
    k = f(ctypes.c_uint32(n), ctypes.c_float(fraction), ctypes.c_uint32(seed), ctypes.c_int32(SHUFFLE_MODELS[std_shuffle]),
          ptr(out))
    return out[:k]


def std_shuffle(n, seed, model="libstdc++"):
    """std::shuffle of 0..n-1 over std::mt19937(seed); returns the permutation
    and the engine's next output (which shows how many draws were taken)."""
    g = (ctypes.c_uint32 * 625)()
    lib().oracle_mt_seed(g, ctypes.c_uint32(seed))
    v = np.arange(max(n, 1), dtype=np.uint32)
    lib().oracle_std_shuffle(ptr(v), ctypes.c_uint32(n), g, ctypes.c_int32(SHUFFLE_MODELS[model]))
    nxt = lib().oracle_mt_next
    nxt.restype = ctypes.c_uint32
    return v[:n], int(nxt(g))


def metric_sum(pred, labels, kind, weights=None, parameter=0.0):
    """(sum of weight * loss, sum of weight) in the reference's fp32 order."""
    pred = np.ascontiguousarray(pred, np.float32)
    labels = np.ascontiguousarray(labels, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    out = np.zeros(2, np.float32)
    lib().oracle_metric_sum(ptr(pred), ptr(labels), ptr(w), ctypes.c_uint32(pred.size), ctypes.c_uint32(kind),
                            ctypes.c_float(parameter), ptr(out))
    return out


def metric_auc(pred, labels, pr=False, weights=None):
    """(area, positive weight, negative weight) in binary64."""
    pred = np.ascontiguousarray(pred, np.float32)
    labels = np.ascontiguousarray(labels, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, np.float32)
    out = np.zeros(3, np.float64)
    lib().oracle_metric_auc(ptr(pred), ptr(labels), ptr(w), ctypes.c_uint32(pred.size), ctypes.c_int(int(pr)),
                            ptr(out))
    return out


def cv_folds(rows, nfold, seed, shuffle=True, stratified=False, labels=None, std_shuffle="libstdc++"):
    fold = np.zeros(max(rows, 1), np.int32)
    y = None if labels is None else np.ascontiguousarray(labels, np.float32)
    lib().oracle_cv_folds(ctypes.c_uint32(rows), ctypes.c_int(nfold), ctypes.c_uint32(seed), ctypes.c_int(int(shuffle)),
                          ctypes.c_int(int(stratified)), ptr(y), ctypes.c_int32(SHUFFLE_MODELS[std_shuffle]), ptr(fold))
    return fold[:rows]
