#!/usr/bin/env python3
"""Benchmark of the MI355X hist engine on BASELINE.json's metric.

Metric: ms per 100 boosting rounds at 262,144 x 64, depth 8,
plus histogram-build throughput against MI355X's 8 TB/s HBM peak.

A step is one boosting round (gradients, quantization scale, one depth-8 tree,
training-margin update) over the device-resident, already quantized matrix.
value = 100 x the mean step time.  The one-time quantile sketch and bin matrix
build are reported separately (fit_* fields), as is the time of a whole
xgb.train call from host numpy arrays.

The roofline object covers the histogram kernel: algorithmic bytes per launch
(rows built x (F code bytes + 4-byte row id + 8-byte gradient pair) + nodes
built x F x (max_bin+1) x 16 bytes of int64 histogram output) divided by the
kernel's duration, measured with HIP events on the library's stream inside the
timed rounds.  cpu_baseline times the CPU oracle (a port of the reference's
algorithm, OpenMP over features) on the host cores on a bounded sample.
"""
import argparse
import hashlib
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "xgboost-metal_amd" / "python"))
sys.path.insert(0, str(ROOT / "tests"))

HBM_PEAK_GBPS = 8000.0
REFERENCE_MS_100 = 222.8  # reference Metal engine, 262,144x64 d8, 100 rounds, M5 Ultra


def config2(rows=262144, cols=64, seed=1337):
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(rows, cols)).astype(np.float32)
    w = rng.normal(size=cols).astype(np.float32)
    y = (X @ w + 0.5 * np.sin(X[:, 0] * X[:, 1]) + 0.1 * rng.normal(size=rows)).astype(np.float32)
    return X, y


PARAMS = {"objective": "reg:squarederror", "tree_method": "hist", "max_depth": 8, "max_bin": 256, "eta": 0.3,
          "lambda": 1}

C4_PARAMS = {"objective": "binary:logistic", "tree_method": "hist", "max_depth": 10, "max_bin": 1024, "eta": 0.1,
             "subsample": 0.8, "colsample_bytree": 0.8}


def config4(rows=10_000_000, seed=1337, chunk=1 << 20):
    """columns 0-63 N(0,1), 64-95 U(0,1), 96-127 integers in
    [0, 999] as float32; y ~ Bernoulli(sigmoid(X[:, :16] . w + 0.3 N)).  Drawn
    in row chunks (float32 storage) so the float64 temporaries stay small."""
    rng = np.random.default_rng(seed)
    w = rng.normal(size=16)
    X = np.empty((rows, 128), np.float32)
    y = np.empty(rows, np.float32)
    for a in range(0, rows, chunk):
        b = min(rows, a + chunk)
        n = b - a
        X[a:b, :64] = rng.normal(size=(n, 64))
        X[a:b, 64:96] = rng.random((n, 32))
        X[a:b, 96:] = rng.integers(0, 1000, size=(n, 32))
        s = X[a:b, :16].astype(np.float64) @ w + 0.3 * rng.normal(size=n)
        y[a:b] = rng.random(n) < 1.0 / (1.0 + np.exp(-s))
    return X, y


def time_rounds(xgb, dtrain, rounds, profile, base=PARAMS):
    params = dict(base, hip_profile=1 if profile else 0)
    bst = xgb.Booster(params, [dtrain])
    bst.update(dtrain, 0)  # initialise (base score, buffers); not timed
    bst.num_boosted_rounds()  # the library queues rounds: wait for the untimed one
    start = time.perf_counter()
    for i in range(rounds):
        bst.update(dtrain, i + 1)
    # Rounds are queued on the device without host synchronisation; the round
    # count waits for all of them and copies their trees to the host, so the
    # timed region covers every round's kernels and its model transfer.
    bst.num_boosted_rounds()
    elapsed = time.perf_counter() - start
    return bst, elapsed


def stream_copy_gbps(mib=1024):
    import ctypes
    import device_lib as D
    n = mib << 20
    src, dst = D.Device(n), D.Device(n)
    lib = D.lib()
    lib.mgb_event_record(0)
    for _ in range(5):
        D.check(lib.mgb_stream_copy(dst.ptr, src.ptr, ctypes.c_size_t(n)))
    lib.mgb_event_record(1)
    ms = ctypes.c_float()
    D.check(lib.mgb_event_elapsed_ms(0, 1, ctypes.byref(ms)))
    return 5 * 2 * n / (ms.value * 1e-3) / 1e9


def cpu_baseline(X, y, target_seconds):
    import oracle_lib as O
    threads = min(os.cpu_count() or 1, 16)
    p = O.make_params(max_depth=8, max_bin=256, eta=0.3, nthread=threads)
    t0 = time.perf_counter()
    O.train(X, y, p, 1)
    one = time.perf_counter() - t0
    t0 = time.perf_counter()
    O.train(X, y, p, 3)
    three = time.perf_counter() - t0
    # Enough extra rounds for about target_seconds of timed CPU work.
    est = max((three - one) / 2, 1e-3)
    rounds = int(min(max(target_seconds / est, 3), 200))
    t0 = time.perf_counter()
    O.train(X, y, p, rounds + 1)
    many = time.perf_counter() - t0
    per_round = max(many - one, 1e-9) / rounds
    return {"value": round(per_round * 100 * 1e3, 1), "unit": "ms/100 rounds", "cores": threads, "kind": "port",
            "sample": f"CPU oracle (C restatement of the reference's hist path, OpenMP over features), config 2 "
                      f"262144x64 d8: {rounds} rounds timed as T({rounds + 1} rounds) - T(1 round), "
                      f"scaled to 100 rounds; {many + one + three:.1f} s of CPU work"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--config", choices=["c2", "c3", "c4"], default="c2",
                    help="c2 (default): the headline metric; c3: 1M x 2000 CSR, 20 nonzeros a row; "
                         "c4: 10M x 128, 1024 bins, depth 10 (HBM-bound check)")
    ap.add_argument("--param", action="append", default=[], metavar="KEY=VALUE",
                    help="extra booster parameter for the timed rounds (repeatable), e.g. hip_histogram_rows=2048")
    args = ap.parse_args()
    extra = {}
    for item in args.param:
        key, sep, value = item.partition("=")
        if not sep:
            ap.error(f"--param expects KEY=VALUE, got {item!r}")
        extra[key] = value
    PARAMS.update(extra)
    for spec in LARGE.values():
        spec["params"].update(extra)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(row-sharded multi-GPU training is a design note, not implemented).", file=sys.stderr)
        sys.exit(2)
    import xgboost as xgb
    if args.config in LARGE:
        return bench_large(xgb, args, args.config)

    X, y = config2()
    dtrain = xgb.DMatrix(X, label=y)
    # Warm-up: code loading, buffers and the one-time sketch + bin matrix.
    t0 = time.perf_counter()
    warm = xgb.train(dict(PARAMS), dtrain, max(1, args.warmup))
    first_fit = time.perf_counter() - t0
    prof0 = warm.profile()["seconds"]
    sketch_s = prof0.get("quantiles", 0.0)
    bins_s = prof0.get("bin_matrix", 0.0)

    # Timed rounds on the resident, quantized matrix (no profiling brackets).
    _, elapsed = time_rounds(xgb, dtrain, args.steps, profile=False)
    ms_per_step = elapsed * 1e3 / args.steps
    value = ms_per_step * 100

    # Same rounds with HIP-event brackets per kernel class (the roofline source).
    import ctypes
    import device_lib as D
    D.lib().mgb_profile_reset()
    bst_p, elapsed_p = time_rounds(xgb, dtrain, args.steps, profile=True)
    prof = bst_p.profile()
    kernels = prof["kernels"]
    hist = kernels["histogram"]
    hist_ms = hist["ms"]
    launches = max(hist["launches"], 1)
    hist_bytes = prof["histogram_bytes"]  # every profiled round, as are the kernel times
    achieved = hist_bytes / (hist_ms * 1e-3) / 1e9 if hist_ms > 0 else 0.0
    rounds_p = args.steps + 1
    breakdown = {k: round(v["ms"] / rounds_p, 4) for k, v in kernels.items() if v["launches"]}

    # Whole xgb.train from host arrays (fresh DMatrix: H2D copy, sketch, bins, 100 rounds).
    t0 = time.perf_counter()
    d2 = xgb.DMatrix(X, label=y)
    fit = xgb.train(dict(PARAMS), d2, 100)
    fit_ms = (time.perf_counter() - t0) * 1e3
    fit_pred = fit.predict(d2)

    copy_gbps = stream_copy_gbps()
    traffic = None
    traffic_file = ROOT / "profiles" / "histogram_traffic_config2.json"
    if traffic_file.exists():
        try:
            traffic = json.loads(traffic_file.read_text()).get("hbm_bytes_per_launch")
        except ValueError:
            traffic = None

    line = {
        "metric": "ms/100 rounds @262,144x64 d8; histogram build HBM GB/s vs peak",
        "value": round(value, 3),
        "unit": "ms/100 rounds",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(value / REFERENCE_MS_100, 4),
        "dtype": "int64",
        "data": "synthetic",
        "config": {"workload": "BASELINE config 2: X 262144x64 N(0,1), y = X.w + 0.5 sin(x0 x1) + 0.1 N (seed 1337); "
                               "reg:squarederror, depth 8, max_bin 256, eta 0.3, lambda 1; step = one boosting "
                               "round on the device-resident u8 bin matrix",
                   "rows": 262144, "features": 64, "max_depth": 8, "max_bin": 256,
                   "vs_baseline_reference": "222.8 ms, reference Metal engine on M5 Ultra, same shape and "
                                            "parameters, its own label generator (README.md:101)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": "k_histogram", "launches": launches,
                     "algorithmic_bytes_per_launch": round(hist_bytes / launches),
                     "avg_launch_us": round(hist_ms * 1e3 / launches, 3)},
        "kernel_ms_per_round": breakdown,
        "profiled_ms_per_100_rounds": round(elapsed_p * 1e3 / args.steps * 100, 3),
        "fit_ms_100_rounds_from_host": round(fit_ms, 2),
        "one_time_ms": {"quantile_sketch": round(sketch_s * 1e3, 2), "bin_matrix": round(bins_s * 1e3, 2)},
        "stream_copy_GBps": round(copy_gbps, 1),
        "fit_prediction_sha256": hashlib.sha256(fit_pred.tobytes()).hexdigest(),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(X, y, args.cpu_seconds)
    print(json.dumps(line))


C3_PARAMS = {"objective": "binary:logistic", "tree_method": "hist", "max_depth": 8, "max_bin": 256, "eta": 0.1}

LARGE = {
    "c3": dict(rounds=100, params=C3_PARAMS,
               metric="ms/100 rounds @1,000,000x2,000 CSR, 20 nonzeros/row, d8 (config 3); histogram build GB/s vs peak",
               workload="BASELINE config 3: CSR 1,000,000x2,000 with 20 distinct uniform columns per row, "
                        "lognormal(0,1) values, logistic labels from 200 informative columns (seed 1337); "
                        "binary:logistic, depth 8, max_bin 256, eta 0.1; step = one boosting round on the resident "
                        "per-nonzero codes (atomics histogram, missing slots from node totals)",
               shape={"rows": 1_000_000, "features": 2000, "nonzeros_per_row": 20, "max_depth": 8, "max_bin": 256}),
    "c4": dict(rounds=200, params=C4_PARAMS,
               metric="ms/200 rounds @10,000,000x128 d10 1024 bins (config 4); histogram build HBM GB/s vs peak",
               workload="BASELINE config 4: X 10,000,000x128 (N(0,1) | U(0,1) | integers 0-999), logistic "
                        "labels; binary:logistic, depth 10, max_bin 1024 (u16 codes), eta 0.1, subsample 0.8, "
                        "colsample_bytree 0.8; step = one boosting round on the resident bin matrix",
               shape={"rows": 10_000_000, "features": 128, "max_depth": 10, "max_bin": 1024}),
}


def bench_large(xgb, args, which):
    """Configs 3 and 4: one GPU, timed rounds on the resident quantized matrix
    (the other configs' workloads; the headline metric is config 2)."""
    spec = LARGE[which]
    steps = args.steps if args.steps != 100 else 20
    warmup = args.warmup if args.warmup != 10 else 2
    t0 = time.perf_counter()
    if which == "c4":
        X, y = config4()
    else:
        import scipy.sparse as sp
        import workloads as W
        indptr, indices, values, y = W.config3()
        X = sp.csr_matrix((values, indices, indptr), shape=(len(indptr) - 1, 2000))
    gen_s = time.perf_counter() - t0
    print(f"{which}: generated {X.shape} in {gen_s:.1f} s", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    dtrain = xgb.DMatrix(X, label=y)
    print(f"{which}: DMatrix in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    warm = xgb.train(dict(spec["params"]), dtrain, max(1, warmup))
    setup_s = time.perf_counter() - t0
    print(f"{which}: sketch, bins and {warmup} warm-up rounds in {setup_s:.1f} s", file=sys.stderr, flush=True)
    prof0 = warm.profile()["seconds"]
    _, elapsed = time_rounds(xgb, dtrain, steps, profile=False, base=spec["params"])
    ms_per_step = elapsed * 1e3 / steps
    print(f"{which}: {steps} timed rounds, {ms_per_step:.2f} ms each", file=sys.stderr, flush=True)
    import device_lib as D
    D.lib().mgb_profile_reset()
    bst_p, _ = time_rounds(xgb, dtrain, steps, profile=True, base=spec["params"])
    prof = bst_p.profile()
    kernels = prof["kernels"]
    hist = kernels["histogram"]
    launches = max(hist["launches"], 1)
    achieved = prof["histogram_bytes"] / (hist["ms"] * 1e-3) / 1e9 if hist["ms"] > 0 else 0.0
    rounds = spec["rounds"]
    traffic = None
    tfile = ROOT / "profiles" / f"histogram_traffic_config{which[1]}.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
    line = {
        "metric": spec["metric"], "value": round(ms_per_step * rounds, 2), "unit": f"ms/{rounds} rounds",
        "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "int64", "data": "synthetic",
        "config": dict({"workload": spec["workload"]}, **spec["shape"]),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": "k_histogram" if which == "c4" else "k_histogram_csr (+ k_zero_built, k_root_totals)",
                     "launches": launches, "algorithmic_bytes_per_launch": round(prof["histogram_bytes"] / launches),
                     "avg_launch_us": round(hist["ms"] * 1e3 / launches, 3)},
        "kernel_ms_per_round": {k: round(v["ms"] / (steps + 1), 4) for k, v in kernels.items() if v["launches"]},
        "one_time_s": {"generate": round(gen_s, 2), "dmatrix_sketch_bins_and_warmup": round(setup_s, 2),
                       "quantile_sketch": round(prof0.get("quantiles", 0.0), 3),
                       "bin_matrix": round(prof0.get("bin_matrix", 0.0), 3)},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
