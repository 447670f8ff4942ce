#!/usr/bin/env python3
"""Benchmark of the MI355X hist engine on BASELINE.json's metric.

Metric: ms per 100 boosting rounds at 262,144 x 64, depth 8,
plus histogram-build throughput against MI355X's 8 TB/s HBM peak.

Protocol (the reference's benchmarks/controlled_comparison.py:82-92, with the
median of three fresh-process fits): a step is one fit = xgb.train of 100 rounds on a DMatrix built
outside the timer (its values and labels already copied to the GPU), so the
lazy quantile sketch, bin matrix and base score are inside it; the booster's
rounds are drained (trees copied back) before the clock stops.  Fits run in
three fresh child processes (subprocess, never exec), each warmed up first with
3 rounds on a 16,384-row slice (the reference's GPU protocol); value = median
fit time.  The steady-state round time on an already quantized matrix is
reported beside it.  One more process times the reference's own 262,144 x 64
workload (the data its published 222.8 ms is quoted on) and checks that its
predictions are stock XGBoost's published SHA-256; --config c0 / c1 run the
same protocol on the reference's 100,000 x 32 d6 workloads (published 107.4 /
111.2 ms), also against their published SHA-256s.

The roofline object covers the histogram kernel: algorithmic bytes per launch
(rows built x (F code bytes + 4-byte row id + 8-byte gradient pair) + nodes
built x F x (max_bin+1) x 16 bytes of int64 histogram output) divided by the
kernel's duration, measured with HIP events on the library's stream; the
split kernel's bytes (parent and built histograms read, sibling written) and
the partition's (per row of a splitting node its id, gradient pair and split
code read and id and pair written; a stopping node's rows their id and
margin) are reported the same way.  cpu_baseline trains the CPU oracle (a
port of the reference's algorithm, OpenMP over features) for the same 100
rounds on the host cores, and its predictions are compared with the GPU fit's
bit for bit.  The default run also times config 3 (1M x 2000 CSR) and config
4 (10M x 128, 1024 bins, the HBM-bound workload), each in one more fresh
process, and reports them under "c3" and "c4".
"""
import argparse
import hashlib
import json
import os
import statistics
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "xgboost-metal_amd" / "python"))
sys.path.insert(0, str(ROOT / "tests"))

HBM_PEAK_GBPS = 8000.0
REFERENCE_MS_100 = 222.8  # the reference's published time: Metal engine, 262,144x64 d8, 100 rounds, M5 Ultra


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


def _known(case):
    import workloads as W
    return W.known_answer_data(case)


# Workloads timed on the fit protocol.  c2 is the headline (BASELINE config 2's
# generator); ref262, c0 and c1 are the reference's own published workloads
# (benchmarks/controlled_comparison.py:68-72: seed 1337, y = 2 x0 + x1^2 +
# 0.1 N), whose stock-XGBoost prediction SHA-256s the fits must reproduce, with
# the reference's published times beside them (README.md:98-104).
PROTOCOL = {
    "c2": dict(data=lambda: config2(), depth=8, ref_ms=REFERENCE_MS_100, sha256=None,
               name="BASELINE config 2: X 262144x64 N(0,1), y = X.w + 0.5 sin(x0 x1) + 0.1 N (seed 1337); "
                    "reg:squarederror, depth 8, max_bin 256, eta 0.3, lambda 1"),
    "ref262": dict(data=lambda: _known("dense262"), depth=8, ref_ms=REFERENCE_MS_100, case="dense262",
                   name="the reference's 262,144x64 d8 workload (controlled_comparison.py: y = 2 x0 + x1^2 + 0.1 N, "
                        "seed 1337), max_bin 256, eta 0.3"),
    "c0": dict(data=lambda: _known("dense100"), depth=6, ref_ms=107.4, case="dense100",
               name="config 0 shape, the reference's 100,000x32 d6 workload (controlled_comparison.py: "
                    "y = 2 x0 + x1^2 + 0.1 N, seed 1337), max_bin 256, eta 0.3"),
    "c1": dict(data=lambda: _known("missing100"), depth=6, ref_ms=111.2, case="missing100",
               name="config 1 shape, the reference's 100,000x32 d6 workload with 15% NaN (controlled_comparison.py), "
                    "max_bin 256, eta 0.3"),
}


def protocol_params(which):
    return dict(PARAMS, max_depth=PROTOCOL[which]["depth"])


def published_sha256(which):
    case = PROTOCOL[which].get("case")
    if not case:
        return None
    import workloads as W
    return W.KNOWN_ANSWERS[case]["prediction_sha256"]


def config4(rows=10_000_000, seed=1337):
    """BASELINE config 4 (tests/workloads.py holds the generator)."""
    import workloads as W
    return W.config4(rows=rows, seed=seed)


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


def rooflines(prof, rounds):
    """Histogram, split and partition rooflines of profiled rounds: the
    algorithmic bytes the library counted on the device over the rounds
    divided by the kernel class's summed HIP-event time."""
    out = {}
    specs = [("roofline", "histogram", "histogram_bytes", "k_histogram"),
             ("split_roofline", "split", "split_bytes", "k_split"),
             ("partition_roofline", "partition", "partition_bytes",
              "k_apply (select + partition; with k_part_count and k_final_order under the stable partition)")]
    for key, kind, field, kernel in specs:
        k = prof["kernels"][kind]
        launches = max(k["launches"], 1)
        achieved = prof[field] / (k["ms"] * 1e-3) / 1e9 if k["ms"] > 0 else 0.0
        out[key] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBPS, 4), "kernel": kernel, "launches": launches,
                    "algorithmic_bytes_per_launch": round(prof[field] / launches),
                    "avg_launch_us": round(k["ms"] * 1e3 / launches, 3),
                    "ms_per_round": round(k["ms"] / max(rounds, 1), 4)}
        sampled = prof.get(field.replace("_bytes", "_bytes_sampled_features"))
        if sampled is not None and sampled != prof[field] and k["ms"] > 0:
            # With colsample_bytree the kernels touch only the sampled
            # features; the bytes above count every feature (F in
            # R_built·(F·s + 12) + N_built·F·(B+1)·16), these only the
            # sampled ones.
            a = sampled / (k["ms"] * 1e-3) / 1e9
            out[key]["sampled_features"] = {"algorithmic_bytes_per_launch": round(sampled / launches),
                                            "achieved": round(a, 1), "frac": round(a / HBM_PEAK_GBPS, 4)}
    return out


def committed_traffic(which):
    """HBM bytes per launch of each kernel class for this workload, from the
    committed counter passes (FETCH_SIZE and WRITE_SIZE, calibrated by a copy
    kernel of known size); None where no pass is committed."""
    out = {"histogram": None, "split": None, "partition": None}
    path = ROOT / "profiles" / f"tree_traffic_config{which[1]}.json"
    if path.exists():
        try:
            data = json.loads(path.read_text())
            for k in out:
                out[k] = data.get(k, {}).get("hbm_bytes_per_launch")
        except ValueError:
            pass
    return out


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


def cpu_threads():
    """Host threads for the CPU leg: OMP_NUM_THREADS when set (the GPU box sets
    it to its per-GPU CPU share, 16), else every core."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)


def cpu_baseline(X, y, rounds=100, which="c2"):
    """The CPU oracle trained for the same rounds as one GPU fit (its own
    one-time sketch included); returns the baseline object and its margins."""
    import oracle_lib as O
    threads = cpu_threads()
    depth = PROTOCOL[which]["depth"]
    p = O.make_params(max_depth=depth, max_bin=256, eta=0.3, nthread=threads)
    t0 = time.perf_counter()
    ref = O.train(X, y, p, rounds)
    seconds = time.perf_counter() - t0
    return ({"value": round(seconds * 1e3 * 100 / rounds, 1), "unit": "ms/100 rounds", "cores": threads,
             "host_cpu_count": os.cpu_count(), "kind": "port",
             "sample": f"CPU oracle (C restatement of the reference's hist path; histograms and split search "
                       f"OpenMP-parallel over features) on the "
                       f"same {X.shape[0]}x{X.shape[1]} d{depth} matrix, one fit of {rounds} rounds including its "
                       f"sketch, {threads} threads ({seconds:.1f} s)"}, ref["margin"])


def fit_child(args):
    """One fresh process: warm-up, then args.fits timed fits; prints one JSON line."""
    import xgboost as xgb
    import device_lib as D
    X, y = PROTOCOL[args.workload]["data"]()
    params = protocol_params(args.workload)
    for _ in range(max(1, args.warmup)):
        warm = xgb.DMatrix(X[:16384], label=y[:16384])
        xgb.train(dict(params), warm, 3).predict(warm)
    times, one_time = [], {}
    bst = d = None
    for _ in range(args.fits):
        d = xgb.DMatrix(X, label=y).to_device()  # outside the timer: host-to-device copy
        D.check(D.lib().mgb_synchronize())
        t0 = time.perf_counter()
        bst = xgb.train(dict(params), d, 100)
        bst.num_boosted_rounds()  # waits for the queued rounds and copies the trees back
        D.check(D.lib().mgb_synchronize())
        times.append((time.perf_counter() - t0) * 1e3)
        one_time = bst.profile()["seconds"]
    pred = bst.predict(d)
    np.save(args.pred_out, pred)
    print(json.dumps({"fit_ms": times, "prediction_sha256": hashlib.sha256(pred.tobytes()).hexdigest(),
                      "quantile_sketch_ms": one_time.get("quantiles", 0.0) * 1e3,
                      "bin_matrix_ms": one_time.get("bin_matrix", 0.0) * 1e3}))


def run_child(fits, warmup, pred_out, extra_params=(), workload="c2"):
    cmd = [sys.executable, str(Path(__file__).resolve()), "--child", "--fits", str(fits), "--warmup", str(warmup),
           "--pred-out", str(pred_out), "--workload", workload]
    for item in extra_params:
        cmd += ["--param", item]
    out = subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=900)
    return json.loads(out.stdout.strip().splitlines()[-1])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=9,
                    help="timed fits (100 rounds each, quantization included), spread over 3 fresh processes")
    ap.add_argument("--warmup", type=int, default=1, help="warm-up fits (3 rounds, 16,384 rows) per process")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--config", choices=["c2", "c0", "c1", "c3", "c4"], default="c2",
                    help="c2 (default): the headline metric; c0/c1: the fit protocol on the reference's "
                         "100,000 x 32 d6 workloads (dense / 15%% missing); c3: 1M x 2000 CSR, 20 nonzeros a row; "
                         "c4: 10M x 128, 1024 bins, depth 10 (HBM-bound check)")
    ap.add_argument("--no-ref", action="store_true",
                    help="c2: skip the extra process timing the reference's own 262,144 x 64 workload")
    ap.add_argument("--no-c3", action="store_true",
                    help="c2: skip the extra process timing config 3 (1M x 2000 CSR, depth 8)")
    ap.add_argument("--no-c4", action="store_true",
                    help="c2: skip the extra process timing config 4 (10M x 128, 1024 bins, depth 10)")
    ap.add_argument("--param", action="append", default=[], metavar="KEY=VALUE",
                    help="extra booster parameter for the timed rounds (repeatable), e.g. hip_histogram_rows=2048")
    ap.add_argument("--child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--fits", type=int, default=1, help=argparse.SUPPRESS)
    ap.add_argument("--pred-out", default="", help=argparse.SUPPRESS)
    ap.add_argument("--workload", default="c2", choices=sorted(PROTOCOL), help=argparse.SUPPRESS)
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
    if args.child:
        return fit_child(args)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(row-sharded multi-GPU training is a design note, not implemented).", file=sys.stderr)
        sys.exit(2)
    if args.config in LARGE:
        import xgboost as xgb
        return bench_large(xgb, args, args.config)

    # Protocol fits in three fresh processes, the CPU leg between the first two.
    which = args.config
    spec = PROTOCOL[which]
    params = protocol_params(which)
    steps = max(1, args.steps)
    shares = [steps // 3 + (1 if i < steps % 3 else 0) for i in range(3)]
    shares = [n for n in shares if n]
    X, y = spec["data"]()
    tmp = Path(tempfile.mkdtemp(prefix="bench_"))
    children, cpu, cpu_margin = [], None, None
    for i, n in enumerate(shares):
        children.append(run_child(n, args.warmup, tmp / f"pred{i}.npy", args.param, which))
        print(f"bench: process {i + 1}: fits {[round(t, 2) for t in children[-1]['fit_ms']]} ms", file=sys.stderr,
              flush=True)
        if i == 0 and not args.no_cpu:
            cpu, cpu_margin = cpu_baseline(X, y, 100, which)
            print(f"bench: CPU oracle {cpu['value']} ms/100 rounds on {cpu['cores']} threads", file=sys.stderr,
                  flush=True)
    fits = [t for c in children for t in c["fit_ms"]]
    value = statistics.median(fits)
    gpu_pred = np.load(tmp / "pred0.npy")
    same_across = len({c["prediction_sha256"] for c in children}) == 1
    reference_workload = None
    if which == "c2" and not args.no_ref:
        # The reference's own 262,144 x 64 workload, the one its 222.8 ms is
        # quoted on, in one more fresh process: its fits and whether the
        # predictions are stock XGBoost's published ones.
        ref = run_child(3, args.warmup, tmp / "pred_ref.npy", args.param, "ref262")
        print(f"bench: reference workload: fits {[round(t, 2) for t in ref['fit_ms']]} ms", file=sys.stderr,
              flush=True)
        reference_workload = {"workload": PROTOCOL["ref262"]["name"], "fits_ms": [round(t, 3) for t in ref["fit_ms"]],
                              "median_ms": round(statistics.median(ref["fit_ms"]), 3),
                              "vs_reference_222_8_ms": round(statistics.median(ref["fit_ms"]) / REFERENCE_MS_100, 4),
                              "prediction_sha256": ref["prediction_sha256"],
                              "equals_published_stock_xgboost_sha256":
                                  ref["prediction_sha256"] == published_sha256("ref262")}

    import xgboost as xgb
    dtrain = xgb.DMatrix(X, label=y)
    xgb.train(dict(params), dtrain, 3)  # this process: code loading, sketch and bins (untimed)

    # Steady state: rounds on the resident, quantized matrix (no profiling brackets).
    _, elapsed = time_rounds(xgb, dtrain, 100, profile=False, base=params)
    steady_ms = elapsed * 1e3

    # Same rounds with HIP-event brackets per kernel class (the roofline source).
    import device_lib as D
    D.lib().mgb_profile_reset()
    bst_p, elapsed_p = time_rounds(xgb, dtrain, 100, profile=True, base=params)
    prof = bst_p.profile()
    kernels = prof["kernels"]
    roof = rooflines(prof, 101)
    breakdown = {k: round(v["ms"] / 101, 4) for k, v in kernels.items() if v["launches"]}

    copy_gbps = stream_copy_gbps()
    traffic = committed_traffic(which)

    rows, cols = X.shape
    depth = spec["depth"]
    line = {
        "metric": f"ms/100 rounds @{rows:,}x{cols} d{depth}; histogram build HBM GB/s vs peak",
        "value": round(value, 3),
        "unit": "ms/100 rounds",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(value, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(value / spec["ref_ms"], 4),
        "dtype": "int64",
        "data": "synthetic",
        "config": {"workload": spec["name"] + "; step = one fit: xgb.train of 100 rounds (quantile sketch, bin matrix "
                               "and base score included) on a DMatrix already on the GPU, in a fresh process after a "
                               "warm-up (benchmarks/controlled_comparison.py:82-92); value = median over steps",
                   "rows": rows, "features": cols, "max_depth": depth, "max_bin": 256,
                   "vs_baseline_reference": f"{spec['ref_ms']} ms, reference Metal engine on M5 Ultra, same shape and "
                                            f"parameters and the same protocol"
                                            + (", its own label generator (README.md:101)" if which == "c2" else
                                               ", the same workload (README.md:98-104)")},
        "roofline": dict(roof["roofline"], traffic=traffic["histogram"]),
        "split_roofline": dict(roof["split_roofline"], traffic=traffic["split"]),
        "partition_roofline": dict(roof["partition_roofline"], traffic=traffic["partition"]),
        "fits_ms": [round(t, 3) for t in fits],
        "process_median_ms": [round(statistics.median(c["fit_ms"]), 3) for c in children],
        "steady_state_ms_per_100_rounds": round(steady_ms, 3),
        "kernel_ms_per_round": breakdown,
        "profiled_ms_per_100_rounds": round(elapsed_p * 1e3, 3),
        "one_time_ms": {"quantile_sketch": round(children[0]["quantile_sketch_ms"], 3),
                        "bin_matrix": round(children[0]["bin_matrix_ms"], 3)},
        "stream_copy_GBps": round(copy_gbps, 1),
        "parity": {"prediction_sha256": children[0]["prediction_sha256"],
                   "identical_across_processes": same_across},
    }
    if published_sha256(which):
        line["parity"]["equals_published_stock_xgboost_sha256"] = \
            children[0]["prediction_sha256"] == published_sha256(which)
    if reference_workload is not None:
        line["reference_workload"] = reference_workload
    if which == "c2" and not args.no_c3:
        line["c3"] = run_large_child("c3", args.param)
    if which == "c2" and not args.no_c4:
        line["c4"] = run_large_child("c4", args.param)
    if cpu is not None:
        line["cpu_baseline"] = cpu
        line["parity"]["equal_to_cpu_oracle_bitwise"] = bool(
            np.array_equal(gpu_pred.view(np.uint32), cpu_margin.view(np.uint32)))
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


def run_large_child(which, extra_params=()):
    """Config 3 or 4 in one more fresh process (subprocess, never exec): its
    own generator, 2 warm-up rounds, 20 timed steady-state rounds; a failure
    gives {"error": ...} instead of the object and leaves the config-2 line
    intact."""
    cmd = [sys.executable, str(Path(__file__).resolve()), "--config", which, "--steps", "20", "--warmup", "2"]
    for item in extra_params:
        cmd += ["--param", item]
    try:
        out = subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=420)
        res = json.loads(out.stdout.strip().splitlines()[-1])
    except (subprocess.SubprocessError, ValueError, IndexError) as e:
        return {"error": f"{type(e).__name__}: {str(e)[:300]}"}
    rounds = LARGE[which]["rounds"]
    print(f"bench: config {which[1]}: {res['value']} ms/{rounds} rounds, histogram {res['roofline']['frac']} of peak",
          file=sys.stderr, flush=True)
    keep = ("metric", "value", "unit", "steps", "warmup", "ms_per_step", "config", "roofline", "split_roofline",
            "partition_roofline", "kernel_ms_per_round", "one_time_s")
    return dict({k: res[k] for k in keep if k in res}, **{f"ms_per_{rounds}_rounds": res["value"]})


def bench_large(xgb, args, which):
    """Configs 3 and 4: one GPU, timed rounds on the resident quantized matrix
    (the other configs' workloads; the headline metric is config 2)."""
    spec = LARGE[which]
    steps = args.steps if args.steps != 9 else 20
    warmup = args.warmup if args.warmup != 1 else 2
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
    roof = rooflines(prof, steps + 1)
    rounds = spec["rounds"]
    traffic = committed_traffic(which)
    line = {
        "metric": spec["metric"], "value": round(ms_per_step * rounds, 2), "unit": f"ms/{rounds} rounds",
        "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "int64", "data": "synthetic",
        "config": dict({"workload": spec["workload"]}, **spec["shape"]),
        "roofline": dict(roof["roofline"], traffic=traffic["histogram"],
                         kernel="k_histogram" if which == "c4" else "k_histogram_csr (+ k_zero_built, k_root_totals)"),
        "split_roofline": dict(roof["split_roofline"], traffic=traffic["split"]),
        "partition_roofline": dict(roof["partition_roofline"], traffic=traffic["partition"]),
        "kernel_ms_per_round": {k: round(v["ms"] / (steps + 1), 4) for k, v in kernels.items() if v["launches"]},
        "one_time_s": {"generate": round(gen_s, 2), "dmatrix_sketch_bins_and_warmup": round(setup_s, 2),
                       "quantile_sketch": round(prof0.get("quantiles", 0.0), 3),
                       "bin_matrix": round(prof0.get("bin_matrix", 0.0), 3)},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
