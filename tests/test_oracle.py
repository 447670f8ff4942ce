"""Pins the CPU oracle (oracle/hist_oracle.c) before it is trusted as the checker.

- End to end: the reference's published prediction SHA-256s of stock XGBoost
  3.4.1 CPU hist on its seed-1337 workloads.
- Sketch/bins: closed forms for columns with few distinct values, invariants
  otherwise, and the rank/budget rule of the sketch.
- Quantization scale: arbitrary-precision integer arithmetic.
- Scoring: exact-rational constructions that separate RN32(RN64(G/H)) from
  RN32(G/H) (construction of the reference's tests/test_scalar_weight.py:29-71).
- Trees: the constructed known answer of tests/test_histogram_present.py:66-81.
"""
import hashlib
from fractions import Fraction

import numpy as np
import pytest

import oracle_lib as O
import workloads as W


@pytest.mark.parametrize("case", ["dense100", "missing100",
                                  pytest.param("dense262", marks=pytest.mark.slow)])
def test_published_prediction_hashes(case):
    spec = W.KNOWN_ANSWERS[case]
    X, y = W.known_answer_data(case)
    if "input_sha256" in spec:
        assert hashlib.sha256(X.tobytes()).hexdigest() == spec["input_sha256"]
        assert hashlib.sha256(y.tobytes()).hexdigest() == spec["label_sha256"]
    r = O.train(X, y, O.make_params(max_depth=spec["depth"], max_bin=256, eta=0.3), 100)
    pred = r["margin"]
    assert hashlib.sha256(pred.tobytes()).hexdigest() == spec["prediction_sha256"]
    rmse = float(np.sqrt(np.mean((pred.astype(np.float64) - y) ** 2)))
    assert abs(rmse - spec["rmse"]) < 1e-12
    # Traversal prediction of the stored trees equals the training margin.
    again = O.predict_margin(X, r, r["base_score"])
    np.testing.assert_array_equal(again.view(np.uint32), pred.view(np.uint32))


def test_planted_mistake_breaks_known_answer():
    """The known answer is sensitive: a one-ulp change of eta changes the hash."""
    spec = W.KNOWN_ANSWERS["dense100"]
    X, y = W.known_answer_data("dense100")
    eta = float(np.nextafter(np.float32(0.3), np.float32(1)))
    r = O.train(X[:20000], y[:20000], O.make_params(max_depth=6, max_bin=256, eta=eta), 5)
    base = O.train(X[:20000], y[:20000], O.make_params(max_depth=6, max_bin=256, eta=0.3), 5)
    assert not np.array_equal(r["margin"], base["margin"])
    assert hashlib.sha256(base["margin"].tobytes()).hexdigest() != spec["prediction_sha256"]


def test_sketch_budget_rule():
    # limit = min(count, ceil(level * 2 * min(bins, count)) + 1) for the first level with 2^level*limit >= count.
    def budget(bins, count):
        if not count:
            return 1
        n = min(bins, count)
        for level in range(1, 32):
            limit = min(count, level * 2 * n + 1)
            if (1 << level) * limit >= count:
                return limit
        return count
    for bins, count in [(256, 100000), (256, 262144), (1024, 10_000_000), (4, 3), (256, 1), (16, 1000)]:
        assert O.lib().oracle_sketch_budget(bins, count) == budget(bins, count)
    assert O.lib().oracle_sketch_budget(256, 100000) == 3073


def test_cuts_closed_form_few_distinct():
    # At most max_bin distinct values: cuts are the distinct values after the
    # first, then max + (|max| + 1e-5).
    rng = np.random.default_rng(0)
    values = np.asarray([-3.5, -1.0, 0.0, 0.25, 2.0, 7.0], np.float32)
    X = rng.choice(values, size=(5000, 3)).astype(np.float32)
    X[:, 2] = 4.0
    cuts, counts, minima = O.sketch_cuts(X, 16)
    for f in range(2):
        d = np.unique(X[:, f])
        want = np.append(d[1:], np.float32(d[-1] + (np.abs(d[-1]) + np.float32(1e-5))))
        assert counts[f] == len(want)
        np.testing.assert_array_equal(cuts[f, :counts[f]], want)
    assert counts[2] == 1 and cuts[2, 0] == np.float32(4.0) + np.float32(4.0 + 1e-5)
    assert np.all(np.isneginf(minima))


def test_cuts_invariants_and_bins():
    X, _ = W.config1(rows=50000, cols=6)
    X[:, 1] = np.round(X[:, 1])
    for max_bin in [4, 64, 256, 1024]:
        cuts, counts, _ = O.sketch_cuts(X, max_bin)
        bins = O.quantize(X, cuts, counts)
        for f in range(X.shape[1]):
            c = cuts[f, :counts[f]]
            assert 1 <= counts[f] <= max_bin
            assert np.all(np.diff(c) > 0), "strictly increasing"
            col = X[:, f]
            present = ~np.isnan(col)
            assert c[-1] > np.nanmax(col)
            # bin = min(upper_bound(cuts, v), count - 1); NaN -> missing.
            want = np.minimum(np.searchsorted(c, col[present], side="right"), counts[f] - 1)
            np.testing.assert_array_equal(bins[present, f], want)
            assert np.all(bins[~present, f] == 0xFFFF)
        # Equal-frequency property: every bin of a continuous feature holds a
        # share close to 1/count (the sketch's rank error bound is ~1/max_bin).
        b0 = bins[~np.isnan(X[:, 0]), 0]
        share = np.bincount(b0, minlength=counts[0]) / len(b0)
        assert share.max() < 3.0 / counts[0] + 0.01


def _scale_reference(values):
    total = sum(abs(Fraction(float(v))) for v in values) * (2 ** 149)
    assert total.denominator == 1
    bitlen = int(total).bit_length()
    exponent = max(0, bitlen - 149)
    return 2.0 ** (62 - exponent)


@pytest.mark.parametrize("values", [
    [1.0, -2.0, 3.5],
    [np.finfo(np.float32).max] * 257,
    [2.0 ** -149, 2.0 ** -149, 1e-40],
    [0.0, -0.0],
    list(np.random.default_rng(1).normal(size=5000).astype(np.float32)),
    [2.0 ** 16, -(2.0 ** 16), 6.118193027759844e-7],
])
def test_gradient_scale_exact(values):
    v = np.asarray(values, np.float32)
    assert O.gradient_scale(v) == _scale_reference(v)


def test_histogram_brute_force():
    rng = np.random.default_rng(2)
    X, _ = W.config1(rows=3000, cols=5)
    cuts, counts, _ = O.sketch_cuts(X, 32)
    bins = O.quantize(X, cuts, counts)
    g = rng.normal(size=len(X)).astype(np.float32)
    h = rng.uniform(0, 1, size=len(X)).astype(np.float32)
    sg, sh = O.gradient_scale(g), O.gradient_scale(h)
    qg = np.rint(g * np.float32(sg)).astype(np.int64)
    qh = np.rint(h * np.float32(sh)).astype(np.int64)
    rows = np.sort(rng.choice(len(X), 1000, replace=False)).astype(np.uint32)
    hist = np.zeros((5, 33, 2), np.int64)
    import ctypes
    O.lib().oracle_histogram(O.ptr(bins), ctypes.c_uint32(5), ctypes.c_uint32(32), O.ptr(rows),
                             ctypes.c_uint32(len(rows)), O.ptr(qg), O.ptr(qh), O.ptr(hist))
    for f in range(5):
        for b in range(33):
            sel = rows[(np.where(bins[rows, f] == 0xFFFF, 32, bins[rows, f]) == b)]
            assert hist[f, b, 0] == int(qg[sel].sum())
            assert hist[f, b, 1] == int(qh[sel].sum())
    # Invariant: each feature's bins (with missing) sum to the node total.
    np.testing.assert_array_equal(hist[:, :, 0].sum(axis=1), np.full(5, qg[rows].sum()))


def _float32_parts(value):
    """Nonnegative binary32 values summing exactly to an integer."""
    parts = []
    while value:
        part = np.float32(value)
        if int(part) > value:
            part = np.nextafter(part, np.float32(0))
        parts.append(part)
        value -= int(part)
    return parts


def _double_rounding_case(parity, inside_cell):
    # Choose an exact quotient N/D just across a binary32 midpoint from its
    # round-to-nearest-even side, so that RN32(RN64(N/D)) differs from
    # RN32(N/D) exactly when the binary64 rounding lands on the midpoint.
    q = 2 ** 23 + parity
    delta = (1 if parity == 0 else -1) * (2 ** 23 + (-1 if inside_cell else 1))
    modulus = 2 ** 24
    denominator = 2 ** 52 + (-delta * pow(2 * q + 1, -1, modulus)) % modulus
    numerator, remainder = divmod((2 * q + 1) * denominator + delta, modulus)
    assert remainder == 0
    return numerator, denominator


@pytest.mark.parametrize("sign", [-1, 1])
@pytest.mark.parametrize("parity", [0, 1])
@pytest.mark.parametrize("inside_cell", [False, True])
@pytest.mark.parametrize("split", [False, True])
def test_weight_double_rounding(sign, parity, inside_cell, split):
    numerator, denominator = _double_rounding_case(parity, inside_cell)
    exact = Fraction(numerator, denominator)
    double_rounded = np.float32(numerator / denominator)
    direct = np.float32(float(min([Fraction(2 ** 23 + parity, 2 ** 23), Fraction(2 ** 23 + parity + 1, 2 ** 23)],
                                  key=lambda e: abs(exact - e))))
    assert (double_rounded != direct) == inside_cell
    g = _float32_parts(numerator)
    h = _float32_parts(denominator)
    rows = max(len(g), len(h))
    grad = np.asarray(g + [0] * (rows - len(g)), np.float32) * -sign
    hess = np.asarray(h + [0] * (rows - len(h)), np.float32)
    X = np.zeros((rows + int(split), 1), np.float32)
    if split:
        X[-1, 0] = 1
        grad = np.append(grad, np.float32(0))
        hess = np.append(hess, np.float32(2 ** 52))
    p = O.make_params(max_depth=1, max_bin=4, eta=1.0, reg_lambda=0.0, min_child_weight=0.0, base_score=0.0)
    r = O.train(X, np.zeros(len(X), np.float32), p, 1, custom_grad=grad[None, :], custom_hess=hess[None, :])
    tree = r["trees"][0][:r["sizes"][0]]
    assert len(tree) == (3 if split else 1)
    got = np.float32(tree["base_weight"][1 if split else 0])
    assert got.view(np.uint32) == np.float32(sign * double_rounded).view(np.uint32)


def test_constructed_tree_known_answer():
    """Leaf base weights [1, 3, -1, -3] (tests/test_histogram_present.py:66-81 of the reference)."""
    X = np.repeat(np.asarray([[0, 0, np.nan], [0, 1, np.nan], [1, 0, np.nan], [1, 1, np.nan]], np.float32), 3, axis=0)
    grad = np.asarray([[2.0 ** 40, -(2.0 ** 40), f] for f in [-1, -3, 1, 3]], np.float32).ravel()
    hess = np.tile(np.asarray([-1, 1, 1], np.float32), 4)
    p = O.make_params(max_depth=3, max_bin=4, eta=1.0, reg_lambda=0.0, min_child_weight=0.0, base_score=0.5)
    r = O.train(X, np.zeros(len(X), np.float32), p, 1, custom_grad=grad[None, :], custom_hess=hess[None, :])
    tree = r["trees"][0][:r["sizes"][0]]
    assert len(tree) == 7
    np.testing.assert_array_equal(tree["base_weight"][3:], np.asarray([1, 3, -1, -3], np.float32))


def test_gain_forms_closed_form():
    """w = RN32(RN64(-G/(H+lambda))); gain = RN32(-(2 G w + (H+lambda) RN32(w^2))) with
    the products fused (fma_contract=1) or separately rounded (fma_contract=0)."""
    rng = np.random.default_rng(9)
    for fma in (0, 1):
        p = O.make_params(reg_lambda=1.0, fma_contract=fma)
        for _ in range(200):
            G = float(rng.normal() * 1e3)
            H = float(rng.uniform(0.5, 1e3))
            w = O.lib().oracle_weight(G, H, p)
            assert np.float32(w) == np.float32(-G / (H + 1.0))
            gain = O.lib().oracle_gain(G, H, w, p)
            sq = float(np.float32(w) * np.float32(w))
            exact = Fraction(2) * Fraction(G) * Fraction(float(np.float32(w))) + Fraction(H + 1.0) * Fraction(sq)
            if fma:
                quad = (H + 1.0) * sq
                want = np.float32(-float(Fraction(2 * G) * Fraction(float(np.float32(w))) + Fraction(quad)))
            else:
                want = np.float32(-((2 * G) * float(np.float32(w)) + (H + 1.0) * sq))
            assert np.float32(gain) == want
            assert abs(float(np.float32(gain)) + float(exact)) <= 1e-6 * abs(float(exact)) + 1e-30


# ---------------------------------------------------------------------------
# Sampling (src/sampling.cpp:11-74, kernels/sampling.metal.h:1-30,
# src/tree.cpp:28-45).
# ---------------------------------------------------------------------------
def _mt_standard_state(seed):
    """std::mersenne_twister_engine::seed for mt19937 (the C++ standard's recurrence)."""
    key = np.zeros(624, np.uint32)
    key[0] = seed
    for i in range(1, 624):
        prev = int(key[i - 1])
        key[i] = (1812433253 * (prev ^ (prev >> 30)) + i) & 0xFFFFFFFF
    return key


def test_mt19937_standard_known_answer():
    """[rand.predef]: the 10000th output of a default-constructed std::mt19937 is 4123659995."""
    out = O.mt_outputs(5489, 10000)
    assert int(out[-1]) == 4123659995


@pytest.mark.parametrize("seed", [0, 1, 42, 123456789, 0xFFFFFFFF])
def test_mt19937_matches_numpy_generator(seed):
    """numpy's MT19937 bit generator, loaded with the standard-seeded state,
    is an independent implementation of the same twist and tempering."""
    bg = np.random.MT19937(0)
    bg.state = {"bit_generator": "MT19937", "state": {"key": _mt_standard_state(seed), "pos": 624}}
    want = np.array([bg.random_raw() for _ in range(1500)], np.uint64).astype(np.uint32)
    np.testing.assert_array_equal(O.mt_outputs(seed, 1500), want)


@pytest.mark.parametrize("seed,subsample", [(0, 0.8), (7, 0.5), (3737844653, 0.8), (99, 1e-3)])
def test_row_sampling_closed_form(seed, subsample):
    """state = seed * 16807^(row+1) mod 2^63 (seed 0 -> 1); keep iff the
    binary64 value of state-1, over 2^63, is below subsample (binary32)."""
    rows = 3000
    got = O.sample_rows(seed, rows, subsample)
    s = np.float32(subsample)
    limit = int(np.float64(s) * 2.0 ** 63)
    want = []
    for r in range(rows):
        state = ((seed or 1) * pow(16807, r + 1, 1 << 63)) % (1 << 63)
        want.append(float(state - 1) < limit)
    np.testing.assert_array_equal(got, np.array(want))
    if subsample >= 0.5:
        assert abs(got.mean() - subsample) < 0.05


def test_row_sampling_planted_mistake_is_caught():
    """Stepping the generator row times instead of row+1 changes the mask."""
    got = O.sample_rows(11, 2000, 0.5)
    wrong = np.array([float(((11 * pow(16807, r, 1 << 63)) % (1 << 63)) - 1) < 2.0 ** 62 for r in range(2000)])
    assert (got != wrong).any()


@pytest.mark.parametrize("n,fraction", [(128, 0.8), (64, 0.5), (7, 0.1), (1, 0.5), (33, 0.999)])
def test_column_sampling_invariants(n, fraction):
    """Sorted distinct features, max(1, floor(n * fraction)) of them, a
    deterministic function of the seed; different seeds give different sets.
    (The draw order itself is pinned by tests/test_shuffle.py.)"""
    keep = max(1, int(np.floor(np.float32(n) * np.float32(fraction))))
    a = O.sample_columns(n, fraction, 12345)
    assert len(a) == keep
    assert np.all(np.diff(a.astype(np.int64)) > 0) and a.max() < n
    np.testing.assert_array_equal(a, O.sample_columns(n, fraction, 12345))
    if 1 < keep < n:
        sets = {tuple(O.sample_columns(n, fraction, s)) for s in range(20)}
        assert len(sets) > 1


def test_sampled_training_drops_rows_and_features():
    """With subsample and colsample_bytree the oracle's trees only split on
    sampled features and differ from the unsampled trees; covers shrink to
    the sampled rows' Hessians."""
    X, y = W.config0(rows=6000, cols=12)
    full = O.train(X, y, O.make_params(max_depth=4, max_bin=64), 3)
    samp = O.train(X, y, O.make_params(max_depth=4, max_bin=64, subsample=0.7, colsample_bytree=0.5, seed=3), 3)
    assert samp["trees"][0]["cover"][0] < 0.8 * full["trees"][0]["cover"][0]
    # Reproduce the engine draws: round t uses draw 2t for rows, 2t+1 for columns.
    draws = O.mt_outputs(3, 6)
    for t in range(3):
        feats = set(O.sample_columns(12, 0.5, int(draws[2 * t + 1])).tolist())
        used = {int(f) for f in samp["trees"][t]["feature"][: samp["sizes"][t]] if f >= 0}
        assert used <= feats


@pytest.mark.parametrize("objective", ["reg:squarederror", "binary:logistic"])
def test_monotone_constraints_make_predictions_monotone(objective):
    """Monotone constraints (src/tree.cpp:15-26, 1083-1086; boost.metal:902-920):
    with +1 on x0 and -1 on x1, every prediction is non-decreasing in x0 and
    non-increasing in x1 with the other features held fixed, while the
    unconstrained model on the same data is not (so the check is not vacuous).
    A flipped sign, a missing clamp or a wrong midpoint fails one of these."""
    rng = np.random.default_rng(21)
    rows = 6000
    X = rng.normal(size=(rows, 4)).astype(np.float32)
    y = (np.sin(3 * X[:, 0]) + X[:, 0] - np.cos(3 * X[:, 1]) - X[:, 1] + 0.5 * X[:, 2]
         + 0.2 * rng.normal(size=rows)).astype(np.float32)
    if objective == "binary:logistic":
        y = (y > np.median(y)).astype(np.float32)
    kw = dict(objective=objective, max_depth=5, max_bin=64, eta=0.3)
    mono = O.train(X, y, O.make_params(monotone=[1, -1, 0, 0], **kw), 12)
    free = O.train(X, y, O.make_params(**kw), 12)
    grid = np.linspace(-2.5, 2.5, 101, dtype=np.float32)
    anchors = rng.normal(size=(20, 4)).astype(np.float32)

    def along(result, feature):
        out = []
        for a in anchors:
            P = np.repeat(a[None, :], len(grid), axis=0)
            P[:, feature] = grid
            out.append(O.predict_margin(P, result, 0.0).astype(np.float64))
        return np.asarray(out)

    d0, d1 = np.diff(along(mono, 0), axis=1), np.diff(along(mono, 1), axis=1)
    assert (d0 >= 0).all() and (d1 <= 0).all()
    f0, f1 = np.diff(along(free, 0), axis=1), np.diff(along(free, 1), axis=1)
    assert (f0 < 0).any() and (f1 > 0).any()
    # Unconstrained features keep splitting both ways, and an all-zero
    # constraint vector is the unconstrained model.
    zero = O.train(X, y, O.make_params(monotone=[0, 0, 0, 0], **kw), 12)
    np.testing.assert_array_equal(zero["trees"], free["trees"])


@pytest.mark.parametrize("fma", [1, 0])
def test_weighted_million_root_literal(fma):
    """The reference's literal 2915099116 (tests/test_scalar_root_statistics.py:
    66-80): weighted squared error over 1,000,000 dense rows, depth 1, 256
    bins.  The root's base weight comes from feature 0's bins summed in bin
    order in binary64; an exact (or row-order float64) sum of the same
    gradients gives 2915099417 and a float32 sum 2956438444, so the literal
    pins the ordered-bin rule, the weighted sketch and the base score."""
    X, y, weight = W.weighted_million()
    ref = O.train(X, y, O.make_params(max_depth=1, max_bin=256, seed=9, fma_contract=fma), 1, weights=weight)
    bits = int(np.float32(ref["trees"][0]["base_weight"][0]).view(np.uint32))
    assert bits == W.WEIGHTED_MILLION_ROOT_BITS


@pytest.mark.parametrize("fma", [1, 0])
def test_weighted_4096_bin_root_literal(fma):
    """The reference's literal 2990026907 (tests/test_parent_statistics.py:55-68):
    weighted squared error over 100,000 dense rows with 4096 bins, depth 1 --
    the root's stored base weight, whose last bit the ordered bin sum fixes."""
    X, y, weight = W.weighted_benchmark()
    ref = O.train(X, y, O.make_params(max_depth=1, max_bin=4096, seed=9, fma_contract=fma), 1, weights=weight)
    assert list(ref["cut_counts"]) == [4096] * 4
    bits = int(np.float32(ref["trees"][0]["base_weight"][0]).view(np.uint32))
    assert bits == W.WEIGHTED_BENCHMARK_ROOT_BITS


def test_root_density_changes_the_root_weight():
    """The reference's root construction (tests/test_scalar_root_statistics.py:
    10-45): gradients [2^40, -2^40, 3 * 2^-14], Hessians [1, 2, 1], depth 1,
    the root kept as a leaf (min_split_loss 1e30 stands in for the
    reference's max_leaves = 1).  A dense root sums feature 0's bins in bin
    order in binary64, where the first bin (2^40 + 3 * 2^-14, rows 0 and 2)
    rounds to 2^40 + 2^-12 before the cancellation; a root with a missing
    value takes the exact integer total, which keeps 3 * 2^-14.  When the root
    splits, its stored weight comes from the applied children's binary64
    sums, the rounded value in both cases (tests/test_parent_statistics.py:
    24-47)."""
    y = np.zeros(3, np.float32)
    g = np.asarray([2 ** 40, -2 ** 40, 3 * 2 ** -14], np.float32)
    h = np.asarray([1, 2, 1], np.float32)
    rounded = np.float32(-((2.0 ** 40 + 3 * 2.0 ** -14) - 2.0 ** 40) / 5.0)
    exact = np.float32(-(3 * 2.0 ** -14) / 5.0)
    assert rounded == np.float32(-2.0 ** -12 / 5.0) and rounded != exact
    dense = np.asarray([[0, 0], [1, 0], [0, 0]], np.float32)
    missing = np.asarray([[0, 0], [1, 0], [0, np.nan]], np.float32)
    for gamma, X, want in [(1e30, dense, rounded), (1e30, missing, exact), (0.0, dense, rounded),
                           (0.0, missing, rounded)]:
        params = O.make_params(max_depth=1, max_bin=4, eta=1.0, base_score=0.0, seed=9, min_split_loss=gamma)
        ref = O.train(X, y, params, 1, custom_grad=g[None, :], custom_hess=h[None, :])
        assert ref["sizes"][0] == (1 if gamma else 3)
        assert np.float32(ref["trees"][0][0]["base_weight"]) == want


def _sort_fixture_keys(pattern, n, k, seed):
    """The key classes tests/golden/make_sort_fixture.cpp sorts."""
    mask = (1 << 64) - 1
    x, out = seed, []
    for i in range(n):
        x = (x * 6364136223846793005 + 1442695040888963407) & mask
        out.append({"r": (x >> 33) % k, "a": i * k // n, "d": (n - 1 - i) * k // n,
                    "o": (i if i < n // 2 else n - 1 - i) % k, "s": (i * 7919) % k}[pattern])
    return np.asarray(out, np.uint32)


def test_sketch_sort_ties_follow_libstdcxx():
    """The oracle's std::sort restatement (the sketch's batch sort, whose
    order decides ties between equal values) leaves every fixture case's
    elements in the order this image's libstdc++ std::sort does: 798 cases of
    0 to 20,000 elements, random and patterned key classes with 1 to 2^30
    classes; the patterned cases reach the heap-sort fallback."""
    import ctypes
    import json
    from pathlib import Path
    lib = O.lib()
    lib.oracle_std_sort_order.restype = ctypes.c_uint64
    fixture = json.loads((Path(__file__).parent / "golden" / "sort_ties_libstdcxx.json").read_text())
    heap_sorts = 0
    for case in fixture["cases"]:
        n = case["n"]
        keys = _sort_fixture_keys(case["pattern"], n, case["k"], case["seed"])
        order = np.zeros(max(n, 1), np.uint32)
        heap_sorts += lib.oracle_std_sort_order(O.ptr(keys), ctypes.c_uint32(n), O.ptr(order))
        order = order[:n].astype(np.uint64)
        checksum = int((order * (2 * np.arange(n, dtype=np.uint64) + 1)).sum(dtype=np.uint64))
        assert checksum == case["checksum"], case
        assert order[:len(case["order"])].tolist() == case["order"], case
    assert heap_sorts > 0


def round_rational_f32(q):
    """A positive rational rounded to binary32, to nearest, ties to even."""
    assert q > 0
    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    e = max(e, -126)
    scaled = q * Fraction(2) ** (23 - e)  # the binary32 significand's units at q's binade
    m = scaled.numerator // scaled.denominator
    rest = scaled - m
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and m % 2):
        m += 1
    return np.float32(float(Fraction(m) * Fraction(2) ** (e - 23)))


def base_closed_form(y, w, scale_pos_weight, float_product):
    """The weighted label mean of a logistic objective, exactly, rounded once
    to binary32 (src/learner.cpp:316-333): terms y * w taken as binary32
    products (the reweighted intercept, kernels/boost.metal:379-381) or exact."""
    y = np.asarray(y, np.float32)
    w = np.where(y == 1, np.asarray(w, np.float32) * np.float32(scale_pos_weight), np.asarray(w, np.float32))
    w = w.astype(np.float32)
    num = sum(Fraction(float(np.float32(a * b))) if float_product else Fraction(float(a)) * Fraction(float(b))
              for a, b in zip(y, w))
    return round_rational_f32(num / sum(Fraction(float(b)) for b in w))


def _product_rounding_rows(count):
    """Single-row (label, weight) pairs whose binary32 product y * w moves the
    rounded mean off y: the two rules give different base scores on them."""
    rng = np.random.default_rng(2024)
    rows = []
    while len(rows) < count:
        y = np.float32(rng.uniform(0.05, 0.95))
        w = np.float32(rng.uniform(0.3, 7.0))
        if base_closed_form([y], [w], 2.5, True) != base_closed_form([y], [w], 2.5, False):
            rows.append((y, w))
    return rows


def test_round_rational_f32_matches_numpy_on_representable_and_tie_values():
    for v in (1.0, 0.1, 3.0e-38, 1.5, 123456.789):
        f = np.float32(v)
        assert round_rational_f32(Fraction(float(f))) == f
    one_ulp = Fraction(2) ** -23
    assert round_rational_f32(1 + one_ulp / 2) == np.float32(1.0)            # tie: to even
    assert round_rational_f32(1 + 3 * one_ulp / 2) == np.float32(1 + 2 * 2.0 ** -23)


@pytest.mark.parametrize("scale_pos_weight", [2.5, 1.0])
def test_base_score_of_reweighted_logistic_sums_binary32_products(scale_pos_weight):
    """With scale_pos_weight != 1 the logistic intercept sums binary32
    products y * w; with 1, exact products.  The single-row cases are chosen
    so that the two rules round to different binary32 means, so a base score
    that took the other rule fails here."""
    for y, w in _product_rounding_rows(6):
        got = np.float32(O.base_score([y], [w], objective=1, scale_pos_weight=scale_pos_weight))
        want = base_closed_form([y], [w], scale_pos_weight, scale_pos_weight != 1.0)
        assert got.view(np.uint32) == want.view(np.uint32), (y, w)
    rng = np.random.default_rng(7)
    y = rng.uniform(0, 1, 5000).astype(np.float32)
    y[::7] = 1.0
    w = rng.uniform(0.1, 3.0, 5000).astype(np.float32)
    got = np.float32(O.base_score(y, w, objective=1, scale_pos_weight=scale_pos_weight))
    want = base_closed_form(y, w, scale_pos_weight, scale_pos_weight != 1.0)
    assert got.view(np.uint32) == want.view(np.uint32)

