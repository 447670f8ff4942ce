"""std::shuffle over std::mt19937, the draws behind colsample_bytree
(reference src/tree.cpp:28-45; upstream XGBoost's ColumnSampler makes the
same call) and the CV folds (src/c_api.cpp:1018-1110).

Stock XGBoost's x86-64 wheels compile std::shuffle with libstdc++; the
reference's own builds (macOS) with libc++, whose draws differ.  The default
is libstdc++, pinned by tests/golden/shuffle_libstdcxx.json, which this
image's g++ wrote by running the real std::shuffle
(tests/golden/make_shuffle_fixture.cpp).  Both the oracle and the library's
host code (mgb_std_shuffle) are checked against it, and against an
independent restatement over numpy's MT19937.
"""
import ctypes
import json
from pathlib import Path

import numpy as np
import pytest

import device_lib as D
import oracle_lib as O

FIXTURE = json.loads((Path(__file__).parent / "golden" / "shuffle_libstdcxx.json").read_text())
CASES = FIXTURE["cases"]
MASK64 = (1 << 64) - 1


def checksum(perm):
    return sum(int(v) * (2 * i + 1) for i, v in enumerate(perm)) & MASK64


def library_shuffle(n, seed, model):
    out = np.zeros(max(n, 1), np.uint32)
    nxt = ctypes.c_uint32(0)
    D.check(D.lib().mgb_std_shuffle(ctypes.c_uint32(seed), ctypes.c_uint32(n), ctypes.c_uint32(model),
                                    out.ctypes.data_as(ctypes.c_void_p), ctypes.byref(nxt)))
    return out[:n], nxt.value


def mt_stream(seed):
    bg = np.random.MT19937()
    bg._legacy_seeding(seed)
    while True:
        for v in bg.random_raw(4096).tolist():
            yield v


def python_shuffle(n, seed, model):
    """Independent restatement over numpy's MT19937 (std::mt19937's engine).
    libstdc++: Lemire's multiply-shift draws, paired while n^2 < 2^32;
    libc++: masked rejection from the front."""
    g = mt_stream(seed)
    v = list(range(n))

    def lemire(rng):
        prod = next(g) * rng
        low = prod & 0xFFFFFFFF
        if low < rng:
            thr = (1 << 32) % rng
            while low < thr:
                prod = next(g) * rng
                low = prod & 0xFFFFFFFF
        return prod >> 32

    if n >= 2 and model == "libstdc++":
        if (2 ** 32 - 1) // n >= n:
            i = 1
            if n % 2 == 0:
                j = lemire(2)
                v[1], v[j] = v[j], v[1]
                i = 2
            while i < n:
                b1 = i + 2
                x = lemire((i + 1) * b1)
                v[i], v[x // b1] = v[x // b1], v[i]
                v[i + 1], v[x % b1] = v[x % b1], v[i + 1]
                i += 2
        else:
            for i in range(1, n):
                j = lemire(i + 1)
                v[i], v[j] = v[j], v[i]
    elif n >= 2:
        for p in range(n - 1):
            span = n - p
            mask = (1 << (span - 1).bit_length()) - 1
            while True:
                u = next(g) & mask
                if u < span:
                    break
            v[p], v[p + u] = v[p + u], v[p]
    return v, next(g)


def _check_case(perm, nxt, case):
    head = case["head"]
    assert list(map(int, perm[:len(head)])) == head
    assert checksum(perm) == case["checksum"]
    assert nxt == case["next_draw"]


@pytest.mark.parametrize("case", CASES, ids=[f"seed{c['seed']}-n{c['n']}" for c in CASES])
def test_oracle_shuffle_equals_libstdcxx(case):
    perm, nxt = O.std_shuffle(case["n"], case["seed"])
    _check_case(perm, nxt, case)


@pytest.mark.parametrize("case", CASES, ids=[f"seed{c['seed']}-n{c['n']}" for c in CASES])
def test_library_shuffle_equals_libstdcxx(case):
    perm, nxt = library_shuffle(case["n"], case["seed"], 0)
    _check_case(perm, nxt, case)


@pytest.mark.parametrize("n", [1, 2, 7, 64, 128, 1000])
def test_independent_restatement(n):
    """The numpy restatement equals the fixture (libstdc++) and the oracle and
    library (both models)."""
    for seed in (3, 42, 3737844653):
        for model, code in (("libstdc++", 0), ("libc++", 1)):
            want, want_next = python_shuffle(n, seed, model)
            got, got_next = O.std_shuffle(n, seed, model)
            assert got.tolist() == want and got_next == want_next
            lib, lib_next = library_shuffle(n, seed, code)
            assert lib.tolist() == want and lib_next == want_next
    for case in CASES:
        if case["n"] == n:
            perm, nxt = python_shuffle(n, case["seed"], "libstdc++")
            _check_case(perm, nxt, case)


def test_models_differ():
    """The two standard libraries draw different column samples at the
    config-4 shape (128 features, 0.8): the choice matters."""
    differ = sum(O.sample_columns(128, 0.8, s).tolist() != O.sample_columns(128, 0.8, s, "libc++").tolist()
                 for s in range(10))
    assert differ == 10


def test_column_sample_is_the_sorted_prefix():
    """colsample_bytree keeps the first max(1, floor(n * fraction)) of the
    shuffled features, sorted (src/tree.cpp:28-45)."""
    for case in CASES:
        n = case["n"]
        if n > 128:
            continue
        for fraction in (0.8, 0.5, 0.1):
            keep = max(1, int(np.floor(np.float32(n) * np.float32(fraction))))
            want = sorted(case["head"][:keep]) if fraction < 1 else list(range(n))
            assert O.sample_columns(n, fraction, case["seed"]).tolist() == want


def test_library_rejects_unknown_model():
    out = np.zeros(4, np.uint32)
    assert D.lib().mgb_std_shuffle(ctypes.c_uint32(1), ctypes.c_uint32(4), ctypes.c_uint32(2),
                                   out.ctypes.data_as(ctypes.c_void_p), None) == -1
