"""The binary32 exp shared by the library's kernels (csrc/binary32_exp.hpp)
against the host libm, and the oracle's sigmoid against its definition.

Stock XGBoost computes binary:logistic's sigmoid with the host libm's expf
(upstream src/common/math.h); the device must produce the same bits for the
trees to be identical, so the restated glibc expf is checked on every one of
the 2^32 binary32 inputs.
"""
import math

import numpy as np
import pytest

import expf_build
import oracle_lib as O


def f32(bits):
    return np.array([bits], np.uint32).view(np.float32)[0]


def test_exp_equals_host_libm_on_all_inputs():
    out = expf_build.run("mismatch")
    assert out.splitlines()[0] == "mismatches 0", out


def test_host_libm_is_the_fma_build():
    # glibc's expf built without FMA contraction rounds these two inputs the
    # other way (the only two of 2^32); the library restates the FMA build.
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    for x_bits, want in ((0x4202422F, float.fromhex("0x1.f93e38p+46")), (0xC27C65D9, float.fromhex("0x1.f45326p-92"))):
        assert libm.expf(float(f32(x_bits))) == want


def test_oracle_sigmoid_definition():
    sig = O.lib().oracle_sigmoid
    assert sig(0.0) == 0.5
    # The clamp: every x below -88.7 gives 1/(e^88.7 + 1), a subnormal.
    clamp = sig(-88.7)
    assert clamp > 0 and clamp < 2.0 ** -126
    for x in (-89.0, -100.0, -1e30, float("-inf")):
        assert sig(x) == clamp
    assert sig(float("inf")) == 1.0
    assert math.isnan(sig(float("nan")))
    # Within two binary32 ulps of the exact logistic on a spread of inputs (the
    # exp's rounding plus the add and the divide); a sign or order mistake
    # would be off by far more.
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.normal(size=2000) * 8, rng.uniform(-87, 20, size=2000)]).astype(np.float32)
    for x in xs:
        got = sig(float(x))
        exact = 1.0 / (1.0 + math.exp(-float(x)))
        assert abs(got - exact) <= 2 * np.spacing(np.float32(exact)), (x, got, exact)
