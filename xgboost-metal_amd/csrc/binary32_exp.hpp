// binary32 e^x and the logistic sigmoid, compiled for the host (g++) and for
// gfx950 (hipcc), giving the bits of the x86-64 host's libm.
//
// Stock XGBoost's CPU objective calls libm expf (upstream
// src/common/math.h `Sigmoid`); on this image's x86-64 hosts that is glibc
// 2.35, whose expf is the published method of ARM's optimized-routines
// (Szabolcs Nagy, 2017; glibc sysdeps/ieee754/flt-32/e_expf.c and
// e_exp2f_data.c):
//   x / ln2 = k/32 + r/32, k integer (round to nearest, via a 1.5*2^52 shift),
//   |r| <= 1/2;  e^x = 2^(k/32) * 2^(r/32);
//   2^(k/32) = (bits of 2^((k mod 32)/32)) + (k << 47), from a 32-entry table;
//   2^(r/32) ~= C0 r^3 + C1 r^2 + C2 r + 1, a cubic in binary64;
//   one final rounding of the binary64 product to binary32.
// glibc selects a build of it compiled with FMA contraction on CPUs that
// have FMA (every x86-64 host this library runs beside): the argument
// reduction and each polynomial step is one fused multiply-add.  The
// reduction's contraction changes two of the 2^32 results (x = 0x4202422f and
// 0xc27c65d9), the polynomial's none; an exhaustive sweep against the host's
// libm checks all 2^32 inputs.
//
// The table entries are 2^(i/32) rounded to binary64, minus i << 47 (so that
// adding k << 47 to the entry scales it by 2^floor(k/32)); the cubic's
// coefficients are optimized-routines' minimax fit (close to the Taylor
// terms ln2^3/6, ln2^2/2, ln2), pre-scaled by 32^-3, 32^-2, 32^-1.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MGB_HOST_DEVICE __host__ __device__
#else
#define MGB_HOST_DEVICE
#endif

namespace mgb {

MGB_HOST_DEVICE inline uint64_t exp2_32_entry(uint32_t i) {
  constexpr uint64_t kTable[32] = {
      0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
      0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
      0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
      0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
      0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
      0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
  return kTable[i & 31];
}

// e^x rounded to binary32 with the host libm's bits (see above).
MGB_HOST_DEVICE inline float exp_binary32(float x) {
  constexpr double kInvLn2x32 = 0x1.71547652b82fep+0 * 32;
  constexpr double kShift = 0x1.8p+52;
  constexpr double kC0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const uint32_t bits = __builtin_bit_cast(uint32_t, x);
  const uint32_t top = (bits >> 20) & 0x7ffu;
  if (top >= 0x42bu) {                      // |x| >= 88, infinite or NaN
    if (bits == 0xff800000u) return 0.0f;   // e^-inf
    if (top >= 0x7f8u) return x + x;        // +inf, NaN
    if (x > 0x1.62e42ep6f) return __builtin_inff();  // above ln(2^128): overflow
    if (x < -0x1.9fe368p6f) return 0.0f;    // below ln(2^-150): underflow to +0
  }
  const double xd = x;
  double kd = __builtin_fma(kInvLn2x32, xd, kShift);  // k + 1.5*2^52, k = nearest integer
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2x32, xd, -kd);  // x*32/ln2 - k, |r| <= 1/2
  const double s = __builtin_bit_cast(double, exp2_32_entry((uint32_t)ki) + (ki << 47));
  const double z = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

// Upstream XGBoost's Sigmoid (src/common/math.h), which binary:logistic's
// gradient and prediction transform call:
//   denom = expf(std::min(-x, 88.7f)) + 1.0f + 1e-16f;  return 1.0f / denom;
// std::min keeps -x when it is NaN.  The reference's kernel omits the clamp
// (kernels/boost.metal:50, `1/(1+exp(-x))`) and restates it with the clamp
// where it follows this function elsewhere (kernels/distributions.metal.h:250);
// the two differ only for x < -88.7.
MGB_HOST_DEVICE inline float sigmoid_binary32(float x) {
  const float neg = -x;
  const float arg = 88.7f < neg ? 88.7f : neg;
  const float denom = exp_binary32(arg) + 1.0f + 1e-16f;
  return 1.0f / denom;
}

}  // namespace mgb
