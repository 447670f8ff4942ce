// Exhaustive checks of the library's binary32 exp (csrc/binary32_exp.hpp)
// against the host libm, built and run by tests/test_expf.py and
// tests/test_gpu_expf.py with g++ -O2 -fopenmp -ffp-contract=off.
//
//   expf_sweep mismatch       all 2^32 inputs: count x with
//                             bits(exp_binary32(x)) != bits(expf(x))
//                             (any NaN equals any NaN); prints up to 8 of them
//   expf_sweep checksum       sum over i < 2^32 of canon(bits(sigmoid(x_i))) * (2i + 1)
//                             mod 2^64, where x_i has the bits i and sigmoid is
//                             upstream XGBoost's expression over libm expf;
//                             canon maps every NaN to 0x7fc00000.  The GPU test
//                             compares the device's sigmoid with it.
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "binary32_exp.hpp"

static inline uint32_t bits_of(float f) { return __builtin_bit_cast(uint32_t, f); }

// Upstream XGBoost's Sigmoid (src/common/math.h) over the host libm's expf.
static inline float sigmoid_libm(float x) {
  const float neg = -x;
  const float arg = 88.7f < neg ? 88.7f : neg;
  return 1.0f / (expf(arg) + 1.0f + 1e-16f);
}

static inline uint64_t canon(float f) { return isnan(f) ? 0x7fc00000u : bits_of(f); }

int main(int argc, char** argv) {
  const char* mode = argc > 1 ? argv[1] : "mismatch";
  if (!strcmp(mode, "mismatch")) {
    uint64_t bad = 0;
    uint32_t shown[8];
    int nshown = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad)
    for (int64_t i = 0; i < (int64_t(1) << 32); ++i) {
      const float x = __builtin_bit_cast(float, (uint32_t)i);
      const float a = expf(x), b = mgb::exp_binary32(x);
      if (bits_of(a) != bits_of(b) && !(isnan(a) && isnan(b))) {
        ++bad;
#pragma omp critical
        if (nshown < 8) shown[nshown++] = (uint32_t)i;
      }
    }
    printf("mismatches %llu\n", (unsigned long long)bad);
    for (int k = 0; k < nshown; ++k) {
      const float x = __builtin_bit_cast(float, shown[k]);
      printf("x=0x%08x libm=0x%08x library=0x%08x\n", shown[k], bits_of(expf(x)), bits_of(mgb::exp_binary32(x)));
    }
    return 0;
  }
  if (!strcmp(mode, "checksum")) {
    uint64_t sum = 0;
#pragma omp parallel for schedule(static) reduction(+ : sum)
    for (int64_t i = 0; i < (int64_t(1) << 32); ++i) {
      const float x = __builtin_bit_cast(float, (uint32_t)i);
      sum += canon(sigmoid_libm(x)) * (2 * (uint64_t)i + 1);
    }
    printf("checksum %llu\n", (unsigned long long)sum);
    return 0;
  }
  fprintf(stderr, "usage: %s mismatch|checksum\n", argv[0]);
  return 2;
}
