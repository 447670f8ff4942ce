// Shared device helpers for the gfx950 kernels (wave64, LDS scans, error
// reporting).  Included only by .hip translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "mgb_kernels.h"

namespace mgb {

constexpr int kWave = 64;

// The library's single stream and last-error slot (defined in runtime.hip).
hipStream_t stream();
void set_error(std::string message);
int check(hipError_t status, const char* what);

#define MGB_CHECK(call)                                   \
  do {                                                    \
    if (::mgb::check((call), #call) != 0) return -1;      \
  } while (0)
#define MGB_LAUNCH_CHECK(name)                            \
  do {                                                    \
    if (::mgb::check(hipGetLastError(), name) != 0) return -1; \
  } while (0)

// Profiling brackets around launches (no-ops unless mgb_profile_enable(1)).
void prof_begin(int kind);
void prof_end(int kind);

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// Inclusive wave64 prefix sum of a 32-bit value.
__device__ __forceinline__ uint32_t wave_inclusive_u32(uint32_t v) {
  const uint32_t lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    uint32_t other = __shfl_up(v, d, kWave);
    if (lane >= (uint32_t)d) v += other;
  }
  return v;
}

__device__ __forceinline__ uint64_t wave_inclusive_u64(uint64_t v) {
  const uint32_t lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    uint64_t other = __shfl_up(v, d, kWave);
    if (lane >= (uint32_t)d) v += other;
  }
  return v;
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}

// Block-wide exclusive scan of 32-bit values; `shared` needs blockDim/64 + 1
// words.  Returns the exclusive prefix; *total receives the block sum.
__device__ __forceinline__ uint32_t block_exclusive_u32(uint32_t v, uint32_t* shared, uint32_t* total) {
  const uint32_t lane = lane_id(), wave = threadIdx.x / kWave, waves = (blockDim.x + kWave - 1) / kWave;
  uint32_t inc = wave_inclusive_u32(v);
  if (lane == kWave - 1) shared[wave] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (uint32_t w = 0; w < waves; ++w) {
      uint32_t t = shared[w];
      shared[w] = run;
      run += t;
    }
    shared[waves] = run;
  }
  __syncthreads();
  uint32_t result = shared[wave] + inc - v;
  *total = shared[waves];
  __syncthreads();
  return result;
}

// Exact binary32 <-> integer helpers.
__device__ __forceinline__ float bits_to_float(uint32_t b) { return __uint_as_float(b); }

}  // namespace mgb
