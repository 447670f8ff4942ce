// Shared device helpers for the gfx950 kernels (wave64, LDS scans, error
// reporting).  Included only by .hip translation units.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "mgb_kernels.h"

namespace mgb {

constexpr int kWave = 64;

// The library's single stream and last-error slot (defined in runtime.hip).
hipStream_t stream();
// The device the library is bound to (binding device 0 on first use), or -1
// with the error set.
int bound_device();
// True while per-kernel timing (mgb_profile_enable) is on.
bool profiling_enabled();
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

// Per-kernel-class timing (mgb_profile_enable).  When it is on, a launch
// through launch() records start and stop timestamps of the dispatch itself
// (hipExtLaunchKernelGGL events), so the time is the kernel's own duration
// with no marker packets between launches.
bool prof_events(int kind, hipEvent_t* begin, hipEvent_t* end);
void prof_record(int kind, hipEvent_t begin, hipEvent_t end);

template <typename... P, typename... A>
void launch(int kind, void (*fn)(P...), dim3 grid, dim3 block, uint32_t lds, A... args) {
  hipEvent_t begin = nullptr, end = nullptr;
  if (prof_events(kind, &begin, &end)) {
    hipExtLaunchKernelGGL(fn, grid, block, lds, stream(), begin, end, 0u, args...);
    prof_record(kind, begin, end);
  } else {
    hipLaunchKernelGGL(fn, grid, block, lds, stream(), args...);
  }
}

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// Wave64 inclusive prefix sums with DPP lane moves (no LDS round trip).
// Within each row of 16 lanes: row_shr 1, 2, 4, 8 (lanes whose source lies
// before the row start keep the identity 0).  Across rows: row_bcast:15 adds
// lane 15's (then lane 47's) total to rows 1 and 3, row_bcast:31 adds lane
// 31's total to rows 2 and 3.  Call with every lane of the wave active.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_move(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, kRowMask, 0xf, false);
}

template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint64_t dpp_move64(uint64_t v) {
  const uint32_t lo = dpp_move<kCtrl, kRowMask>((uint32_t)v);
  const uint32_t hi = dpp_move<kCtrl, kRowMask>((uint32_t)(v >> 32));
  return (uint64_t)lo | ((uint64_t)hi << 32);
}

constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143;

__device__ __forceinline__ uint32_t wave_inclusive_u32(uint32_t v) {
  v += dpp_move<kRowShr1, 0xf>(v);
  v += dpp_move<kRowShr2, 0xf>(v);
  v += dpp_move<kRowShr4, 0xf>(v);
  v += dpp_move<kRowShr8, 0xf>(v);
  v += dpp_move<kRowBcast15, 0xa>(v);
  v += dpp_move<kRowBcast31, 0xc>(v);
  return v;
}

__device__ __forceinline__ uint64_t wave_inclusive_u64(uint64_t v) {
  v += dpp_move64<kRowShr1, 0xf>(v);
  v += dpp_move64<kRowShr2, 0xf>(v);
  v += dpp_move64<kRowShr4, 0xf>(v);
  v += dpp_move64<kRowShr8, 0xf>(v);
  v += dpp_move64<kRowBcast15, 0xa>(v);
  v += dpp_move64<kRowBcast31, 0xc>(v);
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
