// Data-side kernels: bin matrix, gradients, fixed-point scales, base score,
// margin fill and tree prediction.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <string>

#include "binary32_exp.hpp"
#include "device_common.hpp"

namespace mgb {
namespace {

// ---------------------------------------------------------------------------
// Bin matrix (kernels/boost.metal:476-499): bin = min(#{cuts <= v}, count-1),
// NaN -> missing code.  A workgroup takes `tile_features` consecutive
// (padded) features, whose cuts it stages in LDS so that every step of the
// binary search is an LDS read, and walks its rows in chunks: each chunk's
// values are read row by row (consecutive threads on consecutive features),
// quantized into an LDS tile, and written in the output layout's own order
// (consecutive threads on consecutive codes: along a row for the row-major
// layout, along a column for the column-major copy).
// ---------------------------------------------------------------------------
constexpr uint32_t kQuantThreads = 1024;
constexpr uint32_t kQuantCutsLds = 68 * 1024;   // bytes of staged cuts per workgroup (64 features of 256 cuts, 16 of 1024)
constexpr uint32_t kQuantChunkCodes = 8192;     // codes per chunk (LDS tile)

// Address of code (r, f) of a bin matrix.
template <typename BinT>
__device__ __forceinline__ BinT* code_at(BinT* bins, const MgbMatrix& m, uint64_t r, uint32_t f) {
  const uint32_t g = f / m.group_features, j = f % m.group_features;
  return reinterpret_cast<BinT*>(reinterpret_cast<uint8_t*>(bins) + (uint64_t)g * m.group_stride + r * m.row_stride) + j;
}

// tile_features and chunk_rows are powers of two; the cuts of feature j sit
// at s_cuts + j * (cut_stride + 1) (an odd stride, so that the searches of
// different features start in different LDS banks).  columns (may be NULL)
// receives the same codes column-major: code (r, f) at columns[f * rows + r].
template <typename BinT>
__global__ __launch_bounds__(kQuantThreads) void k_quantize(const float* __restrict__ X, const float* __restrict__ cuts,
                                                            const uint32_t* __restrict__ counts, MgbMatrix m,
                                                            uint32_t tile_shift, uint32_t chunk_shift, uint32_t chunks,
                                                            BinT* __restrict__ bins, BinT* __restrict__ columns,
                                                            uint32_t* __restrict__ any_missing) {
  extern __shared__ __align__(16) uint8_t q_smem[];
  const uint32_t tile_features = 1u << tile_shift, chunk_rows = 1u << chunk_shift;
  const uint32_t stride = m.cut_stride + 1;
  float* s_cuts = reinterpret_cast<float*>(q_smem);  // tile_features x stride
  uint32_t* s_count = reinterpret_cast<uint32_t*>(s_cuts + (uint64_t)tile_features * stride);
  BinT* s_codes = reinterpret_cast<BinT*>(s_count + tile_features);  // chunk_rows x tile_features
  const uint32_t G = m.group_features;
  const uint32_t padded = (m.cols + G - 1) / G * G;
  const uint32_t f0 = blockIdx.y << tile_shift;
  const uint32_t nf = padded - f0 < tile_features ? padded - f0 : tile_features;
  for (uint32_t j = threadIdx.x; j < tile_features; j += blockDim.x) s_count[j] = f0 + j < m.cols ? counts[f0 + j] : 0u;
  for (uint32_t j = 0; j < nf; ++j) {
    if (f0 + j >= m.cols) break;
    const float* src = cuts + (uint64_t)(f0 + j) * m.cut_stride;
    for (uint32_t c = threadIdx.x; c < m.cut_stride; c += blockDim.x) s_cuts[j * stride + c] = src[c];
  }
  __syncthreads();
  bool missing = false;
  const uint64_t row0 = (uint64_t)blockIdx.x * chunks << chunk_shift;
  const uint32_t codes = chunk_rows << tile_shift;
  for (uint32_t chunk = 0; chunk < chunks; ++chunk) {
    const uint64_t r0 = row0 + ((uint64_t)chunk << chunk_shift);
    if (r0 >= m.rows) break;
    const uint32_t nr = m.rows - r0 < chunk_rows ? (uint32_t)(m.rows - r0) : chunk_rows;
    // Rows in order, features fastest: consecutive threads read a row's
    // consecutive values.
    for (uint32_t i = threadIdx.x; i < codes; i += blockDim.x) {
      const uint32_t rr = i >> tile_shift, j = i & (tile_features - 1);
      if (rr >= nr || j >= nf) continue;
      const uint32_t f = f0 + j;
      BinT code = (BinT)m.missing_code;
      if (f < m.cols) {
        const float v = X[(r0 + rr) * m.cols + f];
        const uint32_t count = s_count[j];
        if (!isnan(v) && count) {
          const float* column = s_cuts + j * stride;
          uint32_t lo = 0, hi = count;
          while (lo < hi) {
            const uint32_t mid = lo + (hi - lo) / 2;
            if (v >= column[mid]) lo = mid + 1;
            else hi = mid;
          }
          code = (BinT)(lo < count - 1 ? lo : count - 1);
        } else {
          missing = true;
        }
      }
      s_codes[i] = code;
    }
    __syncthreads();
    if (m.row_stride == sizeof(BinT) && G == 1) {
      // A column-major matrix: consecutive threads along a column.
      for (uint32_t i = threadIdx.x; i < codes; i += blockDim.x) {
        const uint32_t rr = i & (chunk_rows - 1), j = i >> chunk_shift;
        if (rr < nr && j < nf) *code_at(bins, m, r0 + rr, f0 + j) = s_codes[(rr << tile_shift) + j];
      }
    } else {
      for (uint32_t i = threadIdx.x; i < codes; i += blockDim.x) {
        const uint32_t rr = i >> tile_shift, j = i & (tile_features - 1);
        if (rr < nr && j < nf) *code_at(bins, m, r0 + rr, f0 + j) = s_codes[i];
      }
    }
    if (columns) {
      for (uint32_t i = threadIdx.x; i < codes; i += blockDim.x) {
        const uint32_t rr = i & (chunk_rows - 1), j = i >> chunk_shift;
        if (rr < nr && j < nf && f0 + j < m.cols) columns[(uint64_t)(f0 + j) * m.rows + r0 + rr] = s_codes[(rr << tile_shift) + j];
      }
    }
    __syncthreads();
  }
  if (__any(missing) && lane_id() == 0) atomicOr(any_missing, 1u);
}

// ---------------------------------------------------------------------------
// Gradients (kernels/boost.metal:553-601) and exact magnitude mass
// (kernels/gradient_quantization.metal.h:4-24).  The exact sum of |g| in
// units of 2^-149 is kept as 256 per-exponent u64 sums of 24-bit mantissas:
// |g| = m * 2^j units with j = max(E,1)-1, so sum = sum_j S_j * 2^j exactly.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void mass_bucket(float v, uint32_t& bucket, uint64_t& mantissa) {
  uint32_t bits = __float_as_uint(v) & 0x7fffffffu;
  uint32_t e = bits >> 23;
  uint32_t m = bits & 0x7fffffu;
  if (e) { m |= 0x800000u; bucket = e - 1; }
  else bucket = 0;
  mantissa = m;
}

constexpr uint32_t kGradThreads = 1024;
constexpr uint32_t kGradBlocks = 256;  // at most; one partial per workgroup
constexpr uint32_t kLimbs = 11;        // 352 bits > 255 + 56 bits of the largest exact sum
constexpr uint32_t kTicket = 2 * kLimbs * kGradBlocks;  // completion counter word of the mass buffer
static_assert(kTicket < MGB_MASS_WORDS, "mass buffer too small");

// Carry-save limbs of sum_j S_j 2^j for both quantities: limbs[q*11 + w]
// receives the 32-bit pieces of every S_j << (j % 32) that land in limb w
// (S_j < 2^56 spans limbs j/32 .. j/32+2).  staged[q*256 + j] = S_j of
// quantity q (0: |g|, 1: |h|).  Thread t < 512 takes bucket (t / 256, t % 256);
// the 32 buckets sharing j/32 are one half-wave, which sums its pieces with
// shuffles (each sum < 2^37) and adds them to three limbs.  limbs must be
// zero on entry; blockDim.x >= 512.  Ends with a barrier.
__device__ void block_carry_save(const uint64_t* staged, uint64_t* limbs) {
  const uint32_t t = threadIdx.x;
  uint64_t p0 = 0, p1 = 0, p2 = 0;
  if (t < 512) {
    const uint64_t v = staged[t];
    const uint32_t shift = t % 32;
    const uint64_t lo = v << shift, hi = shift ? (v >> (64 - shift)) : 0;
    p0 = (uint32_t)lo; p1 = (uint32_t)(lo >> 32); p2 = (uint32_t)hi;
  }
#pragma unroll
  for (int d = 16; d > 0; d >>= 1) {
    p0 += __shfl_xor(p0, d, kWave);
    p1 += __shfl_xor(p1, d, kWave);
    p2 += __shfl_xor(p2, d, kWave);
  }
  if (t < 512 && t % 32 == 0) {
    const uint32_t q = t / 256, w = (t % 256) / 32;
    atomicAdd((unsigned long long*)&limbs[q * kLimbs + w], (unsigned long long)p0);
    atomicAdd((unsigned long long*)&limbs[q * kLimbs + w + 1], (unsigned long long)p1);
    atomicAdd((unsigned long long*)&limbs[q * kLimbs + w + 2], (unsigned long long)p2);
  }
  __syncthreads();
}

// scale = 2^(62 - max(0, bitlen(sum) - 149)); gradient_quantization.metal.h:52-63.
// limbs: carry-save limbs of both sums (any entries below 2^63); threads 0
// and 1 propagate the carries, exactly as a serial big-integer add would.
__device__ void scales_from_limbs(const uint64_t* limbs, float* scales) {
  const uint32_t tid = threadIdx.x;
  if (tid < 2) {
    uint32_t limb[kLimbs + 1];
    uint64_t carry = 0;
    for (uint32_t w = 0; w < kLimbs; ++w) {
      const uint64_t v = (limbs[tid * kLimbs + w] & 0xffffffffull) + carry;
      limb[w] = (uint32_t)v;
      carry = (v >> 32) + (limbs[tid * kLimbs + w] >> 32);
    }
    limb[kLimbs] = (uint32_t)carry;
    int exponent = 0;
    for (int w = kLimbs; w >= 0; --w) {
      if (limb[w]) {
        const int bitlen = w * 32 + 32 - __clz(limb[w]);
        exponent = bitlen - 149 > 0 ? bitlen - 149 : 0;
        break;
      }
    }
    scales[tid] = __uint_as_float((uint32_t)(62 - exponent + 127) << 23);
  }
}

// kMassCopies copies of the 512 buckets, lanes spread over them: the lanes of
// a wave often share one bucket (every h of squared error), and LDS atomics
// on one address serialize.
constexpr uint32_t kMassCopies = 4;

// Per-workgroup exponent buckets in LDS, reduced to 22 carry-save limbs and
// published to the workgroup's own slot of the mass buffer; the last
// workgroup to finish (completion counter) sums the slots and writes the
// scales.  Every cross-workgroup access is a device-scope atomic: the slot
// writes are exchanges whose returned values the workgroup waits for (they
// feed an LDS store) before its counter increment, so they have been
// performed at the device's point of coherence when the counter moves --
// without an agent-scope fence, which would write back the whole L2.  No two
// workgroups touch the same word except the counter.
__device__ void mass_flush_and_scale(uint64_t* local, uint64_t* mass, float* scales) {
  __shared__ uint64_t limbs[2 * kLimbs];
  constexpr uint32_t kShare = 32;                  // threads per limb in the final sum
  constexpr uint32_t kPer = kGradBlocks / kShare;  // slots per thread, loaded together
  __shared__ uint64_t partial[2 * kLimbs][kShare];
  __shared__ uint32_t last;
  __shared__ volatile uint64_t sink;
  (void)sink;
  const uint32_t tid = threadIdx.x;
  if (tid < 2 * kLimbs) limbs[tid] = 0;
  __syncthreads();
  for (uint32_t i = tid; i < 512; i += blockDim.x) {
    uint64_t v = local[i];
    for (uint32_t k = 1; k < kMassCopies; ++k) v += local[k * 512 + i];
    local[i] = v;
  }
  __syncthreads();
  block_carry_save(local, limbs);
  if (tid < 2 * kLimbs)
    sink = __hip_atomic_exchange(&mass[(uint64_t)blockIdx.x * 2 * kLimbs + tid], limbs[tid], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (tid == 0)
    last = __hip_atomic_fetch_add(&mass[kTicket], (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           (uint64_t)(gridDim.x - 1);
  __syncthreads();
  if (!last) return;
  // kShare threads per limb, each loading its kPer workgroup slots at once.
  if (tid < 2 * kLimbs * kShare) {
    const uint32_t l = tid / kShare, part = tid % kShare;
    uint64_t v[kPer];
#pragma unroll
    for (uint32_t k = 0; k < kPer; ++k) {
      const uint32_t b = part + k * kShare;
      v[k] = b < gridDim.x ? __hip_atomic_load(&mass[(uint64_t)b * 2 * kLimbs + l], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT)
                           : 0;
    }
    uint64_t acc = 0;
#pragma unroll
    for (uint32_t k = 0; k < kPer; ++k) acc += v[k];
    partial[l][part] = acc;
  }
  if (tid == 0) __hip_atomic_store(&mass[kTicket], (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (tid < 2 * kLimbs) {
    uint64_t acc = 0;
    for (uint32_t k = 0; k < kShare; ++k) acc += partial[tid][k];
    limbs[tid] = acc;
  }
  __syncthreads();
  scales_from_limbs(limbs, scales);
}

// Uniform row sampling (kernels/sampling.metal.h:1-30): the row's state is
// the round seed times 16807^(row+1) modulo 2^63; the row is kept when the
// binary64 value of state-1 over 2^63 (the canonical draw of a 63-bit engine)
// is below subsample, compared in binary32 when subsample < 2^-39.
constexpr uint64_t kStateMask = 0x7fffffffffffffffull;

// base * 16807^e mod 2^63 (square and multiply; products mod 2^64, then the mask).
__device__ __forceinline__ uint64_t times_16807_pow(uint64_t base, uint64_t e) {
  uint64_t state = base, factor = 16807u;
  for (; e; e >>= 1) {
    if (e & 1) state = (state * factor) & kStateMask;
    factor = (factor * factor) & kStateMask;
  }
  return state;
}

// A thread's rows r, r + S, r + 2S, ...: the first state by square and
// multiply, each next one by one multiply by 16807^S (exact mod 2^63).
struct RowSampler {
  uint64_t state, step;
  __device__ RowSampler(uint32_t seed, uint32_t first, uint32_t stride, bool on)
      : state(on ? times_16807_pow(seed ? seed : 1u, (uint64_t)first + 1) : 0),
        step(on ? times_16807_pow(1u, stride) : 0) {}
  __device__ __forceinline__ void next() { state = (state * step) & kStateMask; }
};

__device__ __forceinline__ bool keep_state(uint64_t state, float subsample) {
  const double rounded = (double)(state - 1);
  const float limit = subsample * 0x1p63f;
  if (limit < 0x1p24f) return (float)rounded < limit;
  return rounded < (double)limit;
}

__device__ __forceinline__ void mass_add(uint64_t* local, float g, float h) {
  uint32_t bg, bh;
  uint64_t mg, mh;
  mass_bucket(g, bg, mg);
  mass_bucket(h, bh, mh);
  uint64_t* copy = local + (lane_id() % kMassCopies) * 512;
  if (mg) atomicAdd((unsigned long long*)&copy[bg], (unsigned long long)mg);
  if (mh) atomicAdd((unsigned long long*)&copy[256 + bh], (unsigned long long)mh);
}

__global__ __launch_bounds__(kGradThreads) void k_gradients(MgbGradParams p, const float* __restrict__ margin,
                                                            const float* __restrict__ labels,
                                                            const float* __restrict__ weights,
                                                            float2* __restrict__ grad, uint64_t* __restrict__ mass,
                                                            float* __restrict__ scales) {
  __shared__ uint64_t local[kMassCopies * 512];
  for (uint32_t i = threadIdx.x; i < kMassCopies * 512; i += blockDim.x) local[i] = 0;
  __syncthreads();
  const uint32_t first = blockIdx.x * blockDim.x + threadIdx.x, stride = gridDim.x * blockDim.x;
  RowSampler sampler(p.sample_seed, first, stride, p.subsample < 1.0f);
  for (uint64_t r = first; r < p.rows; r += stride, sampler.next()) {
    float pred = margin[r], label = labels[r];
    float weight = p.has_weight ? weights[r] : 1.0f;
    float g = pred - label, h = 1.0f;
    if (p.objective == 1 || p.objective == 2) {
      // Upstream XGBoost's Sigmoid over a binary32 exp with the host libm's
      // bits (binary32_exp.hpp); kernels/boost.metal:566-570.
      float prob = mgb::sigmoid_binary32(pred);
      weight *= label == 1.0f ? p.scale_pos_weight : 1.0f;
      g = prob - label;
      h = fmaxf(prob * (1.0f - prob), 1.0e-16f);
    }
    g = g * weight;
    h = h * weight;
    if (p.subsample < 1.0f && !keep_state(sampler.state, p.subsample)) g = h = 0.0f;
    grad[r] = make_float2(g, h);
    mass_add(local, g, h);
  }
  mass_flush_and_scale(local, mass, scales);
}

__global__ __launch_bounds__(kGradThreads) void k_gradient_mass(MgbGradParams p, float2* __restrict__ grad,
                                                                uint64_t* __restrict__ mass,
                                                                float* __restrict__ scales) {
  __shared__ uint64_t local[kMassCopies * 512];
  for (uint32_t i = threadIdx.x; i < kMassCopies * 512; i += blockDim.x) local[i] = 0;
  __syncthreads();
  const uint32_t first = blockIdx.x * blockDim.x + threadIdx.x, stride = gridDim.x * blockDim.x;
  RowSampler sampler(p.sample_seed, first, stride, p.subsample < 1.0f);
  for (uint64_t r = first; r < p.rows; r += stride, sampler.next()) {
    float2 v = grad[r];
    if (p.subsample < 1.0f && !keep_state(sampler.state, p.subsample)) {
      v = make_float2(0.0f, 0.0f);
      grad[r] = v;
    }
    mass_add(local, v.x, v.y);
  }
  mass_flush_and_scale(local, mass, scales);
}

__global__ void k_gradient_scales(uint64_t* __restrict__ mass, float* __restrict__ scales) {
  __shared__ uint64_t staged[512];
  __shared__ uint64_t limbs[2 * kLimbs];
  for (uint32_t i = threadIdx.x; i < 512; i += blockDim.x) staged[i] = mass[i];
  if (threadIdx.x < 2 * kLimbs) limbs[threadIdx.x] = 0;
  __syncthreads();
  block_carry_save(staged, limbs);
  scales_from_limbs(limbs, scales);
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < 512; i += blockDim.x) mass[i] = 0;
}

// ---------------------------------------------------------------------------
// Base score (src/learner.cpp:316-333, kernels/boost.metal:356-423): weighted
// label mean.  Each thread keeps a compensated binary64 sum (products of two
// binary32 values are exact), then a fixed-order tree reduction combines them.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void two_sum_add(double& s, double& c, double x) {
  double t = s + x;
  c += fabs(s) >= fabs(x) ? (s - t) + x : (x - t) + s;
  s = t;
}

// Weighted label sum and weight sum (src/learner.cpp:316-333) as binary64
// sums with a compensation term each (two-sum), first per workgroup over a
// strided share of the rows, then over the workgroups' partials by the last
// workgroup; the mean is rounded once to binary32.  Products of two binary32
// values are exact in binary64, and the compensated sums carry about twice
// binary64's precision.  The workgroup count and the combining tree are fixed
// for a given row count, so the result is deterministic for a given row
// count; the compensation terms themselves are added plainly, so another
// tree of partial sums could round differently in the last bits.
constexpr uint32_t kBaseThreads = 1024;
constexpr uint32_t kBaseBlocks = 256;
__device__ double g_base_partials[kBaseBlocks][4];
__device__ uint32_t g_base_ticket;

__device__ void base_tree(double (*sh)[kBaseThreads], uint32_t n) {
  for (uint32_t d = kBaseThreads / 2; d > 0; d >>= 1) {
    if (threadIdx.x < d && threadIdx.x + d < n) {
      double a = sh[0][threadIdx.x], ac = sh[1][threadIdx.x];
      two_sum_add(a, ac, sh[0][threadIdx.x + d]);
      ac += sh[1][threadIdx.x + d];
      double b = sh[2][threadIdx.x], bc = sh[3][threadIdx.x];
      two_sum_add(b, bc, sh[2][threadIdx.x + d]);
      bc += sh[3][threadIdx.x + d];
      sh[0][threadIdx.x] = a; sh[1][threadIdx.x] = ac; sh[2][threadIdx.x] = b; sh[3][threadIdx.x] = bc;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(kBaseThreads) void k_base_score(const float* __restrict__ labels,
                                                             const float* __restrict__ weights, uint32_t rows,
                                                             uint32_t objective, float spw, float* __restrict__ out) {
  __shared__ double sh[4][kBaseThreads];
  __shared__ uint32_t s_last;
  // A logistic objective whose scale_pos_weight is not 1 sums the binary32
  // products y * w (the reweighted intercept, kernels/boost.metal:379-381);
  // otherwise the products are exact in binary64.
  const bool logistic = objective == 1 || objective == 2;
  const bool float_product = logistic && fabsf(spw - 1.0f) > 1.0e-6f;
  double s = 0, c = 0, ws = 0, wc = 0;
  for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (uint64_t)gridDim.x * blockDim.x) {
    float w = weights ? weights[r] : 1.0f;
    float y = labels[r];
    if (logistic) w *= y == 1.0f ? spw : 1.0f;
    const float product = y * w;
    two_sum_add(s, c, float_product ? (double)product : (double)y * (double)w);
    two_sum_add(ws, wc, (double)w);
  }
  sh[0][threadIdx.x] = s; sh[1][threadIdx.x] = c; sh[2][threadIdx.x] = ws; sh[3][threadIdx.x] = wc;
  __syncthreads();
  base_tree(sh, kBaseThreads);
  if (threadIdx.x == 0) {
    for (int k = 0; k < 4; ++k) g_base_partials[blockIdx.x][k] = sh[k][0];
    __threadfence();
    s_last = atomicAdd(&g_base_ticket, 1u) == gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  // The last workgroup: every partial is visible after its fence.
  __threadfence();
  const uint32_t n = gridDim.x;
  for (int k = 0; k < 4; ++k)
    sh[k][threadIdx.x] = threadIdx.x < n ? __builtin_nontemporal_load(&g_base_partials[threadIdx.x][k]) : 0.0;
  __syncthreads();
  base_tree(sh, n);
  if (threadIdx.x == 0) {
    g_base_ticket = 0;  // ready for the next call on this stream
    double value = sh[0][0] + sh[1][0], weight = sh[2][0] + sh[3][0];
    float result;
    if (!(weight > 0)) result = objective == 0 && rows == 0 ? 0.0f : 0.5f;
    else result = (float)(value / weight);
    out[0] = result;
  }
}

__global__ void k_any_missing(const float* __restrict__ data, uint64_t count, uint32_t* __restrict__ flag) {
  bool missing = false;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (uint64_t)gridDim.x * blockDim.x)
    missing |= isnan(data[i]);
  if (__any(missing) && lane_id() == 0) atomicOr(flag, 1u);
}

// Prediction transform of binary:logistic (sigmoid of the margin, the same
// function as the gradient's).
__global__ void k_transform(float* __restrict__ data, uint64_t count, uint32_t objective) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (uint64_t)gridDim.x * blockDim.x) {
    if (objective == 1) data[i] = mgb::sigmoid_binary32(data[i]);
  }
}

__global__ __launch_bounds__(256) void k_copy(uint4* __restrict__ dst, const uint4* __restrict__ src, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

__global__ void k_fill(float* __restrict__ data, uint64_t count, float value) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (uint64_t)gridDim.x * blockDim.x)
    data[i] = value;
}

// Prediction (kernels/boost.metal:1325-1329 split_left, :1738-1763 predict):
// float traversal on the raw values; NaN follows default_left.
__global__ void k_predict(const float* __restrict__ X, uint32_t rows, uint32_t cols,
                          const MgbTreeNode* __restrict__ nodes, const uint32_t* __restrict__ offsets,
                          uint32_t trees, float* __restrict__ margin) {
  for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (uint64_t)gridDim.x * blockDim.x) {
    const float* row = X + (uint64_t)r * cols;
    float sum = margin[r];
    for (uint32_t t = 0; t < trees; ++t) {
      const MgbTreeNode* tree = nodes + offsets[t];
      int32_t id = 0;
      while (tree[id].left >= 0) {
        float v = row[tree[id].feature];
        bool left = isnan(v) ? tree[id].default_left != 0 : v < tree[id].threshold;
        id = left ? tree[id].left : tree[id].right;
      }
      sum = sum + tree[id].leaf;
    }
    margin[r] = sum;
  }
}

uint32_t grid_for(uint64_t work, uint32_t block, uint32_t cap = 8192) {
  uint64_t g = (work + block - 1) / block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (uint32_t)g;
}

}  // namespace
}  // namespace mgb

using namespace mgb;

extern "C" {

static int quantize(const float* X, const float* cuts, const uint32_t* counts, const MgbMatrix* m, void* bins,
                    void* columns, uint32_t* any_missing) {
  if (!m || !bins || !any_missing) { set_error("mgb_quantize_bins: null argument"); return -1; }
  if (m->bin_bytes != 1 && m->bin_bytes != 2) { set_error("mgb_quantize_bins: bin_bytes must be 1 or 2"); return -1; }
  const uint32_t G = m->group_features;
  if (G != 1 && G != 2 && G != 4 && G != 8 && G != 16) {
    set_error("mgb_quantize_bins: group_features must be a power of two <= 16");
    return -1;
  }
  const uint64_t groups = (m->cols + G - 1) / G, gbytes = (uint64_t)G * m->bin_bytes;
  const bool row_major = m->group_stride == gbytes && m->row_stride == groups * gbytes;
  const bool group_major = m->row_stride == gbytes && m->group_stride == (uint64_t)m->rows * gbytes;
  if (!row_major && !group_major) {
    set_error("mgb_quantize_bins: row_stride/group_stride describe neither the row-major nor the group-major layout");
    return -1;
  }
  if (!m->rows || !m->cols) return 0;
  if (((uint64_t)m->cut_stride + 1) * 4 > kQuantCutsLds) {
    set_error("mgb_quantize_bins: cut_stride above " + std::to_string(kQuantCutsLds / 4 - 1) + " cuts per feature");
    return -1;
  }
  // Features per workgroup: the largest power of two (at most 64) whose cuts
  // fit the staging budget; rows in chunks of kQuantChunkCodes codes, and as
  // many chunks per workgroup as keep about 2048 workgroups busy.
  const uint32_t padded = (uint32_t)(groups * G);
  uint32_t tile_shift = 6;
  while (tile_shift > 0 && ((((uint64_t)1 << tile_shift) * (m->cut_stride + 1) * 4 > kQuantCutsLds) ||
                            (1u << (tile_shift - 1)) >= padded))
    --tile_shift;
  uint32_t chunk_shift = 0;
  while ((1u << (chunk_shift + 1 + tile_shift)) <= kQuantChunkCodes) ++chunk_shift;
  const uint32_t tiles = (padded + (1u << tile_shift) - 1) >> tile_shift;
  const uint64_t row_chunks = (m->rows + (1ull << chunk_shift) - 1) >> chunk_shift;
  const uint32_t chunks =
      (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(8, row_chunks * tiles / 2048));
  const dim3 grid((uint32_t)((row_chunks + chunks - 1) / chunks), tiles);
  const uint32_t lds = (1u << tile_shift) * ((m->cut_stride + 1) * 4 + 4) + (1u << (chunk_shift + tile_shift)) * m->bin_bytes;
  if (m->bin_bytes == 1) {
    if (check(hipFuncSetAttribute((const void*)k_quantize<uint8_t>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
              "hipFuncSetAttribute(k_quantize)"))
      return -1;
    hipLaunchKernelGGL(k_quantize<uint8_t>, grid, dim3(kQuantThreads), lds, stream(), X, cuts, counts, *m, tile_shift,
                       chunk_shift, chunks, (uint8_t*)bins, (uint8_t*)columns, any_missing);
  } else {
    if (check(hipFuncSetAttribute((const void*)k_quantize<uint16_t>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
              "hipFuncSetAttribute(k_quantize)"))
      return -1;
    hipLaunchKernelGGL(k_quantize<uint16_t>, grid, dim3(kQuantThreads), lds, stream(), X, cuts, counts, *m, tile_shift,
                       chunk_shift, chunks, (uint16_t*)bins, (uint16_t*)columns, any_missing);
  }
  MGB_LAUNCH_CHECK("k_quantize");
  return 0;
}

int mgb_quantize_bins(const float* X, const float* cuts, const uint32_t* counts, const MgbMatrix* m, void* bins,
                      uint32_t* any_missing) {
  return quantize(X, cuts, counts, m, bins, nullptr, any_missing);
}

int mgb_quantize_bins_columns(const float* X, const float* cuts, const uint32_t* counts, const MgbMatrix* m,
                              void* bins, void* columns, uint32_t* any_missing) {
  if (!columns) { set_error("mgb_quantize_bins_columns: null columns"); return -1; }
  return quantize(X, cuts, counts, m, bins, columns, any_missing);
}

// Workgroups of the gradient passes: one per kGradRows rows, at most
// kGradBlocks.  The pass ends in a chain of device-scope atomics and the last
// workgroup's sum of every workgroup's limbs, so a small matrix takes fewer,
// fuller workgroups (262,144 rows: 128 workgroups, the gradients 12.6 -> 9.5
// us per round); 10M rows still fill the chip.
constexpr uint32_t kGradRows = 2 * kGradThreads;

int mgb_gradients(const MgbGradParams* p, const float* margin, const float* labels, const float* weights,
                  float* grad, uint64_t* mass, float* scales) {
  uint32_t grid = grid_for(p->rows, kGradRows, kGradBlocks);
  launch(MGB_PROF_GRADIENT, k_gradients, dim3(grid), dim3(kGradThreads), 0, *p, margin, labels, weights,
         (float2*)grad, mass, scales);
  MGB_LAUNCH_CHECK("k_gradients");
  return 0;
}

int mgb_gradient_mass(const MgbGradParams* p, float* grad, uint64_t* mass, float* scales) {
  uint32_t grid = grid_for(p->rows, kGradRows, kGradBlocks);
  launch(MGB_PROF_GRADIENT, k_gradient_mass, dim3(grid), dim3(kGradThreads), 0, *p, (float2*)grad, mass, scales);
  MGB_LAUNCH_CHECK("k_gradient_mass");
  return 0;
}

int mgb_gradient_scales(uint64_t* mass, float* scales) {
  launch(MGB_PROF_GRADIENT, k_gradient_scales, dim3(1), dim3(512), 0, mass, scales);
  MGB_LAUNCH_CHECK("k_gradient_scales");
  return 0;
}

int mgb_base_score(const float* labels, const float* weights, uint32_t rows, uint32_t objective,
                   float scale_pos_weight, float* out) {
  const uint32_t grid = std::max<uint32_t>(1, std::min<uint32_t>(kBaseBlocks, (rows + kBaseThreads - 1) / kBaseThreads));
  hipLaunchKernelGGL(k_base_score, dim3(grid), dim3(kBaseThreads), 0, stream(), labels, weights, rows, objective,
                     scale_pos_weight, out);
  MGB_LAUNCH_CHECK("k_base_score");
  return 0;
}

int mgb_stream_copy(void* dst, const void* src, size_t bytes) {
  if (bytes % 16 || ((uintptr_t)dst % 16) || ((uintptr_t)src % 16)) {
    set_error("mgb_stream_copy: 16-byte aligned buffers and sizes only");
    return -1;
  }
  uint64_t n = bytes / 16;
  if (!n) return 0;
  hipLaunchKernelGGL(k_copy, dim3(grid_for(n, 256, 8192)), dim3(256), 0, stream(), (uint4*)dst, (const uint4*)src, n);
  MGB_LAUNCH_CHECK("k_copy");
  return 0;
}

int mgb_fill_f32(float* data, uint64_t count, float value) {
  if (!count) return 0;
  hipLaunchKernelGGL(k_fill, dim3(grid_for(count, 256)), dim3(256), 0, stream(), data, count, value);
  MGB_LAUNCH_CHECK("k_fill");
  return 0;
}

int mgb_any_missing(const float* data, uint64_t count, uint32_t* flag) {
  if (!count) return 0;
  hipLaunchKernelGGL(k_any_missing, dim3(grid_for(count, 256, 4096)), dim3(256), 0, stream(), data, count, flag);
  MGB_LAUNCH_CHECK("k_any_missing");
  return 0;
}

int mgb_transform(float* data, uint64_t count, uint32_t objective) {
  if (!count || objective != 1) return 0;
  hipLaunchKernelGGL(k_transform, dim3(grid_for(count, 256)), dim3(256), 0, stream(), data, count, objective);
  MGB_LAUNCH_CHECK("k_transform");
  return 0;
}

int mgb_predict(const float* X, uint32_t rows, uint32_t cols, const MgbTreeNode* nodes, const uint32_t* offsets,
                uint32_t trees, float* margin) {
  if (!rows || !trees) return 0;
  launch(MGB_PROF_PREDICT, k_predict, dim3(grid_for(rows, 256)), dim3(256), 0, X, rows, cols, nodes, offsets, trees,
         margin);
  MGB_LAUNCH_CHECK("k_predict");
  return 0;
}

}  // extern "C"
