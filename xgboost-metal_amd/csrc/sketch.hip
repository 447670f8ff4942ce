// Weighted quantile sketch on the GPU: the per-feature cut points of the
// reference's hist method (src/quantile.cpp:22-212, kernels/quantile.metal.h,
// XGBoost's WQSummary semantics).  Features are processed in groups of at
// most kChunkEntries entries; for each group:
//
//  1. (dense input) transpose the group's columns (coalesced reads per feature);
//  2. runs of equal values in row order over each feature's non-missing,
//     nonzero-weight entries, in 1024-entry blocks: per-block counts, a
//     per-feature scan over blocks that joins runs crossing block edges, the
//     runs written at their scanned offsets, then each run's weight (its
//     length, or the in-order binary32 sum of its entries' weights);
//  3. the host plans batches of 2*limit runs (limit = sketch budget) from the
//     per-feature counts;
//  4. a segmented, stable radix sort orders every batch's runs by value;
//  5. one workgroup per batch summarizes it and prunes the summary to limit;
//  6. the serial rule merges batch summaries through a stack of levels like a
//     binary counter (kernels/quantile.metal.h:317-352): while every merge
//     yields more than `limit` entries that is a balanced tree, computed here
//     one level per launch with one workgroup per node; a feature where some
//     merge yields fewer (many equal values) is redone serially by the
//     finishing kernel from its batch summaries;
//  7. one workgroup per feature merges the tree's roots (the stack's final
//     contents), prunes to the budget and selects the cuts.
// Summaries, prunes and merges are data-parallel restatements of the serial
// rules: prune positions come from binary searches over monotone rank sums,
// merges from merge-path ranks, the error fix-up from prefix maxima, and
// sequential binary32 sums stay sequential, so every rounding step is the
// same operation on the same operands.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "device_common.hpp"

namespace mgb {
namespace {

constexpr uint32_t kSketchThreads = 1024;
constexpr uint32_t kBlockEntries = 1024;                 // entries per workgroup in the run passes
constexpr uint64_t kChunkEntries = uint64_t(1) << 27;    // entries per group of features
constexpr uint32_t kMaxGroupFeatures = 65535;            // features per group
constexpr uint32_t kFinishLds = 96 * 1024;               // k_finish's staging LDS, at most

struct SkEntry { float rmin, rmax, wmin, value; };
struct SkStats { uint32_t nonmissing, elements, runs, padding; };

// Runs of one 1024-entry block of a feature.  `runs` counts the block's first
// valid entry as a run start; k_run_scan fills the offsets and the last valid
// value before the block.
struct SkBlock {
  uint32_t valid, present, runs, has;
  float first, last;
  uint32_t elem_off, run_off;
  uint32_t prev_has;
  float prev;
};

// Plan of one feature.  Tree node n (level l, index k: n = first(l) + k,
// first(l) = sum over j < l of batches >> j) covers batches
// [k 2^l, (k + 1) 2^l) and holds at most `limit` entries at
// tree + n * limit.
struct SkFeature {
  uint64_t base;        // first entry of the feature in the group's entry arrays
  uint64_t tree;        // first SkEntry of its tree nodes
  uint64_t fin;         // first SkEntry of its finishing buffers
  uint64_t scratch;     // first word of its per-node scratch (node k of a level: + k * (2 limit + 2))
  uint64_t fin_scratch; // first word of its finishing scratch
  uint32_t node_base;   // first slot of its node counts
  uint32_t limit, budget, batches;
  uint32_t levels;      // bit_width(batches) + 1: the serial stack's depth
  uint32_t exact;       // integer run weights summing below 2^24
  uint32_t final_cap;   // max(budget, limit)
  uint32_t padding;
};

__host__ __device__ inline uint32_t level_first(uint32_t batches, uint32_t level) {
  uint32_t s = 0;
  for (uint32_t j = 0; j < level && j < 32; ++j) s += batches >> j;
  return s;
}

__device__ __forceinline__ uint32_t order_key(float v) {
  uint32_t bits = __float_as_uint(v);
  return bits ^ ((bits & 0x80000000u) ? 0xffffffffu : 0x80000000u);
}
// The value of an order key (order_key's inverse).
__device__ __forceinline__ float key_value(uint32_t key) {
  return __uint_as_float(key ^ ((key & 0x80000000u) ? 0x80000000u : 0xffffffffu));
}
__device__ __forceinline__ float min_next(const SkEntry& e) { return e.rmin + e.wmin; }
__device__ __forceinline__ float max_prev(const SkEntry& e) { return e.rmax - e.wmin; }

// Columns [col0, col0 + ncols) of a row-major rows x cols matrix into
// column-major Xt (ncols columns of `rows` entries).
__global__ void k_transpose(const float* __restrict__ X, uint32_t rows, uint32_t cols, uint32_t col0, uint32_t ncols,
                            float* __restrict__ Xt) {
  __shared__ float tile[32][33];
  const uint32_t r0 = blockIdx.x * 32, c0 = blockIdx.y * 32;
  for (uint32_t k = threadIdx.y; k < 32; k += blockDim.y) {
    const uint32_t r = r0 + k, c = c0 + threadIdx.x;
    if (r < rows && c < ncols) tile[k][threadIdx.x] = X[(uint64_t)r * cols + col0 + c];
  }
  __syncthreads();
  for (uint32_t k = threadIdx.y; k < 32; k += blockDim.y) {
    const uint32_t c = c0 + k, r = r0 + threadIdx.x;
    if (r < rows && c < ncols) Xt[(uint64_t)c * rows + r] = tile[threadIdx.x][k];
  }
}

// One entry per thread of block blockIdx.x of feature blockIdx.y: is it
// present (not NaN) and valid (present with a nonzero weight), and the last
// valid value before it within the block.  Also the block's first and last
// valid values.  `s_*` hold one slot per wave.
struct EntryView {
  float v, w;
  bool present, valid, have_prev;
  float prev;
};

__device__ __forceinline__ EntryView view_entry(const float* __restrict__ vals, const uint64_t* __restrict__ seg,
                                                const uint32_t* __restrict__ row_of, const float* __restrict__ weights,
                                                uint32_t* s_has, float* s_first, float* s_last, bool& block_has,
                                                float& block_first, float& block_last) {
  const uint32_t c = blockIdx.y;
  const uint64_t base = seg[c];
  const uint32_t count = (uint32_t)(seg[c + 1] - base);
  const uint32_t r = blockIdx.x * kBlockEntries + threadIdx.x;
  const bool in = r < count;
  EntryView e;
  e.v = in ? vals[base + r] : __uint_as_float(0x7fc00000u);
  e.w = (in && weights) ? weights[row_of ? row_of[base + r] : r] : 1.0f;
  e.present = in && !isnan(e.v);
  e.valid = e.present && (__float_as_uint(e.w) & 0x7fffffffu) != 0;
  const uint32_t lane = lane_id(), wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
  const uint64_t mask = __ballot(e.valid);
  const uint64_t below = mask & ((uint64_t(1) << lane) - 1);
  e.prev = __shfl(e.v, below ? 63 - __clzll(below) : 0, kWave);
  e.have_prev = below != 0;
  const float first_in_wave = __shfl(e.v, mask ? __ffsll((long long)mask) - 1 : 0, kWave);
  const float last_in_wave = __shfl(e.v, mask ? 63 - __clzll(mask) : 0, kWave);
  if (lane == 0) {
    s_has[wave] = mask != 0;
    s_first[wave] = first_in_wave;
    s_last[wave] = last_in_wave;
  }
  __syncthreads();
  if (!e.have_prev) {
    for (int k = (int)wave - 1; k >= 0; --k)
      if (s_has[k]) { e.prev = s_last[k]; e.have_prev = true; break; }
  }
  block_has = false;
  for (uint32_t k = 0; k < waves; ++k)
    if (s_has[k]) { block_has = true; block_first = s_first[k]; break; }
  for (int k = (int)waves - 1; k >= 0; --k)
    if (s_has[k]) { block_last = s_last[k]; break; }
  return e;
}

__global__ __launch_bounds__(kSketchThreads) void k_run_count(const float* __restrict__ vals,
                                                              const uint64_t* __restrict__ seg,
                                                              const uint32_t* __restrict__ row_of,
                                                              const float* __restrict__ weights, uint32_t max_blocks,
                                                              SkBlock* __restrict__ blocks) {
  __shared__ uint32_t s_has[kSketchThreads / kWave], scan[kSketchThreads / kWave + 1];
  __shared__ float s_first[kSketchThreads / kWave], s_last[kSketchThreads / kWave];
  const uint32_t c = blockIdx.y;
  if ((uint64_t)blockIdx.x * kBlockEntries >= seg[c + 1] - seg[c]) return;  // the whole block is past the feature
  bool has = false;
  float first = 0.0f, last = 0.0f;
  const EntryView e = view_entry(vals, seg, row_of, weights, s_has, s_first, s_last, has, first, last);
  const bool new_run = e.valid && (!e.have_prev || e.v != e.prev);
  uint32_t valid, present, runs;
  block_exclusive_u32(e.valid ? 1u : 0u, scan, &valid);
  block_exclusive_u32(e.present ? 1u : 0u, scan, &present);
  block_exclusive_u32(new_run ? 1u : 0u, scan, &runs);
  if (threadIdx.x == 0) {
    SkBlock b{};
    b.valid = valid; b.present = present; b.runs = runs; b.has = has ? 1u : 0u;
    b.first = first; b.last = last;
    blocks[(uint64_t)c * max_blocks + blockIdx.x] = b;
  }
}

// One workgroup per feature: offsets of its blocks' elements and runs, with a
// block whose first valid value equals the last valid value before it
// continuing that run; the feature's totals.
__global__ __launch_bounds__(kSketchThreads) void k_run_scan(const uint64_t* __restrict__ seg, uint32_t max_blocks,
                                                             SkBlock* __restrict__ blocks,
                                                             SkStats* __restrict__ stats) {
  __shared__ uint32_t s_has[kSketchThreads / kWave], scan[kSketchThreads / kWave + 1];
  __shared__ float s_last[kSketchThreads / kWave];
  __shared__ uint32_t carry_has;
  __shared__ float carry_last;
  const uint32_t c = blockIdx.x;
  const uint64_t count = seg[c + 1] - seg[c];
  const uint32_t nblocks = (uint32_t)((count + kBlockEntries - 1) / kBlockEntries);
  SkBlock* fb = blocks + (uint64_t)c * max_blocks;
  const uint32_t lane = lane_id(), wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
  uint32_t elements = 0, runs = 0, present = 0;
  if (threadIdx.x == 0) { carry_has = 0; carry_last = 0.0f; }
  __syncthreads();
  for (uint32_t t0 = 0; t0 < nblocks; t0 += blockDim.x) {
    const uint32_t b = t0 + threadIdx.x;
    const bool in = b < nblocks;
    SkBlock blk{};
    if (in) blk = fb[b];
    const bool has = in && blk.has;
    const uint64_t mask = __ballot(has);
    const uint64_t below = mask & ((uint64_t(1) << lane) - 1);
    float prev = __shfl(blk.last, below ? 63 - __clzll(below) : 0, kWave);
    bool have_prev = below != 0;
    const float last_in_wave = __shfl(blk.last, mask ? 63 - __clzll(mask) : 0, kWave);
    if (lane == 0) { s_has[wave] = mask != 0; s_last[wave] = last_in_wave; }
    __syncthreads();
    if (!have_prev) {
      for (int k = (int)wave - 1; k >= 0; --k)
        if (s_has[k]) { prev = s_last[k]; have_prev = true; break; }
      if (!have_prev && carry_has) { prev = carry_last; have_prev = true; }
    }
    const uint32_t adj = in ? blk.runs - ((has && have_prev && blk.first == prev) ? 1u : 0u) : 0u;
    uint32_t te, tr, tp;
    const uint32_t eoff = elements + block_exclusive_u32(in ? blk.valid : 0u, scan, &te);
    const uint32_t roff = runs + block_exclusive_u32(adj, scan, &tr);
    block_exclusive_u32(in ? blk.present : 0u, scan, &tp);
    if (in) {
      fb[b].elem_off = eoff;
      fb[b].run_off = roff;
      fb[b].prev_has = have_prev ? 1u : 0u;
      fb[b].prev = prev;
    }
    elements += te;
    runs += tr;
    present += tp;
    __syncthreads();
    if (threadIdx.x == 0)
      for (int k = (int)waves - 1; k >= 0; --k)
        if (s_has[k]) { carry_has = 1; carry_last = s_last[k]; break; }
    __syncthreads();
  }
  if (threadIdx.x == 0) stats[c] = SkStats{present, elements, runs, 0};
}

// The runs of each block at their scanned offsets: run_v (value), run_start
// (element index within the feature) and, with weights, each valid entry's
// weight at its element index.
__global__ __launch_bounds__(kSketchThreads) void k_run_emit(const float* __restrict__ vals,
                                                             const uint64_t* __restrict__ seg,
                                                             const uint32_t* __restrict__ row_of,
                                                             const float* __restrict__ weights, uint32_t max_blocks,
                                                             const SkBlock* __restrict__ blocks,
                                                             float* __restrict__ run_v, uint32_t* __restrict__ run_start,
                                                             float* __restrict__ elem_w) {
  __shared__ uint32_t s_has[kSketchThreads / kWave], scan[kSketchThreads / kWave + 1];
  __shared__ float s_first[kSketchThreads / kWave], s_last[kSketchThreads / kWave];
  const uint32_t c = blockIdx.y;
  const uint64_t base = seg[c];
  if ((uint64_t)blockIdx.x * kBlockEntries >= seg[c + 1] - base) return;
  const SkBlock blk = blocks[(uint64_t)c * max_blocks + blockIdx.x];
  bool has = false;
  float first = 0.0f, last = 0.0f;
  EntryView e = view_entry(vals, seg, row_of, weights, s_has, s_first, s_last, has, first, last);
  if (!e.have_prev && blk.prev_has) { e.prev = blk.prev; e.have_prev = true; }
  const bool new_run = e.valid && (!e.have_prev || e.v != e.prev);
  uint32_t tv, tr;
  const uint32_t eidx = blk.elem_off + block_exclusive_u32(e.valid ? 1u : 0u, scan, &tv);
  const uint32_t ridx = blk.run_off + block_exclusive_u32(new_run ? 1u : 0u, scan, &tr);
  if (new_run) {
    run_v[base + ridx] = e.v;
    run_start[base + ridx] = eidx;
  }
  if (e.valid && weights) elem_w[base + eidx] = e.w;
}

// Each run's weight: its length (below 2^24) or, with weights, the binary32
// sum of its entries' weights in row order (kernels/quantile.metal.h:19-140).
__global__ void k_run_weights(const uint64_t* __restrict__ seg, const SkStats* __restrict__ stats,
                              const uint32_t* __restrict__ run_start, const float* __restrict__ elem_w,
                              float* __restrict__ run_w) {
  const uint32_t c = blockIdx.y;
  const uint64_t base = seg[c];
  const SkStats st = stats[c];
  const uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= st.runs) return;
  const uint32_t s = run_start[base + k];
  const uint32_t e = k + 1 < st.runs ? run_start[base + k + 1] : st.elements;
  float w;
  if (!elem_w) {
    const uint32_t len = e - s;
    w = (float)(len < (1u << 24) ? len : (1u << 24));
  } else {
    w = elem_w[base + s];
    for (uint32_t i = s + 1; i < e; ++i) w = w + elem_w[base + i];
  }
  run_w[base + k] = w;
}

// Sort keys (value order) and payloads (the run's weight) of every run: the
// stable sort hands the summaries each batch's values and weights in value
// order, contiguous, with equal values in run order.
__global__ void k_sort_keys(const uint64_t* __restrict__ seg, const SkStats* __restrict__ stats,
                            const float* __restrict__ run_v, const float* __restrict__ run_w,
                            uint32_t* __restrict__ keys, float* __restrict__ weight) {
  const uint32_t c = blockIdx.y;
  const uint64_t base = seg[c];
  const uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= stats[c].runs) return;
  keys[base + k] = order_key(run_v[base + k]);
  weight[base + k] = run_w[base + k];
}

__device__ __forceinline__ uint32_t block_inclusive_max_u32(uint32_t v, uint32_t* shared) {
  const uint32_t lane = lane_id(), wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    uint32_t o = __shfl_up(v, d, kWave);
    if (lane >= (uint32_t)d) v = o > v ? o : v;
  }
  if (lane == kWave - 1) shared[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (uint32_t w = 0; w < waves; ++w) {
      uint32_t t = shared[w];
      shared[w] = run;
      run = t > run ? t : run;
    }
  }
  __syncthreads();
  uint32_t before = shared[wave];
  __syncthreads();
  return before > v ? before : v;
}

// Two-level searches over a sorted summary: every s-th search key staged in
// LDS (kSamples at most) narrows a bound to a window of fewer than s entries,
// which a search over global memory finishes -- the same index as one binary
// search over the whole array, with log2(s) dependent global loads instead of
// log2(size) (a 41K-entry summary: 5 instead of 16).
constexpr uint32_t kSamples = 2048;

__device__ __forceinline__ uint32_t sample_stride(uint32_t size) {
  uint32_t s = 16;
  while ((uint64_t)s * kSamples < size) s <<= 1;
  return s;
}

// smp[t] = arr[t * s].value for t < ceil(m / s).  Call with the whole
// workgroup; the caller synchronizes before reading smp.
__device__ __forceinline__ void sample_values(const SkEntry* arr, uint32_t m, uint32_t s, float* smp) {
  const uint32_t samples = (m + s - 1) / s;
  for (uint32_t t = threadIdx.x; t < samples; t += blockDim.x) smp[t] = arr[(uint64_t)t * s].value;
}

// First i in [0, m) with !(arr[i].value < x), arr sorted by value.
__device__ __forceinline__ uint32_t lower_bound_sampled(const SkEntry* arr, uint32_t m, const float* smp, uint32_t s,
                                                        float x) {
  const uint32_t samples = (m + s - 1) / s;
  uint32_t lo = 0, hi = samples;  // first sample t with !(smp[t] < x)
  while (lo < hi) {
    const uint32_t mid = lo + (hi - lo) / 2;
    if (smp[mid] < x) lo = mid + 1;
    else hi = mid;
  }
  const uint32_t t = lo;
  lo = t == 0 ? 0u : (t - 1) * s + 1;
  hi = t < samples ? t * s : m;
  while (lo < hi) {
    const uint32_t mid = lo + (hi - lo) / 2;
    if (arr[mid].value < x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// kernels/quantile.metal.h:192-214 (sketch_prune_serial), data-parallel.
// The serial loop walks i forward while rank_k >= rmax_{i+1} + rmin_{i+1};
// both ranks and these sums are nondecreasing, so i_k is a binary search and
// the chosen indices c_k are nondecreasing: "append if c_k != last" keeps the
// first k of each run of equal c_k.  in[0..size) -> out (out != in).
__device__ uint32_t prune(const SkEntry* in, uint32_t size, uint32_t capacity, SkEntry* out, uint32_t* scan,
                          float* smp) {
  __shared__ uint32_t s_last, s_dead;
  __shared__ uint32_t s_wave_tail[kSketchThreads / kWave];
  if (size <= capacity) {
    for (uint32_t i = threadIdx.x; i < size; i += blockDim.x) out[i] = in[i];
    __syncthreads();
    return size;
  }
  if (!capacity) return 0;
  if (capacity == 1) {
    if (threadIdx.x == 0) out[0] = in[0];
    __syncthreads();
    return 1;
  }
  const float begin = in[0].rmax, range = in[size - 1].rmin - begin;
  const uint32_t n = capacity - 1;
  const uint32_t lane = lane_id(), wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
  // Sampled keys rmax_j + rmin_j at j = 2 + t * stride.
  const uint32_t stride = sample_stride(size), samples = size > 2 ? (size - 2 + stride - 1) / stride : 0;
  __syncthreads();  // smp may still be read by the previous search
  for (uint32_t t = threadIdx.x; t < samples; t += blockDim.x) {
    const SkEntry& e = in[2 + (uint64_t)t * stride];
    smp[t] = e.rmax + e.rmin;
  }
  if (threadIdx.x == 0) { out[0] = in[0]; s_last = 0; s_dead = 0; }
  __syncthreads();
  uint32_t carry = 0, prev_chunk = 0;
  for (uint32_t base = 1; base < n; base += blockDim.x) {
    const uint32_t k = base + threadIdx.x;
    uint32_t choice = 0;
    bool live = false;
    if (k < n) {
      const float rank = 2.0f * (((float)k * range) / (float)n + begin);
      // First j in [2, size) with rank < rmax_j + rmin_j: the first sample
      // above rank bounds it from above, the one before from below.
      uint32_t lo = 0, hi = samples;
      while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (rank >= smp[mid]) lo = mid + 1;
        else hi = mid;
      }
      const uint32_t t = lo;
      lo = t == 0 ? 2u : 2 + (t - 1) * stride + 1;
      hi = t < samples ? 2 + t * stride : size;
      while (lo < hi) {
        uint32_t mid = lo + (hi - lo) / 2;
        if (rank >= in[mid].rmax + in[mid].rmin) lo = mid + 1;
        else hi = mid;
      }
      const uint32_t i = lo - 1;
      if (i < size - 1) {
        live = true;
        choice = rank < min_next(in[i]) + max_prev(in[i + 1]) ? i : i + 1;
      }
    }
    uint32_t prev = __shfl_up(choice, 1, kWave);
    if (lane == kWave - 1) s_wave_tail[wave] = choice;
    __syncthreads();
    if (lane == 0) prev = wave == 0 ? prev_chunk : s_wave_tail[wave - 1];
    const uint32_t chunk_tail = s_wave_tail[waves - 1];
    const bool emit = live && choice != prev;
    uint32_t total;
    const uint32_t off = block_exclusive_u32(emit ? 1u : 0u, scan, &total);
    if (emit) out[1 + carry + off] = in[choice];
    carry += total;
    if (live) atomicMax(&s_last, choice);
    if (k < n && !live) s_dead = 1;
    __syncthreads();
    prev_chunk = chunk_tail;
    if (s_dead) break;
  }
  __syncthreads();
  uint32_t count = 1 + carry;
  const bool tail = s_last != size - 1;
  __syncthreads();
  if (tail) {
    if (threadIdx.x == 0) out[count] = in[size - 1];
    ++count;
  }
  __syncthreads();
  return count;
}

// kernels/quantile.metal.h:266-311 (sketch_combine_serial), merge-path form.
// a[0..n) and b[0..m) -> out; out must differ from both.  eq_prefix needs
// 2n + 1 words.
__device__ uint32_t combine(const SkEntry* a, uint32_t n, const SkEntry* b, uint32_t m, SkEntry* out,
                            uint32_t* eq_prefix, uint32_t* scan, float* smp) {
  if (!m) {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) out[i] = a[i];
    __syncthreads();
    return n;
  }
  if (!n) {
    for (uint32_t i = threadIdx.x; i < m; i += blockDim.x) out[i] = b[i];
    __syncthreads();
    return m;
  }
  // Sampled values of both summaries (b's in smp, a's in smp + kSamples).
  const uint32_t sb = sample_stride(m), sa = sample_stride(n);
  float* smp_b = smp;
  float* smp_a = smp + kSamples;
  __syncthreads();  // smp may still be read by the previous search
  sample_values(b, m, sb, smp_b);
  sample_values(a, n, sa, smp_a);
  __syncthreads();
  // Equal-value pairs, indexed by a: eq_prefix[i] = #pairs with a-index < i;
  // each a value's position in b kept in rank_a for the placement below.
  uint32_t* rank_a = eq_prefix + n + 1;
  uint32_t carry = 0;
  for (uint32_t base = 0; base < n; base += blockDim.x) {
    uint32_t i = base + threadIdx.x;
    uint32_t eq = 0;
    if (i < n) {
      float x = a[i].value;
      const uint32_t lo = lower_bound_sampled(b, m, smp_b, sb, x);
      rank_a[i] = lo;
      eq = lo < m && b[lo].value == x;
    }
    uint32_t total;
    uint32_t off = block_exclusive_u32(eq, scan, &total);
    if (i < n) eq_prefix[i] = carry + off;
    carry += total;
  }
  if (threadIdx.x == 0) eq_prefix[n] = carry;
  __syncthreads();
  const uint32_t count = n + m - carry;
  const float tail_a = a[n - 1].rmax, tail_b = b[m - 1].rmax;
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
    const SkEntry x = a[i];
    const uint32_t lo = rank_a[i];
    SkEntry r;
    if (lo < m && b[lo].value == x.value) {
      const SkEntry y = b[lo];
      r.rmin = x.rmin + y.rmin; r.rmax = x.rmax + y.rmax; r.wmin = x.wmin + y.wmin; r.value = x.value;
    } else {
      float prev_b = lo > 0 ? min_next(b[lo - 1]) : 0.0f;
      float add = lo < m ? max_prev(b[lo]) : tail_b;
      r.rmin = x.rmin + prev_b; r.rmax = x.rmax + add; r.wmin = x.wmin; r.value = x.value;
    }
    out[i + lo - eq_prefix[i]] = r;
  }
  for (uint32_t j = threadIdx.x; j < m; j += blockDim.x) {
    const SkEntry y = b[j];
    const uint32_t lo = lower_bound_sampled(a, n, smp_a, sa, y.value);
    if (lo < n && a[lo].value == y.value) continue;
    float prev_a = lo > 0 ? min_next(a[lo - 1]) : 0.0f;
    float add = lo < n ? max_prev(a[lo]) : tail_a;
    SkEntry r;
    r.rmin = y.rmin + prev_a; r.rmax = y.rmax + add; r.wmin = y.wmin; r.value = y.value;
    out[j + lo - eq_prefix[lo]] = r;
  }
  __syncthreads();
  // Error fix-up: rmin = prefix max of rmin; rmax = prefix max of
  // max(rmax, rmin' + wmin).  All values are nonnegative, so binary32 order
  // equals the order of their bit patterns.
  uint32_t run_min = 0, run_max = 0;
  for (uint32_t base = 0; base < count; base += blockDim.x) {
    uint32_t i = base + threadIdx.x;
    SkEntry e;
    uint32_t kmin = 0;
    if (i < count) { e = out[i]; kmin = __float_as_uint(e.rmin); }
    uint32_t pmin = block_inclusive_max_u32(kmin, scan);
    pmin = pmin > run_min ? pmin : run_min;
    uint32_t kmax = 0;
    if (i < count) {
      e.rmin = __uint_as_float(pmin);
      float a2 = e.rmin + e.wmin;
      kmax = __float_as_uint(e.rmax > a2 ? e.rmax : a2);
    }
    uint32_t pmax = block_inclusive_max_u32(kmax, scan);
    pmax = pmax > run_max ? pmax : run_max;
    __syncthreads();
    if (i < count) {
      e.rmax = __uint_as_float(pmax);
      out[i] = e;
    }
    // Carry the chunk's last prefix values.
    __shared__ uint32_t carry_min, carry_max;
    if (threadIdx.x == blockDim.x - 1 || i == count - 1) { carry_min = pmin; carry_max = pmax; }
    __syncthreads();
    run_min = carry_min;
    run_max = carry_max;
    __syncthreads();
  }
  return count;
}


// Summary of one sorted batch (kernels/quantile.metal.h:216-240): one entry
// per distinct value, in value order, holding the value's weight w (the
// binary32 sum of its runs' weights in sort order) and the running binary32
// total before (rmin) and after (rmax) it.  keys[0..size) and wts[0..size)
// are the batch's runs' order keys and weights in value order; scratch needs
// size + 1 words.
__device__ uint32_t summarize(const uint32_t* __restrict__ keys, const float* __restrict__ wts, uint32_t size,
                              bool exact, SkEntry* out,
                              uint32_t* scratch, uint32_t* scan) {
  // Group starts (value changes in sort order) and each group's first
  // position; with integer weights summing below 2^24 (exact) also each
  // group's weight prefix, since every binary32 partial sum is then exact and
  // a parallel prefix gives the serial sums bit for bit.
  uint32_t carry_w = 0, carry_s = 0;
  for (uint32_t base = 0; base < size; base += blockDim.x) {
    const uint32_t i = base + threadIdx.x;
    uint32_t w = 0, start = 0;
    float v = 0.0f;
    if (i < size) {
      v = key_value(keys[i]);
      if (exact) w = (uint32_t)wts[i];
      start = i == 0 || key_value(keys[i - 1]) != v;
    }
    uint32_t tw = 0, ts;
    const uint32_t pw = (exact ? block_exclusive_u32(w, scan, &tw) : 0u) + carry_w;
    const uint32_t ps = block_exclusive_u32(start, scan, &ts) + carry_s;
    if (start) {
      scratch[ps] = exact ? pw : i;
      out[ps].value = v;
    }
    carry_w += tw;
    carry_s += ts;
  }
  if (threadIdx.x == 0) scratch[carry_s] = exact ? carry_w : size;
  __syncthreads();
  const uint32_t n = carry_s;
  if (exact) {
    for (uint32_t o = threadIdx.x; o < n; o += blockDim.x) {
      const uint32_t p = scratch[o], q = scratch[o + 1];
      out[o].rmin = (float)p;
      out[o].rmax = (float)q;
      out[o].wmin = (float)(q - p);
    }
    __syncthreads();
    return n;
  }
  // Each group's weight: its runs' weights summed in sort order.
  for (uint32_t o = threadIdx.x; o < n; o += blockDim.x) {
    const uint32_t s = scratch[o], e = scratch[o + 1];
    float w = wts[s];
    for (uint32_t i = s + 1; i < e; ++i) w = w + wts[i];
    out[o].wmin = w;
  }
  __syncthreads();
  // The running total, strictly in order: wave 0 loads 64 weights at a time
  // and every lane applies the same 64 additions in sequence.
  if (threadIdx.x < kWave) {
    const uint32_t lane = threadIdx.x;
    float total = 0.0f;
    for (uint32_t g0 = 0; g0 < n; g0 += kWave) {
      const uint32_t g = g0 + lane;
      const float w = g < n ? out[g].wmin : 0.0f;
      const uint32_t count = n - g0 < kWave ? n - g0 : kWave;
      float before = 0.0f, after = 0.0f;
      for (uint32_t j = 0; j < count; ++j) {
        const float wj = __shfl(w, (int)j, kWave);
        if (lane == j) before = total;
        total = total + wj;
        if (lane == j) after = total;
      }
      if (g < n) {
        out[g].rmin = before;
        out[g].rmax = after;
      }
    }
  }
  __syncthreads();
  return n;
}

// Level 0 of every feature's tree: one workgroup per batch summarizes the
// batch's sorted runs into the feature's work area and prunes the summary to
// `limit` entries (the serial rule's first step for each batch,
// kernels/quantile.metal.h:317-352).
__global__ __launch_bounds__(kSketchThreads) void k_level0(const uint32_t* __restrict__ table,
                                                           const SkFeature* __restrict__ features,
                                                           const SkStats* __restrict__ stats,
                                                           const uint32_t* __restrict__ keys,
                                                           const float* __restrict__ wts, SkEntry* __restrict__ work,
                                                           SkEntry* __restrict__ tree, uint32_t* __restrict__ scratch,
                                                           uint32_t* __restrict__ node_count) {
  __shared__ uint32_t scan[kSketchThreads / kWave + 1];
  __shared__ float s_smp[2 * kSamples];
  const uint32_t c = table[2 * blockIdx.x], b = table[2 * blockIdx.x + 1];
  const SkFeature fe = features[c];
  const uint64_t begin = (uint64_t)b * 2 * fe.limit;
  const uint32_t runs = stats[c].runs;
  const uint32_t size = (uint32_t)(runs - begin < 2ull * fe.limit ? runs - begin : 2ull * fe.limit);
  SkEntry* summary = work + fe.base + begin;
  const uint32_t n = summarize(keys + fe.base + begin, wts + fe.base + begin, size, fe.exact != 0, summary,
                               scratch + fe.scratch + (uint64_t)b * (2 * fe.limit + 2), scan);
  const uint32_t m = prune(summary, n, fe.limit, tree + fe.tree + (uint64_t)b * fe.limit, scan, s_smp);
  if (threadIdx.x == 0) node_count[fe.node_base + b] = m;
}

// Level `level` >= 1: node k merges nodes 2k + 1 and 2k of the level below
// (the serial rule's merge of a new summary into an occupied level) and
// prunes the merge to `limit`.  A merge of at most `limit` entries stays at
// its level in the serial rule instead of moving up, so the tree no longer
// matches it: the feature is marked for the serial rebuild.
__global__ __launch_bounds__(kSketchThreads) void k_level_up(uint32_t level, const uint32_t* __restrict__ table,
                                                             const SkFeature* __restrict__ features,
                                                             SkEntry* __restrict__ work, SkEntry* __restrict__ tree,
                                                             uint32_t* __restrict__ scratch,
                                                             uint32_t* __restrict__ node_count,
                                                             uint32_t* __restrict__ serial) {
  __shared__ uint32_t scan[kSketchThreads / kWave + 1];
  __shared__ float s_smp[2 * kSamples];
  __shared__ uint32_t s_serial;
  const uint32_t c = table[2 * blockIdx.x], k = table[2 * blockIdx.x + 1];
  // Other workgroups of this level may set the flag meanwhile: one read,
  // shared, so the whole workgroup takes the same branch.
  if (threadIdx.x == 0) s_serial = serial[c];
  __syncthreads();
  if (s_serial) return;
  const SkFeature fe = features[c];
  const uint32_t below = level_first(fe.batches, level - 1), here = level_first(fe.batches, level);
  const uint32_t newer = below + 2 * k + 1, older = below + 2 * k;
  const uint32_t na = node_count[fe.node_base + newer], nb = node_count[fe.node_base + older];
  SkEntry* merged = work + fe.base + (uint64_t)k * 2 * fe.limit;
  const uint32_t n = combine(tree + fe.tree + (uint64_t)newer * fe.limit, na, tree + fe.tree + (uint64_t)older * fe.limit,
                             nb, merged, scratch + fe.scratch + (uint64_t)k * (2 * fe.limit + 2), scan, s_smp);
  if (n <= fe.limit) {
    if (threadIdx.x == 0) atomicOr(&serial[c], 1u);
    return;
  }
  const uint32_t m = prune(merged, n, fe.limit, tree + fe.tree + (uint64_t)(here + k) * fe.limit, scan, s_smp);
  if (threadIdx.x == 0) node_count[fe.node_base + here + k] = m;
}

// One workgroup per feature: the stack's final contents merged level by level
// with a prune to max(budget, limit) after each, a prune to the budget, and
// the cuts (kernels/quantile.metal.h:317-400).  The stack holds, at each level
// l whose bit is set in the batch count, the tree node over the last complete
// 2^l batches; a feature marked serial first replays the serial rule over its
// batch summaries.
__global__ __launch_bounds__(kSketchThreads) void k_finish(const SkFeature* __restrict__ features,
                                                           const SkEntry* __restrict__ tree,
                                                           const uint32_t* __restrict__ node_count,
                                                           const uint32_t* __restrict__ serial,
                                                           SkEntry* __restrict__ fin, uint32_t* __restrict__ fin_scratch,
                                                           uint32_t f0, uint32_t max_bin, float* __restrict__ cut_values,
                                                           uint32_t lds_values, float* __restrict__ cuts,
                                                           uint32_t* __restrict__ counts) {
  __shared__ uint32_t scan[kSketchThreads / kWave + 1];
  __shared__ float s_smp[2 * kSamples];
  __shared__ uint32_t level_count[64];
  // lds_values summary values, then max_bin candidate cuts (0 bytes when
  // lds_values is 0).
  extern __shared__ float s_stage[];
  const uint32_t c = blockIdx.x;
  const SkFeature fe = features[c];
  const uint32_t limit = fe.limit, batches = fe.batches;
  const uint64_t buf = 2ull * fe.final_cap + 2;
  SkEntry* cur = fin + fe.fin;
  SkEntry* oth = cur + buf;
  SkEntry* lvl = oth + buf;  // the serial stack: (levels + 1) x limit
  uint32_t* scr = fin_scratch + fe.fin_scratch;
  uint32_t n = 0;
  if (batches && !serial[c]) {
    for (uint32_t level = 0; level < fe.levels && level < 32; ++level) {
      if ((batches >> level) & 1u) {
        const uint32_t node = level_first(batches, level) + (batches >> level) - 1;
        n = combine(cur, n, tree + fe.tree + (uint64_t)node * limit, node_count[fe.node_base + node], oth, scr, scan,
                    s_smp);
        SkEntry* t = cur; cur = oth; oth = t;
      }
      n = prune(cur, n, fe.final_cap, oth, scan, s_smp);
      SkEntry* t = cur; cur = oth; oth = t;
    }
  } else if (batches) {
    for (uint32_t i = threadIdx.x; i < 64; i += blockDim.x) level_count[i] = 0;
    __syncthreads();
    for (uint32_t b = 0; b < batches; ++b) {
      n = node_count[fe.node_base + b];
      const SkEntry* src = tree + fe.tree + (uint64_t)b * limit;
      for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) cur[i] = src[i];
      __syncthreads();
      uint32_t level = 0;
      for (;;) {
        const uint32_t m = level_count[level];
        if (m) {
          n = combine(cur, n, lvl + (uint64_t)level * limit, m, oth, scr, scan, s_smp);
          SkEntry* t = cur; cur = oth; oth = t;
        }
        __syncthreads();
        if (threadIdx.x == 0) level_count[level] = 0;
        __syncthreads();
        if (n <= limit) break;
        ++level;
        n = prune(cur, n, limit, oth, scan, s_smp);
        SkEntry* t = cur; cur = oth; oth = t;
      }
      for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) lvl[(uint64_t)level * limit + i] = cur[i];
      __syncthreads();
      if (threadIdx.x == 0) level_count[level] = n;
      __syncthreads();
    }
    n = 0;
    for (uint32_t level = 0; level < fe.levels && level < 64; ++level) {
      const uint32_t m = level_count[level];
      if (m) {
        n = combine(cur, n, lvl + (uint64_t)level * limit, m, oth, scr, scan, s_smp);
        SkEntry* t = cur; cur = oth; oth = t;
      }
      n = prune(cur, n, fe.final_cap, oth, scan, s_smp);
      SkEntry* t = cur; cur = oth; oth = t;
    }
  }
  n = prune(cur, n, fe.budget, oth, scan, s_smp);
  { SkEntry* t = cur; cur = oth; oth = t; }
  // Cuts (kernels/quantile.metal.h:354-400).
  const uint32_t f = f0 + c;
  float* out = cuts + (uint64_t)f * max_bin;
  for (uint32_t i = threadIdx.x; i < max_bin; i += blockDim.x) out[i] = 0.0f;
  __syncthreads();
  if (!n) {
    if (threadIdx.x == 0) { out[0] = 1e-5f; counts[f] = 1; }
    return;
  }
  const uint32_t size = n;
  if (size <= max_bin) {
    for (uint32_t i = 1 + threadIdx.x; i < size; i += blockDim.x) out[i - 1] = cur[i].value;
    __syncthreads();
    if (threadIdx.x == 0) {
      const float tail = cur[size - 1].value;
      out[size - 1] = tail + (fabsf(tail) + 1e-5f);
      counts[f] = size;
    }
    return;
  }
  // Rank queries in parallel; the order-preserving dedup pass is serial, on
  // values staged in LDS when they fit.
  const bool staged = size <= lds_values;
  float* values = staged ? s_stage + lds_values : cut_values + (uint64_t)c * max_bin;
  if (staged)
    for (uint32_t i = threadIdx.x; i < size; i += blockDim.x) s_stage[i] = cur[i].value;
  const double total = (double)cur[size - 1].rmax, denominator = (double)max_bin;
  for (uint32_t i = 1 + threadIdx.x; i < max_bin; i += blockDim.x) {
    const double rank = ((double)i * total) / denominator * 2.0;
    uint32_t lo = 1, hi = size - 1;  // cursor = #{j in [1, size-2] : rmin_j + rmax_j <= rank}
    while (lo < hi) {
      const uint32_t mid = lo + (hi - lo) / 2;
      if (rank >= (double)(cur[mid].rmin + cur[mid].rmax)) lo = mid + 1;
      else hi = mid;
    }
    const uint32_t cursor = lo - 1;
    const float boundary = min_next(cur[cursor]) + max_prev(cur[cursor + 1]);
    values[i] = cur[cursor + ((isnan(boundary) || rank >= (double)boundary) ? 1u : 0u)].value;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    auto entry = [&](uint32_t j) { return staged ? s_stage[j] : cur[j].value; };
    float last = entry(0);
    uint32_t next = 1, count = 0;
    for (uint32_t i = 1; i < max_bin; ++i) {
      float value = values[i];
      if (value <= last) {
        while (next < size && entry(next) <= last) ++next;
        if (next == size) break;
        value = entry(next);
      } else if (next < size && entry(next) <= value) {
        do { ++next; } while (next < size && entry(next) <= value);
      }
      out[count++] = value;
      last = value;
    }
    const float tail = cur[size - 1].value;
    out[count++] = tail + (fabsf(tail) + 1e-5f);
    counts[f] = count;
  }
}

uint32_t sketch_budget(uint32_t bins, uint32_t count) {
  if (!count) return 1;
  double epsilon = 1.0 / (double)std::min(bins, count);
  for (uint32_t level = 1; level < 32; ++level) {
    uint64_t limit = std::min<uint64_t>(count, (uint64_t)std::ceil(level / (epsilon / 2.0)) + 1);
    if ((uint64_t{1} << level) * limit >= count) return (uint32_t)limit;
  }
  return count;
}

uint32_t bit_width(uint32_t v) { return v ? 32u - (uint32_t)__builtin_clz(v) : 0u; }

// Device memory of one sketch pass, allocated and freed in order on the
// library stream: a free is queued behind the kernels that use the buffer
// instead of waiting for the device, and the memory pool keeps it for the
// next pass.
struct StreamBuffer {
  void* p = nullptr;
  StreamBuffer() = default;
  StreamBuffer(const StreamBuffer&) = delete;
  StreamBuffer& operator=(const StreamBuffer&) = delete;
  ~StreamBuffer() {
    if (p) (void)hipFreeAsync(p, stream());
  }
  int alloc(size_t bytes) { return check(hipMallocAsync(&p, bytes ? bytes : 16, stream()), "hipMallocAsync(sketch)"); }
  template <typename T> T* as() const { return static_cast<T*>(p); }
};

// Buffers carved from one stream-ordered allocation: reserve() hands out
// 256-byte-aligned offsets, commit() allocates once.  Host tables are
// gathered into a staging image of the arena's first bytes and copied in one
// transfer.
struct Arena {
  StreamBuffer buffer;
  uint64_t size = 0;
  std::vector<uint8_t> staged;  // host image of [0, staged.size())
  uint64_t reserve(uint64_t bytes) {
    const uint64_t off = size;
    size += (std::max<uint64_t>(bytes, 1) + 255) / 256 * 256;
    return off;
  }
  template <typename T>
  uint64_t stage(const std::vector<T>& src) {
    const uint64_t off = reserve(src.size() * sizeof(T));
    staged.resize(size);
    if (!src.empty()) std::memcpy(staged.data() + off, src.data(), src.size() * sizeof(T));
    return off;
  }
  int commit() {
    if (buffer.alloc(size)) return -1;
    if (!staged.empty())
      MGB_CHECK(hipMemcpyAsync(buffer.p, staged.data(), staged.size(), hipMemcpyHostToDevice, stream()));
    return 0;
  }
  template <typename T> T* at(uint64_t off) const { return reinterpret_cast<T*>(buffer.as<uint8_t>() + off); }
};

// Cuts of the features f0 .. f0 + nf - 1 whose entries are
// vals[seg[c] .. seg[c + 1]) (device values; host offsets, seg[0] = 0), see
// view_entry for the meaning of row_of and weights.
int sketch_group(const float* vals, const std::vector<uint64_t>& seg, const uint32_t* row_of, uint32_t nf, uint32_t f0,
                 const float* weights, uint32_t max_bin, float* cuts, uint32_t* counts) {
  hipStream_t s = stream();
  const uint64_t total = seg[nf];
  // Positions are 32-bit and the segmented sort counts in int.
  if (total >= (1ull << 31)) { set_error("sketch: more than 2^31 - 1 entries in one group"); return -1; }
  uint64_t longest = 0;
  for (uint32_t c = 0; c < nf; ++c) longest = std::max<uint64_t>(longest, seg[c + 1] - seg[c]);
  const uint32_t max_blocks = (uint32_t)std::max<uint64_t>(1, (longest + kBlockEntries - 1) / kBlockEntries);
  const uint64_t E = total ? total : 1;
  Arena a1;
  const uint64_t o_seg = a1.stage(seg);
  const uint64_t o_blocks = a1.reserve((uint64_t)nf * max_blocks * sizeof(SkBlock));
  const uint64_t o_stats = a1.reserve(nf * sizeof(SkStats));
  const uint64_t o_run_v = a1.reserve(E * 4), o_run_w = a1.reserve(E * 4);
  const uint64_t o_region = a1.reserve(E * 16);
  const uint64_t o_keys_out = a1.reserve(E * 4), o_weight_out = a1.reserve(E * 4);
  if (a1.commit()) return -1;
  const uint64_t* seg_d = a1.at<uint64_t>(o_seg);
  SkBlock* blocks = a1.at<SkBlock>(o_blocks);
  SkStats* stats_d = a1.at<SkStats>(o_stats);
  float* run_v = a1.at<float>(o_run_v);
  float* run_w = a1.at<float>(o_run_w);
  uint32_t* keys_out = a1.at<uint32_t>(o_keys_out);
  uint32_t* weight_out = a1.at<uint32_t>(o_weight_out);
  // One 16-byte-per-entry region: run starts, sort inputs and entry weights
  // until the sort, then the summaries' and merges' work area.
  uint32_t* run_start = a1.at<uint32_t>(o_region);
  uint32_t* keys_in = run_start + E;
  uint32_t* weight_in = keys_in + E;
  float* elem_w = reinterpret_cast<float*>(weight_in + E);
  SkEntry* work = a1.at<SkEntry>(o_region);
  const dim3 grid(max_blocks, nf);
  hipLaunchKernelGGL(k_run_count, grid, dim3(kSketchThreads), 0, s, vals, seg_d, row_of, weights,
                     max_blocks, blocks);
  MGB_LAUNCH_CHECK("k_run_count");
  hipLaunchKernelGGL(k_run_scan, dim3(nf), dim3(kSketchThreads), 0, s, seg_d, max_blocks,
                     blocks, stats_d);
  MGB_LAUNCH_CHECK("k_run_scan");
  hipLaunchKernelGGL(k_run_emit, grid, dim3(kSketchThreads), 0, s, vals, seg_d, row_of, weights,
                     max_blocks, blocks, run_v, run_start, elem_w);
  MGB_LAUNCH_CHECK("k_run_emit");
  hipLaunchKernelGGL(k_run_weights, grid, dim3(kSketchThreads), 0, s, seg_d, stats_d,
                     run_start, weights ? elem_w : nullptr, run_w);
  MGB_LAUNCH_CHECK("k_run_weights");
  hipLaunchKernelGGL(k_sort_keys, grid, dim3(kSketchThreads), 0, s, seg_d, stats_d,
                     run_v, run_w, keys_in, reinterpret_cast<float*>(weight_in));
  MGB_LAUNCH_CHECK("k_sort_keys");
  std::vector<SkStats> stats(nf);
  MGB_CHECK(hipMemcpyAsync(stats.data(), stats_d, nf * sizeof(SkStats), hipMemcpyDeviceToHost, s));
  MGB_CHECK(hipStreamSynchronize(s));

  // Batch plan (src/quantile.cpp:87-122) and tree layout.
  std::vector<SkFeature> features(nf);
  std::vector<uint32_t> seg_begin, seg_end, table0;
  std::vector<std::vector<uint32_t>> tables;  // levels 1, 2, ...
  uint64_t tree_total = 0, scratch_total = 0, fin_total = 0, fin_scratch_total = 0;
  uint32_t node_total = 0;
  for (uint32_t c = 0; c < nf; ++c) {
    const SkStats& st = stats[c];
    SkFeature fe{};
    fe.base = seg[c];
    fe.limit = sketch_budget(max_bin, st.nonmissing);
    fe.budget = sketch_budget(max_bin, st.elements);
    const uint64_t capacity = 2ull * fe.limit;
    fe.batches = (uint32_t)((st.runs + capacity - 1) / capacity);
    fe.levels = bit_width(std::max(1u, fe.batches)) + 1;
    fe.exact = !weights && st.elements <= (1u << 24);
    fe.final_cap = std::max(fe.budget, fe.limit);
    const uint32_t nodes = level_first(fe.batches, 32);
    fe.node_base = node_total;
    fe.tree = tree_total;
    fe.scratch = scratch_total;
    fe.fin = fin_total;
    fe.fin_scratch = fin_scratch_total;
    node_total += nodes;
    tree_total += (uint64_t)nodes * fe.limit;
    scratch_total += (uint64_t)fe.batches * (2ull * fe.limit + 2);
    fin_total += 2 * (2ull * fe.final_cap + 2) + (uint64_t)(fe.levels + 1) * fe.limit;
    fin_scratch_total += 2ull * fe.final_cap + 4;
    for (uint32_t b = 0; b < fe.batches; ++b) {
      const uint64_t begin = (uint64_t)b * capacity;
      seg_begin.push_back((uint32_t)(seg[c] + begin));
      seg_end.push_back((uint32_t)(seg[c] + std::min<uint64_t>(st.runs, begin + capacity)));
      table0.push_back(c);
      table0.push_back(b);
    }
    for (uint32_t level = 1; (fe.batches >> level) != 0; ++level) {
      if (tables.size() < level) tables.emplace_back();
      for (uint32_t k = 0; k < (fe.batches >> level); ++k) {
        tables[level - 1].push_back(c);
        tables[level - 1].push_back(k);
      }
    }
    features[c] = fe;
  }
  size_t temp_bytes = 0;
  if (!seg_begin.empty())
    MGB_CHECK(hipcub::DeviceSegmentedRadixSort::SortPairs(nullptr, temp_bytes, keys_in, keys_out, weight_in, weight_out,
                                                           (int)total, (int)seg_begin.size(), (const uint32_t*)nullptr,
                                                           (const uint32_t*)nullptr, 0, 32, s));
  Arena a2;
  const uint64_t o_features = a2.stage(features), o_table0 = a2.stage(table0);
  const uint64_t o_seg_b = a2.stage(seg_begin), o_seg_e = a2.stage(seg_end);
  std::vector<uint64_t> o_tables(tables.size());
  for (size_t l = 0; l < tables.size(); ++l) o_tables[l] = a2.stage(tables[l]);
  uint32_t max_budget = 1;
  for (const SkFeature& fe : features) max_budget = std::max(max_budget, fe.budget);
  const uint64_t o_tree = a2.reserve(tree_total * sizeof(SkEntry)), o_scratch = a2.reserve(scratch_total * 4);
  const uint64_t o_node_count = a2.reserve((uint64_t)node_total * 4), o_serial = a2.reserve(nf * 4);
  const uint64_t o_fin = a2.reserve(fin_total * sizeof(SkEntry)), o_fin_scratch = a2.reserve(fin_scratch_total * 4);
  const uint64_t o_values = a2.reserve((uint64_t)nf * max_bin * 4), o_temp = a2.reserve(temp_bytes);
  if (a2.commit()) return -1;
  const SkFeature* features_d = a2.at<SkFeature>(o_features);
  SkEntry* tree = a2.at<SkEntry>(o_tree);
  uint32_t* scratch = a2.at<uint32_t>(o_scratch);
  uint32_t* node_count = a2.at<uint32_t>(o_node_count);
  uint32_t* serial = a2.at<uint32_t>(o_serial);
  MGB_CHECK(hipMemsetAsync(serial, 0, nf * 4, s));
  if (!seg_begin.empty()) {
    MGB_CHECK(hipcub::DeviceSegmentedRadixSort::SortPairs(a2.at<void>(o_temp), temp_bytes, keys_in, keys_out, weight_in,
                                                           weight_out, (int)total, (int)seg_begin.size(),
                                                           a2.at<uint32_t>(o_seg_b), a2.at<uint32_t>(o_seg_e), 0, 32,
                                                           s));
    hipLaunchKernelGGL(k_level0, dim3((uint32_t)seg_begin.size()), dim3(kSketchThreads), 0, s,
                       a2.at<uint32_t>(o_table0), features_d, stats_d, keys_out,
                       reinterpret_cast<const float*>(weight_out), work, tree, scratch,
                       node_count);
    MGB_LAUNCH_CHECK("k_level0");
  }
  for (size_t l = 0; l < tables.size(); ++l) {
    hipLaunchKernelGGL(k_level_up, dim3((uint32_t)(tables[l].size() / 2)), dim3(kSketchThreads), 0, s,
                       (uint32_t)(l + 1), a2.at<uint32_t>(o_tables[l]), features_d, work, tree, scratch, node_count,
                       serial);
    MGB_LAUNCH_CHECK("k_level_up");
  }
  // k_finish stages the pruned summary's values and the candidate cuts in LDS
  // for its serial pass when they fit.
  const uint32_t lds_values = (uint64_t)(max_budget + max_bin) * 4 <= kFinishLds ? max_budget : 0;
  const uint32_t lds_bytes = lds_values ? (lds_values + max_bin) * 4 : 0;
  if (lds_bytes &&
      hipFuncSetAttribute((const void*)k_finish, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes) != hipSuccess) {
    set_error("hipFuncSetAttribute(k_finish LDS) failed");
    return -1;
  }
  hipLaunchKernelGGL(k_finish, dim3(nf), dim3(kSketchThreads), lds_bytes, s, features_d, tree, node_count, serial,
                     a2.at<SkEntry>(o_fin), a2.at<uint32_t>(o_fin_scratch), f0, max_bin, a2.at<float>(o_values), lds_values,
                     cuts, counts);
  MGB_LAUNCH_CHECK("k_finish");
  MGB_CHECK(hipStreamSynchronize(s));
  return 0;
}

}  // namespace
}  // namespace mgb

using namespace mgb;

extern "C" {

int mgb_sketch_cuts(const float* X, uint32_t rows, uint32_t cols, const float* weights, uint32_t max_bin,
                    float* cuts, uint32_t* counts) {
  if (max_bin < 2) { set_error("max_bin must be at least 2"); return -1; }
  if (!cols) return 0;
  if (rows >= (1u << 31)) { set_error("sketch: rows must be below 2^31"); return -1; }
  // Feature groups of at most kChunkEntries entries and kMaxGroupFeatures
  // features (the run passes put the feature in gridDim.y).
  const uint32_t group = (uint32_t)std::max<uint64_t>(
      1, std::min<uint64_t>(std::min<uint64_t>(cols, kMaxGroupFeatures), kChunkEntries / std::max(1u, rows)));
  for (uint32_t f0 = 0; f0 < cols; f0 += group) {
    const uint32_t nf = std::min(group, cols - f0);
    StreamBuffer xt;
    if (xt.alloc(std::max<uint64_t>((uint64_t)rows * nf, 1) * 4)) return -1;
    if (rows) {
      const dim3 grid((rows + 31) / 32, (nf + 31) / 32), block(32, 8);
      hipLaunchKernelGGL(k_transpose, grid, block, 0, stream(), X, rows, cols, f0, nf, xt.as<float>());
      MGB_LAUNCH_CHECK("k_transpose");
    }
    std::vector<uint64_t> seg(nf + 1);
    for (uint32_t c = 0; c <= nf; ++c) seg[c] = (uint64_t)c * rows;
    if (sketch_group(xt.as<float>(), seg, nullptr, nf, f0, weights, max_bin, cuts, counts)) return -1;
  }
  return 0;
}

int mgb_sketch_cuts_csc(const float* values, const uint32_t* row_of, const uint64_t* colptr, uint32_t rows,
                        uint32_t cols, const float* weights, uint32_t max_bin, float* cuts, uint32_t* counts) {
  if (max_bin < 2) { set_error("max_bin must be at least 2"); return -1; }
  if (!cols) return 0;
  (void)rows;
  std::vector<uint64_t> colptr_host(cols + 1);
  MGB_CHECK(hipMemcpyAsync(colptr_host.data(), colptr, (cols + 1) * sizeof(uint64_t), hipMemcpyDeviceToHost, stream()));
  MGB_CHECK(hipStreamSynchronize(stream()));
  // Groups of whole columns of at most kChunkEntries entries (a longer column
  // forms a group of its own) and kMaxGroupFeatures columns.
  for (uint32_t f0 = 0; f0 < cols;) {
    uint32_t f1 = f0 + 1;
    while (f1 < cols && f1 - f0 < kMaxGroupFeatures && colptr_host[f1 + 1] - colptr_host[f0] <= kChunkEntries) ++f1;
    std::vector<uint64_t> seg(f1 - f0 + 1);
    for (uint32_t c = 0; c <= f1 - f0; ++c) seg[c] = colptr_host[f0 + c] - colptr_host[f0];
    const uint64_t first = colptr_host[f0];
    if (sketch_group(values + first, seg, row_of + first, f1 - f0, f0, weights, max_bin, cuts, counts)) return -1;
    f0 = f1;
  }
  return 0;
}

}  // extern "C"
