// Weighted quantile sketch on the GPU: the per-feature cut points of the
// reference's hist method (src/quantile.cpp:22-212, kernels/quantile.metal.h,
// XGBoost's WQSummary semantics).  Features are processed in groups of at
// most group_entries() entries (by default as many as a quarter of the free
// device memory holds, so on a 288 GB device one group takes every feature of
// a 10M x 128 matrix and each launch below has all of them in flight); for
// each group:
//
//  1. (dense input) transpose the group's columns (coalesced reads per feature);
//  2. runs of equal values in row order over each feature's non-missing,
//     nonzero-weight entries, in 1024-entry blocks: per-block counts, a
//     per-feature scan over blocks that joins runs crossing block edges, the
//     run starts written at their scanned offsets with the sort keys (an exact
//     feature's every entry, any other's each run), then each run's weight
//     as the sort's payload (its length, or the in-order binary32 sum of its
//     entries' weights);
//  3. the host plans batches of 2*limit runs (limit = sketch budget) from the
//     per-feature counts;
//  4. a segmented radix sort orders every batch by value: an exact feature's
//     (unweighted, below 2^24 entries) as its runs' entries, keys alone --
//     a value's weight, its runs' lengths summed, is its count in the batch;
//     any other's as its runs, stably, carrying each run's weight;
//  5. one workgroup per batch summarizes it (integer weights: its distinct
//     values and weight prefixes) and prunes the summary to limit;
//  6. the serial rule merges batch summaries through a stack of levels like a
//     binary counter (kernels/quantile.metal.h:317-352): while every merge
//     yields more than `limit` entries that is a balanced tree, computed here
//     one level per launch with one workgroup per node; a feature where some
//     merge yields fewer (many equal values) is redone serially by the
//     finishing kernel from its batch summaries;
//  7. one workgroup per feature merges the tree's roots (the stack's final
//     contents), prunes to the budget and selects the cuts.
// Summaries, prunes and merges are data-parallel restatements of the serial
// rules: merges and prunes walk merge-path tiles staged in LDS (a prune is
// the merge of its nondecreasing ranks with the summary's monotone rank
// sums), the error fix-up is a prefix maximum, and sequential binary32 sums
// stay sequential, so every rounding step is the same operation on the same
// operands.
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
constexpr uint32_t kBlockEntries = 1024;                 // entries per block of the run passes
constexpr uint32_t kRunBlocks = 8;                       // consecutive blocks per workgroup in the run passes
constexpr uint64_t kGroupBytesPerEntry = 64;              // a group's temporaries per entry (typical)
constexpr uint64_t kMaxGroupEntries = (uint64_t(1) << 31) - 1;  // 32-bit positions; the sort counts in int
constexpr uint32_t kMaxGroupFeatures = 65535;            // features per group
constexpr uint32_t kMaxBinSketch = 4096;                 // cut candidates per feature, at most

struct SkEntry { float rmin, rmax, wmin, value; };
struct SkStats { uint32_t nonmissing, elements, runs, padding; };
// One workgroup of the run passes: up to kRunBlocks consecutive blocks of one
// feature, starting at block `first` of feature `feature`, whose blocks start
// at `block_base` in the group's block table.  The host lists them feature
// after feature, so a launch has exactly one workgroup per item however
// unequal the features' lengths are.
struct SkRunItem { uint32_t feature, first, block_base, padding; };

// Runs of one 1024-entry block of a feature.  `runs` counts the block's first
// valid entry as a run start; k_run_scan fills the offsets and the last valid
// value before the block.  A group's blocks are stored feature after feature
// (feature c's block b at block_off[c] + b), so the table grows with the
// group's entries, not with its feature count times its longest feature.
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
  uint64_t scratch;     // first word of its batch summaries' scratch (batch b: + b * (2 limit + 2))
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

// Exclusive prefix sums of two values over the workgroup's threads, with
// their totals.
__device__ __forceinline__ void block_exclusive_u32x2(uint32_t a, uint32_t b, uint32_t* shared, uint32_t& ea,
                                                      uint32_t& eb, uint32_t& ta, uint32_t& tb) {
  const uint32_t lane = lane_id(), wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
  const uint32_t ia = wave_inclusive_u32(a), ib = wave_inclusive_u32(b);
  if (lane == kWave - 1) { shared[2 * wave] = ia; shared[2 * wave + 1] = ib; }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t ra = 0, rb = 0;
    for (uint32_t w = 0; w < waves; ++w) {
      const uint32_t xa = shared[2 * w], xb = shared[2 * w + 1];
      shared[2 * w] = ra; shared[2 * w + 1] = rb;
      ra += xa; rb += xb;
    }
    shared[2 * waves] = ra; shared[2 * waves + 1] = rb;
  }
  __syncthreads();
  ea = shared[2 * wave] + ia - a;
  eb = shared[2 * wave + 1] + ib - b;
  ta = shared[2 * waves];
  tb = shared[2 * waves + 1];
  __syncthreads();
}

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

// One entry per thread of block blk of feature c: is it
// present (not NaN) and valid (present with a nonzero weight), and the last
// valid value before it within the block.  Also the block's first and last
// valid values.  `s_*` hold one slot per wave.
struct EntryView {
  float v, w;
  bool present, valid, have_prev;
  float prev;
};

// The thread's entry of block blk (its value, weight and whether it exists);
// the kernels load all their blocks' entries before the first is used.
struct EntryLoad {
  float v, w;
  bool in;
};

__device__ __forceinline__ EntryLoad load_entry(const float* __restrict__ vals, const uint64_t* __restrict__ seg,
                                                const uint32_t* __restrict__ row_of, const float* __restrict__ weights,
                                                uint32_t c, uint32_t blk) {
  const uint64_t base = seg[c];
  const uint32_t count = (uint32_t)(seg[c + 1] - base);
  const uint32_t r = blk * kBlockEntries + threadIdx.x;
  EntryLoad l;
  l.in = r < count;
  l.v = l.in ? vals[base + r] : __uint_as_float(0x7fc00000u);
  l.w = (l.in && weights) ? weights[row_of ? row_of[base + r] : r] : 1.0f;
  return l;
}

__device__ __forceinline__ EntryView view_entry(const EntryLoad& l, uint32_t* s_has, float* s_first, float* s_last,
                                                bool& block_has, float& block_first, float& block_last) {
  const bool in = l.in;
  EntryView e;
  e.v = l.v;
  e.w = l.w;
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
                                                              const float* __restrict__ weights,
                                                              const SkRunItem* __restrict__ items,
                                                              SkBlock* __restrict__ blocks) {
  __shared__ uint32_t s_has[kSketchThreads / kWave], counts[kSketchThreads / kWave][3];
  __shared__ float s_first[kSketchThreads / kWave], s_last[kSketchThreads / kWave];
  const SkRunItem item = items[blockIdx.x];
  const uint32_t c = item.feature;
  const uint32_t nblocks = (uint32_t)((seg[c + 1] - seg[c] + kBlockEntries - 1) / kBlockEntries);
  const uint32_t b0 = item.first;
  EntryLoad loads[kRunBlocks];
#pragma unroll
  for (uint32_t q = 0; q < kRunBlocks; ++q) loads[q] = load_entry(vals, seg, row_of, weights, c, b0 + q);
#pragma unroll
  for (uint32_t q = 0; q < kRunBlocks; ++q) {
    const uint32_t blk = b0 + q;
    if (blk >= nblocks) break;
    bool has = false;
    float first = 0.0f, last = 0.0f;
    const EntryView e = view_entry(loads[q], s_has, s_first, s_last, has, first, last);
    const bool new_run = e.valid && (!e.have_prev || e.v != e.prev);
    // Block totals: each wave's counts from its ballots, summed by thread 0.
    const uint32_t wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
    const uint32_t cv = (uint32_t)__popcll(__ballot(e.valid));
    const uint32_t cp = (uint32_t)__popcll(__ballot(e.present));
    const uint32_t cr = (uint32_t)__popcll(__ballot(new_run));
    if (lane_id() == 0) { counts[wave][0] = cv; counts[wave][1] = cp; counts[wave][2] = cr; }
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t valid = 0, present = 0, runs = 0;
      for (uint32_t w = 0; w < waves; ++w) { valid += counts[w][0]; present += counts[w][1]; runs += counts[w][2]; }
      SkBlock b{};
      b.valid = valid; b.present = present; b.runs = runs; b.has = has ? 1u : 0u;
      b.first = first; b.last = last;
      blocks[(uint64_t)item.block_base + blk] = b;
    }
    __syncthreads();
  }
}

// One workgroup per feature: offsets of its blocks' elements and runs, with a
// block whose first valid value equals the last valid value before it
// continuing that run; the feature's totals.
__global__ __launch_bounds__(kSketchThreads) void k_run_scan(const uint64_t* __restrict__ seg,
                                                             const uint32_t* __restrict__ block_off,
                                                             SkBlock* __restrict__ blocks,
                                                             SkStats* __restrict__ stats) {
  __shared__ uint32_t s_has[kSketchThreads / kWave], scan[kSketchThreads / kWave + 1];
  __shared__ float s_last[kSketchThreads / kWave];
  __shared__ uint32_t carry_has;
  __shared__ float carry_last;
  const uint32_t c = blockIdx.x;
  const uint64_t count = seg[c + 1] - seg[c];
  const uint32_t nblocks = (uint32_t)((count + kBlockEntries - 1) / kBlockEntries);
  SkBlock* fb = blocks + block_off[c];
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

// Whether a feature's summaries are exact integer sums: unweighted, fewer
// than 2^24 valid entries.  Such a feature's batch is sorted as its entries
// (each of weight 1: a value's weight is its run lengths' sum, its count in
// the batch) instead of as runs carrying their lengths.
__host__ __device__ inline bool exact_feature(bool weighted, uint32_t elements) {
  return !weighted && elements <= (1u << 24);
}

// The runs of each block at their scanned offsets: run_start (element index
// within the feature) and the sort keys (order_key) -- of every valid entry at
// its element index for an exact feature, else of each run at its run index
// with, under weights, each valid entry's weight at its element index.
__global__ __launch_bounds__(kSketchThreads) void k_run_emit(const float* __restrict__ vals,
                                                             const uint64_t* __restrict__ seg,
                                                             const uint32_t* __restrict__ row_of,
                                                             const float* __restrict__ weights,
                                                             const SkRunItem* __restrict__ items,
                                                             const SkBlock* __restrict__ blocks,
                                                             const SkStats* __restrict__ stats,
                                                             uint32_t* __restrict__ keys, uint32_t* __restrict__ run_start,
                                                             float* __restrict__ elem_w) {
  __shared__ uint32_t s_has[kSketchThreads / kWave], scan[2 * (kSketchThreads / kWave + 1)];
  __shared__ float s_first[kSketchThreads / kWave], s_last[kSketchThreads / kWave];
  const SkRunItem item = items[blockIdx.x];
  const uint32_t c = item.feature;
  const uint64_t base = seg[c];
  const uint32_t nblocks = (uint32_t)((seg[c + 1] - base + kBlockEntries - 1) / kBlockEntries);
  const bool exact = exact_feature(weights != nullptr, stats[c].elements);
  const uint32_t b0 = item.first;
  EntryLoad loads[kRunBlocks];
#pragma unroll
  for (uint32_t q = 0; q < kRunBlocks; ++q) loads[q] = load_entry(vals, seg, row_of, weights, c, b0 + q);
#pragma unroll
  for (uint32_t q = 0; q < kRunBlocks; ++q) {
    const uint32_t bi = b0 + q;
    if (bi >= nblocks) break;
    const SkBlock blk = blocks[(uint64_t)item.block_base + bi];
    bool has = false;
    float first = 0.0f, last = 0.0f;
    EntryView e = view_entry(loads[q], s_has, s_first, s_last, has, first, last);
    if (!e.have_prev && blk.prev_has) { e.prev = blk.prev; e.have_prev = true; }
    const bool new_run = e.valid && (!e.have_prev || e.v != e.prev);
    uint32_t ev, er, tv, tr;
    block_exclusive_u32x2(e.valid ? 1u : 0u, new_run ? 1u : 0u, scan, ev, er, tv, tr);
    const uint32_t eidx = blk.elem_off + ev, ridx = blk.run_off + er;
    if (new_run) run_start[base + ridx] = eidx;
    if (exact) {
      if (e.valid) keys[base + eidx] = order_key(e.v);
    } else {
      if (new_run) keys[base + ridx] = order_key(e.v);
      if (e.valid && weights) elem_w[base + eidx] = e.w;
    }
  }
}

// Each run's weight, the sort's payload: its length (below 2^24) or, with
// weights, the binary32 sum of its entries' weights in row order
// (kernels/quantile.metal.h:19-140).  Exact features sort their entries and
// need none.
// A feature has at most as many runs as entries, so the run items cover its
// runs too: item (c, b0) takes runs [b0, b0 + kRunBlocks) * kBlockEntries.
__global__ __launch_bounds__(kSketchThreads) void k_run_weights(const uint64_t* __restrict__ seg,
                                                                const SkStats* __restrict__ stats,
                                                                const SkRunItem* __restrict__ items,
                                                                const uint32_t* __restrict__ run_start,
                                                                const float* __restrict__ elem_w,
                                                                float* __restrict__ weight) {
  const SkRunItem item = items[blockIdx.x];
  const uint32_t c = item.feature;
  const uint64_t base = seg[c];
  const SkStats st = stats[c];
  if (exact_feature(elem_w != nullptr, st.elements)) return;
  for (uint32_t q = 0; q < kRunBlocks; ++q) {
    const uint64_t k64 = (uint64_t)(item.first + q) * kBlockEntries + threadIdx.x;
    if (k64 >= st.runs) break;
    const uint32_t k = (uint32_t)k64;
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
    weight[base + k] = w;
  }
}

// Merges and prunes walk their inputs in tiles of a merge path (merge-path
// partitioning, Odeh et al. / Green et al.): a tile's boundaries come from
// one binary search each over global memory, its two input windows are
// staged in LDS with coalesced loads, and every search inside the tile runs
// over LDS.  Each entry is read from global memory once per pass instead of
// once per step of a global binary search.  A workgroup of kThreads threads
// walks tiles of 2 kThreads steps (two per thread) and searches kThreads tile
// boundaries at a time.
constexpr uint32_t kMergeThreads = 256;  // the merge tree's workgroups: four per CU
constexpr uint32_t kWideLevelNodes = 512;  // merge-tree levels with fewer nodes use kSketchThreads

template <uint32_t kThreads>
struct MergeLds {
  static constexpr uint32_t kTile = 2 * kThreads;
  SkEntry a[kTile + 2];   // window of the first input: one entry either side
  SkEntry b[kTile + 2];   // window of the second input
  uint32_t flag[kTile + 1];
  uint32_t bound[kThreads + 1];
  uint32_t scan[2 * (kThreads / kWave + 1)];
};

// Exclusive prefix maximum of v over the workgroup's threads (0 for thread 0);
// *all receives the maximum over every thread.
__device__ __forceinline__ uint32_t block_exclusive_max_u32(uint32_t v, uint32_t* shared, uint32_t* all) {
  const uint32_t lane = lane_id(), wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
  uint32_t inc = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t o = __shfl_up(inc, d, kWave);
    if (lane >= (uint32_t)d) inc = o > inc ? o : inc;
  }
  uint32_t exc = __shfl_up(inc, 1, kWave);
  if (lane == 0) exc = 0;
  if (lane == kWave - 1) shared[wave] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (uint32_t w = 0; w < waves; ++w) {
      const uint32_t t = shared[w];
      shared[w] = run;
      run = t > run ? t : run;
    }
    shared[waves] = run;
  }
  __syncthreads();
  const uint32_t before = shared[wave];
  *all = shared[waves];
  __syncthreads();
  return before > exc ? before : exc;
}

// Number of a[0..len) with value < x (ascending values in LDS).
__device__ __forceinline__ uint32_t count_below(const SkEntry* a, uint32_t len, float x) {
  uint32_t lo = 0, hi = len;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (a[mid].value < x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// Number of a[0..len) with value <= x.
__device__ __forceinline__ uint32_t count_not_above(const SkEntry* a, uint32_t len, float x) {
  uint32_t lo = 0, hi = len;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (a[mid].value <= x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// Merge path of a[0..n) and b[0..m) by value, an a entry before an equal b
// entry: how many a entries are among the first d merged ones.
__device__ __forceinline__ uint32_t merge_split(const SkEntry* a, uint32_t n, const SkEntry* b, uint32_t m,
                                                uint32_t d) {
  uint32_t lo = d > m ? d - m : 0, hi = d < n ? d : n;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (a[mid].value <= b[d - mid - 1].value) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// kernels/quantile.metal.h:192-214 (sketch_prune_serial), data-parallel.
// The serial loop walks i forward while rank_k >= rmax_{i+1} + rmin_{i+1}:
// for k = 1 .. n-1 (n = capacity - 1), with rank_k = 2 (k range / n + begin),
// i_k = 1 + #{j in [2, size) : rmax_j + rmin_j <= rank_k}; the entry taken is
// c_k = i_k or i_k + 1 by the midpoint test, k is live while i_k < size - 1,
// and c_k is appended when it differs from c_{k-1} (c_0 = 0: out[0] = in[0]),
// then in[size-1] unless it was the last one taken.  The sums rmax_j + rmin_j
// are nondecreasing (prefix maxima), so for nondecreasing ranks (range >= 0)
// the counts are one merge path of the ranks against the sums and every c_k
// is nondecreasing; a negative range takes one binary search per k.
__device__ __forceinline__ float prune_rank(uint32_t k, float range, uint32_t n, float begin) {
  return 2.0f * (((float)k * range) / (float)n + begin);
}

__device__ __forceinline__ float prune_key(const SkEntry& e) { return e.rmax + e.rmin; }

// Entry sources for prune: a summary in memory, or a batch summary with
// integer weights kept as its values and the weight prefix at each value
// (rmin = prefix[j], rmax = prefix[j + 1], wmin = their difference; every one
// exact in binary32 below 2^24).
struct EntryArray {
  const SkEntry* p;
  __device__ __forceinline__ SkEntry operator[](uint32_t j) const { return p[j]; }
};

struct ExactSummary {
  const float* value;
  const uint32_t* prefix;
  __device__ __forceinline__ SkEntry operator[](uint32_t j) const {
    const uint32_t lo = prefix[j], hi = prefix[j + 1];
    return SkEntry{(float)lo, (float)hi, (float)(hi - lo), value[j]};
  }
};

template <uint32_t kThreads, typename Src>
__device__ uint32_t prune(const Src& in, uint32_t size, uint32_t capacity, SkEntry* out, MergeLds<kThreads>& L) {
  constexpr uint32_t kMergeTile = MergeLds<kThreads>::kTile, kBoundBatch = kThreads;
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
  if (threadIdx.x == 0) out[0] = in[0];
  if (!(range >= 0.0f)) {
    // Ranks that do not grow with k: the serial walk's i only moves forward,
    // so i_k = 1 + the largest count so far (a prefix maximum over k, one
    // binary search per k); k stops at the first i_k = size - 1.
    uint32_t emitted = 0, prev = 0, cmax = 0;
    for (uint32_t base = 1; base < n; base += blockDim.x) {
      const uint32_t k = base + threadIdx.x;
      const uint32_t chunk = n - base < blockDim.x ? n - base : blockDim.x;
      float rank = 0.0f;
      uint32_t c = 0;
      if (k < n) {
        rank = prune_rank(k, range, n, begin);
        uint32_t lo = 2, hi = size;
        while (lo < hi) {
          const uint32_t mid = (lo + hi) >> 1;
          if (rank >= prune_key(in[mid])) lo = mid + 1;
          else hi = mid;
        }
        c = lo - 2;
      }
      uint32_t all;
      uint32_t m = block_exclusive_max_u32(c, L.scan, &all);
      m = m > cmax ? m : cmax;
      m = c > m ? c : m;
      cmax = all > cmax ? all : cmax;
      const uint32_t i = 1 + m;
      const bool live = k < n && i < size - 1;
      const uint32_t choice = live ? (rank < min_next(in[i]) + max_prev(in[i + 1]) ? i : i + 1) : 0xffffffffu;
      L.flag[threadIdx.x] = choice;
      __syncthreads();
      const uint32_t before = threadIdx.x ? L.flag[threadIdx.x - 1] : prev;
      const bool emit = live && choice != before;
      uint32_t total;
      const uint32_t off = block_exclusive_u32(emit ? 1u : 0u, L.scan, &total);
      if (emit) out[1 + emitted + off] = in[choice];
      emitted += total;
      // Live ks are a prefix of the chunk (i_k grows with k).
      uint32_t lo = 0, hi = chunk;
      while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (L.flag[mid] != 0xffffffffu) lo = mid + 1;
        else hi = mid;
      }
      if (lo) prev = L.flag[lo - 1];
      __syncthreads();
      if (lo < chunk) break;
    }
    uint32_t count = 1 + emitted;
    if (prev != size - 1) {
      if (threadIdx.x == 0) out[count] = in[size - 1];
      ++count;
    }
    __syncthreads();
    return count;
  }
  // Merge path of the ranks (A, x = k - 1) against the sums (B, y = j - 2): a
  // rank goes before a sum when rank < sum, so the B entries before rank x
  // are the count above.
  const uint32_t NA = n - 1, NB = size - 2, total = NA + NB;
  const uint32_t tiles = (total + kMergeTile - 1) / kMergeTile;
  uint32_t emitted = 0, prev = 0;
  bool dead = false;
  for (uint32_t tb = 0; tb < tiles && !dead; tb += kBoundBatch) {
    const uint32_t tn = tiles - tb < kBoundBatch ? tiles - tb : kBoundBatch;
    __syncthreads();
    for (uint32_t t = threadIdx.x; t <= tn; t += blockDim.x) {
      const uint32_t d = (tb + t) * kMergeTile < total ? (tb + t) * kMergeTile : total;
      uint32_t lo = d > NB ? d - NB : 0, hi = d < NA ? d : NA;
      while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (prune_rank(mid + 1, range, n, begin) < prune_key(in[d - mid - 1 + 2])) lo = mid + 1;
        else hi = mid;
      }
      L.bound[t] = lo;
    }
    __syncthreads();
    for (uint32_t t = 0; t < tn; ++t) {
      const uint32_t d0 = (tb + t) * kMergeTile, d1 = d0 + kMergeTile < total ? d0 + kMergeTile : total;
      const uint32_t x0 = L.bound[t], x1 = L.bound[t + 1];
      const uint32_t na = x1 - x0, y0 = d0 - x0, y1 = d1 - x1;
      if (!na) continue;  // sums only: no rank to place
      // Window: in[y0 + 1 .. min(y1 + 2, size - 1)] at w[0 ..]; B entry y is
      // in[y + 2] = w[1 + y - y0].
      SkEntry* w = L.a;
      const uint32_t wlen = (y1 + 2 < size - 1 ? y1 + 2 : size - 1) - y0;
      for (uint32_t e = threadIdx.x; e < wlen; e += blockDim.x) w[e] = in[y0 + 1 + e];
      __syncthreads();
      uint32_t choice[2];
      uint32_t flags = 0;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint32_t e = 2 * threadIdx.x + s;
        choice[s] = 0xffffffffu;
        if (e < na) {
          const float rank = prune_rank(x0 + e + 1, range, n, begin);
          uint32_t lo = 0, hi = y1 - y0;
          while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (prune_key(w[1 + mid]) <= rank) lo = mid + 1;
            else hi = mid;
          }
          const uint32_t i = 1 + y0 + lo;  // in[i] = w[lo], in[i + 1] = w[lo + 1]
          if (i < size - 1) choice[s] = rank < min_next(w[lo]) + max_prev(w[lo + 1]) ? i : i + 1;
        }
        L.flag[e] = choice[s];
      }
      __syncthreads();
      // Live ranks are a prefix (the counts grow with k).
      uint32_t emit[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint32_t e = 2 * threadIdx.x + s;
        const uint32_t before = e ? L.flag[e - 1] : prev;
        emit[s] = e < na && choice[s] != 0xffffffffu && choice[s] != before;
        flags += emit[s];
      }
      uint32_t tot;
      const uint32_t off = block_exclusive_u32(flags, L.scan, &tot);
      uint32_t o = 1 + emitted + off;
#pragma unroll
      for (int s = 0; s < 2; ++s)
        if (emit[s]) out[o++] = w[choice[s] - y0 - 1];
      emitted += tot;
      // The tile's last live choice, and whether a rank was not live.
      const uint32_t last_flag = L.flag[na - 1];
      if (last_flag == 0xffffffffu) {
        dead = true;
        // First non-live rank of the tile: the live prefix ends before it.
        uint32_t lo = 0, hi = na;
        while (lo < hi) {
          const uint32_t mid = (lo + hi) >> 1;
          if (L.flag[mid] != 0xffffffffu) lo = mid + 1;
          else hi = mid;
        }
        if (lo) prev = L.flag[lo - 1];
      } else {
        prev = last_flag;
      }
      __syncthreads();
      if (dead) break;
    }
  }
  uint32_t count = 1 + emitted;
  if (prev != size - 1) {
    if (threadIdx.x == 0) out[count] = in[size - 1];
    ++count;
  }
  __syncthreads();
  return count;
}

// kernels/quantile.metal.h:266-311 (sketch_combine_serial), merge-path form.
// a[0..n) and b[0..m) -> out; out must differ from both.  An a entry whose
// value b also holds absorbs that b entry (sums of rmin, rmax and wmin); any
// other entry adds the neighbouring bounds of the other summary: rmin +=
// min_next of its last entry below, rmax += max_prev of its first entry
// above (or that summary's last rmax).  Then the error fix-up: rmin = prefix
// max of rmin; rmax = prefix max of max(rmax, rmin' + wmin).
template <uint32_t kThreads>
__device__ uint32_t combine(const SkEntry* a, uint32_t n, const SkEntry* b, uint32_t m, SkEntry* out,
                            MergeLds<kThreads>& L) {
  constexpr uint32_t kMergeTile = MergeLds<kThreads>::kTile, kBoundBatch = kThreads;
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
  const float tail_a = a[n - 1].rmax, tail_b = b[m - 1].rmax;
  const uint32_t total = n + m, tiles = (total + kMergeTile - 1) / kMergeTile;
  uint32_t pairs = 0;                 // equal pairs whose a entry is in an earlier tile
  uint32_t run_min = 0, run_max = 0;  // fix-up maxima so far (bit patterns: all values are >= 0)
  for (uint32_t tb = 0; tb < tiles; tb += kBoundBatch) {
    const uint32_t tn = tiles - tb < kBoundBatch ? tiles - tb : kBoundBatch;
    __syncthreads();
    for (uint32_t t = threadIdx.x; t <= tn; t += blockDim.x)
      L.bound[t] = merge_split(a, n, b, m, (tb + t) * kMergeTile < total ? (tb + t) * kMergeTile : total);
    __syncthreads();
    for (uint32_t t = 0; t < tn; ++t) {
      const uint32_t d0 = (tb + t) * kMergeTile, d1 = d0 + kMergeTile < total ? d0 + kMergeTile : total;
      const uint32_t i0 = L.bound[t], i1 = L.bound[t + 1];
      const uint32_t j0 = d0 - i0, j1 = d1 - i1;
      const uint32_t na = i1 - i0, nb = j1 - j0;
      // a[i0-1 .. i1] at L.a[0 .. na+1], b[j0-1 .. j1] at L.b[0 .. nb+1]
      // (the entries that exist).
      for (uint32_t e = threadIdx.x; e < na + 2; e += blockDim.x)
        if (i0 + e >= 1 && i0 + e - 1 < n) L.a[e] = a[i0 + e - 1];
      for (uint32_t e = threadIdx.x; e < nb + 2; e += blockDim.x)
        if (j0 + e >= 1 && j0 + e - 1 < m) L.b[e] = b[j0 + e - 1];
      __syncthreads();
      // The tile's elements: a entries e < na, then b entries; two per thread.
      uint32_t pos[2], lo[2];
      SkEntry r[2];
      bool has[2];
      uint32_t flags = 0;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint32_t e = 2 * threadIdx.x + s;
        has[s] = false;
        lo[s] = 0;
        if (e < na) {
          const SkEntry x = L.a[1 + e];
          // b entries below x: all of the earlier tiles', some of this one's.
          lo[s] = j0 + count_below(L.b + 1, nb, x.value);
          const SkEntry& at = L.b[1 + lo[s] - j0];  // b[lo] when lo < m
          const bool eq = lo[s] < m && at.value == x.value;
          if (eq) {
            r[s].rmin = x.rmin + at.rmin; r[s].rmax = x.rmax + at.rmax; r[s].wmin = x.wmin + at.wmin;
            r[s].value = x.value;
          } else {
            const float prev_b = lo[s] > 0 ? min_next(L.b[lo[s] - j0]) : 0.0f;
            const float add = lo[s] < m ? max_prev(at) : tail_b;
            r[s].rmin = x.rmin + prev_b; r[s].rmax = x.rmax + add; r[s].wmin = x.wmin; r[s].value = x.value;
          }
          has[s] = true;
          flags += eq ? 1u : 0u;
          L.flag[e] = eq ? 1u : 0u;
        }
      }
      // Equal pairs among the tile's a entries before each one.
      uint32_t tile_pairs;
      uint32_t ex = block_exclusive_u32(flags, L.scan, &tile_pairs);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint32_t e = 2 * threadIdx.x + s;
        if (e < na) {
          const uint32_t f = L.flag[e];
          L.flag[e] = ex;
          ex += f;
        }
      }
      if (threadIdx.x == 0) L.flag[na] = tile_pairs;
      __syncthreads();
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint32_t e = 2 * threadIdx.x + s;
        if (e < na) {
          pos[s] = e + (lo[s] - j0) - L.flag[e];
        } else if (e < na + nb) {
          const uint32_t f = e - na;
          const SkEntry y = L.b[1 + f];
          // a entries at or below y: this tile's and the earlier ones.
          const uint32_t ub = i0 + count_not_above(L.a + 1, na, y.value);
          if (ub > 0 && L.a[ub - i0].value == y.value) continue;  // absorbed by a[ub - 1]
          const float prev_a = ub > 0 ? min_next(L.a[ub - i0]) : 0.0f;
          const float add = ub < n ? max_prev(L.a[1 + ub - i0]) : tail_a;
          r[s].rmin = y.rmin + prev_a; r[s].rmax = y.rmax + add; r[s].wmin = y.wmin; r[s].value = y.value;
          pos[s] = f + (ub - i0) - L.flag[ub - i0];
          has[s] = true;
        }
      }
      // An equal pair split by a tile edge: its a entry (the earlier tile's
      // last) writes the combined entry at the later tile's first position,
      // which the later tile's positions leave free.  The outputs are local
      // positions [first, first + count).
      const uint32_t first = (i0 > 0 && j0 < m && L.a[0].value == L.b[1].value) ? 1u : 0u;
      const uint32_t split_next = (i1 > 0 && j1 < m && L.a[na].value == L.b[nb + 1].value) ? 1u : 0u;
      const uint32_t count = (d1 - d0) - L.flag[na] - first + split_next;
      __syncthreads();  // windows read: L.a becomes the tile's output
#pragma unroll
      for (int s = 0; s < 2; ++s)
        if (has[s]) L.a[pos[s]] = r[s];
      __syncthreads();
      // Fix-up over the tile's outputs in order, two per thread.
      SkEntry o[2];
      uint32_t kmin[2], kmax[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint32_t q = 2 * threadIdx.x + s;
        kmin[s] = 0;
        if (q < count) { o[s] = L.a[first + q]; kmin[s] = __float_as_uint(o[s].rmin); }
      }
      uint32_t all_min;
      uint32_t pm = block_exclusive_max_u32(kmin[0] > kmin[1] ? kmin[0] : kmin[1], L.scan, &all_min);
      pm = pm > run_min ? pm : run_min;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint32_t q = 2 * threadIdx.x + s;
        pm = kmin[s] > pm ? kmin[s] : pm;
        kmax[s] = 0;
        if (q < count) {
          o[s].rmin = __uint_as_float(pm);
          const float a2 = o[s].rmin + o[s].wmin;
          kmax[s] = __float_as_uint(o[s].rmax > a2 ? o[s].rmax : a2);
        }
      }
      uint32_t all_max;
      uint32_t px = block_exclusive_max_u32(kmax[0] > kmax[1] ? kmax[0] : kmax[1], L.scan, &all_max);
      px = px > run_max ? px : run_max;
      const uint32_t base = d0 - pairs + first;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint32_t q = 2 * threadIdx.x + s;
        px = kmax[s] > px ? kmax[s] : px;
        if (q < count) {
          o[s].rmax = __uint_as_float(px);
          out[base + q] = o[s];
        }
      }
      run_min = all_min > run_min ? all_min : run_min;
      run_max = all_max > run_max ? all_max : run_max;
      pairs += L.flag[na];
      __syncthreads();
    }
  }
  __syncthreads();
  return total - pairs;
}

// Summary of one sorted batch (kernels/quantile.metal.h:216-240): one entry
// per distinct value, in value order, holding the value's weight w (the
// binary32 sum of its runs' weights in sort order) and the running binary32
// total before (rmin) and after (rmax) it.  keys[0..size) and wts[0..size)
// are the batch's runs' order keys and weights in value order; scratch needs
// size + 1 words.  (Integer weights summing below 2^24 take summarize_exact.)
__device__ uint32_t summarize(const uint32_t* __restrict__ keys, const float* __restrict__ wts, uint32_t size,
                              SkEntry* out, uint32_t* scratch, uint32_t* scan) {
  // Group starts (value changes in sort order) and each group's first position.
  uint32_t carry_s = 0;
  for (uint32_t base = 0; base < size; base += blockDim.x) {
    const uint32_t i = base + threadIdx.x;
    uint32_t start = 0;
    float v = 0.0f;
    if (i < size) {
      v = key_value(keys[i]);
      start = i == 0 || key_value(keys[i - 1]) != v;
    }
    uint32_t ts;
    const uint32_t ps = block_exclusive_u32(start, scan, &ts) + carry_s;
    if (start) {
      scratch[ps] = i;
      out[ps].value = v;
    }
    carry_s += ts;
  }
  if (threadIdx.x == 0) scratch[carry_s] = size;
  __syncthreads();
  const uint32_t n = carry_s;
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

// Summary of one sorted batch with integer weights summing below 2^24
// (kernels/quantile.metal.h:216-240): value[g] is the g-th distinct value
// and prefix[g] the weight of every key before it (prefix[n] the total), so
// the summary entry is (rmin, rmax, wmin) = (prefix[g], prefix[g + 1], their
// difference) -- every binary32 partial sum is exact, so the prefix gives the
// serial sums bit for bit.  wts null: every weight is 1.  Four consecutive
// keys per thread; scan needs 2 (waves + 1) words.  Returns the number of
// distinct values.
__device__ uint32_t summarize_exact(const uint32_t* __restrict__ keys, const float* __restrict__ wts, uint32_t size,
                                    float* __restrict__ value, uint32_t* __restrict__ prefix, uint32_t* scan) {
  constexpr uint32_t kPer = 4;
  const uint32_t chunk = kPer * blockDim.x;
  uint32_t carry_g = 0, carry_w = 0;
  for (uint32_t base = 0; base < size; base += chunk) {
    const uint32_t i0 = base + kPer * threadIdx.x;
    float v[kPer];
    uint32_t w[kPer];
    bool start[kPer];
    float prev = 0.0f;
    if (i0 > 0 && i0 < size) prev = key_value(keys[i0 - 1]);
    uint32_t groups = 0, weight = 0;
#pragma unroll
    for (uint32_t u = 0; u < kPer; ++u) {
      const uint32_t i = i0 + u;
      const bool in = i < size;
      v[u] = in ? key_value(keys[i]) : 0.0f;
      w[u] = in ? (wts ? (uint32_t)wts[i] : 1u) : 0u;
      start[u] = in && (i == 0 || v[u] != (u ? v[u - 1] : prev));
      groups += start[u] ? 1u : 0u;
      weight += w[u];
    }
    uint32_t eg, ew, tg, tw;
    block_exclusive_u32x2(groups, weight, scan, eg, ew, tg, tw);
    uint32_t g = carry_g + eg, pw = carry_w + ew;
#pragma unroll
    for (uint32_t u = 0; u < kPer; ++u) {
      if (start[u]) {
        value[g] = v[u];
        prefix[g] = pw;
        ++g;
      }
      pw += w[u];
    }
    carry_g += tg;
    carry_w += tw;
  }
  if (threadIdx.x == 0) prefix[carry_g] = carry_w;
  __syncthreads();
  return carry_g;
}

// Key range of each batch (table: feature, batch) in the sort's arrays: its
// runs [b 2 limit, min((b + 1) 2 limit, runs)) for a feature sorted as runs;
// the entries of those runs, from the first one's start to the next batch's
// first start (or the last entry), for an exact feature.
__global__ void k_batch_keys(const uint32_t* __restrict__ table, uint32_t count,
                             const SkFeature* __restrict__ features, const SkStats* __restrict__ stats,
                             const uint32_t* __restrict__ run_start, uint32_t* __restrict__ key_begin,
                             uint32_t* __restrict__ key_end) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  const uint32_t c = table[2 * i], b = table[2 * i + 1];
  const SkFeature fe = features[c];
  const SkStats st = stats[c];
  const uint32_t base = (uint32_t)fe.base;
  const uint64_t cap = 2ull * fe.limit;
  const uint32_t rb = (uint32_t)((uint64_t)b * cap);
  const uint32_t re = (uint32_t)std::min<uint64_t>((uint64_t)rb + cap, st.runs);
  if (fe.exact) {
    key_begin[i] = base + run_start[base + rb];
    key_end[i] = base + (re == st.runs ? st.elements : run_start[base + re]);
  } else {
    key_begin[i] = base + rb;
    key_end[i] = base + re;
  }
}

// ---------------------------------------------------------------------------
// Tie order.  Stock XGBoost sorts each batch of (value, weight) entries with
// std::sort on the value alone and merges equal values in the order it
// leaves them (upstream WQSummary::Queue::MakeSummary): the first one's
// value represents the group (the sign of a zero) and the weights are added
// in that order.  The radix sort orders by key, stably, which gives the same
// summary unless a group of equal values holds both zeros or (run-weighted
// batches) runs of different weights; such a batch is re-sorted from its
// runs in row order with libstdc++'s std::sort steps (x86-64 builds; the
// reference restates libc++'s for its macOS builds,
// kernels/sketch_sort.metal.h), by one thread, in LDS when it fits.
// ---------------------------------------------------------------------------
// The value of an order key, on the host too (the tie sort below runs there
// for its test hook, mgb_tie_sort_order).
__host__ __device__ inline float tie_value(uint32_t key) {
  const uint32_t bits = key ^ ((key & 0x80000000u) ? 0x80000000u : 0xffffffffu);
  float v;
  memcpy(&v, &bits, 4);
  return v;
}

struct TieRuns {  // element i: (key[i], weight[i]); compared by the key's value
  uint32_t* key;
  uint32_t* weight;
  __host__ __device__ bool less(uint32_t a, uint32_t b) const { return tie_value(key[a]) < tie_value(key[b]); }
  __host__ __device__ bool less_value(uint32_t a, uint32_t k) const { return tie_value(key[a]) < tie_value(k); }
  __host__ __device__ bool value_less(uint32_t k, uint32_t b) const { return tie_value(k) < tie_value(key[b]); }
  __host__ __device__ void swap(uint32_t a, uint32_t b) {
    const uint32_t k = key[a], w = weight[a];
    key[a] = key[b]; weight[a] = weight[b];
    key[b] = k; weight[b] = w;
  }
  __host__ __device__ void move(uint32_t to, uint32_t from) { key[to] = key[from]; weight[to] = weight[from]; }
};

// __adjust_heap with __push_heap over [first, first + len) (value = (vk, vw)).
__host__ __device__ void tie_adjust_heap(TieRuns& r, uint32_t first, int64_t hole, int64_t len, uint32_t vk, uint32_t vw) {
  const int64_t top = hole;
  int64_t child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (r.less(first + (uint32_t)child, first + (uint32_t)child - 1)) --child;
    r.move(first + (uint32_t)hole, first + (uint32_t)child);
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    r.move(first + (uint32_t)hole, first + (uint32_t)child - 1);
    hole = child - 1;
  }
  int64_t parent = (hole - 1) / 2;
  while (hole > top && r.less_value(first + (uint32_t)parent, vk)) {
    r.move(first + (uint32_t)hole, first + (uint32_t)parent);
    hole = parent;
    parent = (hole - 1) / 2;
  }
  r.key[first + hole] = vk;
  r.weight[first + hole] = vw;
}

// std::sort (libstdc++, GCC 11 bits/stl_algo.h) of r[0, n): introsort with
// depth 2 floor(log2 n) -- the median of the second, middle and last
// elements moved to the front, an unguarded partition, heap sort when the
// depth runs out -- then insertion sort (the first 16 guarded, the rest
// unguarded).  The loop keeps the pending right parts on a stack instead of
// recursing; sorting disjoint ranges in another order moves the same
// elements the same way.  The "unguarded" scans also stop at their range's
// ends: with the median of three in front they never reach them, so the
// order is unchanged, and no index leaves the range whatever the input.
__host__ __device__ void tie_std_sort(TieRuns& r, uint32_t n) {
  if (n < 2) return;
  int lg = 0;
  while (((uint64_t)2 << lg) <= n) ++lg;
  uint32_t stack_first[72], stack_last[72];
  int stack_depth[72];
  int top = 0;
  stack_first[0] = 0; stack_last[0] = n; stack_depth[0] = 2 * lg;
  top = 1;
  while (top > 0) {
    --top;
    uint32_t first = stack_first[top], last = stack_last[top];
    int depth = stack_depth[top];
    while (last - first > 16) {
      if (depth == 0) {  // __partial_sort(first, last, last): make_heap, sort_heap
        const int64_t len = last - first;
        for (int64_t parent = (len - 2) / 2;; --parent) {
          tie_adjust_heap(r, first, parent, len, r.key[first + parent], r.weight[first + parent]);
          if (parent == 0) break;
        }
        for (uint32_t end = last; end - first > 1;) {
          --end;
          const uint32_t vk = r.key[end], vw = r.weight[end];
          r.move(end, first);
          tie_adjust_heap(r, first, 0, (int64_t)(end - first), vk, vw);
        }
        break;
      }
      --depth;
      const uint32_t mid = first + (last - first) / 2, a = first + 1, b = mid, c = last - 1;
      if (r.less(a, b)) {
        if (r.less(b, c)) r.swap(first, b);
        else if (r.less(a, c)) r.swap(first, c);
        else r.swap(first, a);
      } else if (r.less(a, c)) {
        r.swap(first, a);
      } else if (r.less(b, c)) {
        r.swap(first, c);
      } else {
        r.swap(first, b);
      }
      uint32_t lo = first + 1, hi = last;
      for (;;) {
        while (lo + 1 < last && r.less(lo, first)) ++lo;
        --hi;
        while (hi > first && r.less(first, hi)) --hi;
        if (!(lo < hi)) break;
        r.swap(lo, hi);
        ++lo;
      }
      // Right part [lo, last) is sorted later (the recursion's callee), the
      // left part [first, lo) now.
      stack_first[top] = lo; stack_last[top] = last; stack_depth[top] = depth;
      ++top;
      last = lo;
    }
  }
  // __final_insertion_sort
  const uint32_t guarded = n > 16 ? 16 : n;
  for (uint32_t i = 1; i < guarded; ++i) {
    const uint32_t vk = r.key[i], vw = r.weight[i];
    if (r.value_less(vk, 0)) {
      for (uint32_t j = i; j > 0; --j) r.move(j, j - 1);
      r.key[0] = vk; r.weight[0] = vw;
    } else {
      uint32_t j = i;
      while (j > 0 && r.value_less(vk, j - 1)) { r.move(j, j - 1); --j; }
      r.key[j] = vk; r.weight[j] = vw;
    }
  }
  for (uint32_t i = guarded; i < n; ++i) {
    const uint32_t vk = r.key[i], vw = r.weight[i];
    uint32_t j = i;
    while (j > 0 && r.value_less(vk, j - 1)) { r.move(j, j - 1); --j; }
    r.key[j] = vk; r.weight[j] = vw;
  }
}

constexpr uint32_t kTieThreads = 256;
constexpr uint32_t kTieLdsRuns = 8000;  // runs sorted in LDS (62.5 KiB); longer batches sort in global memory

// One workgroup per batch (the level-0 table): finds whether the batch has a
// tie the merge order decides and, if so, writes its sorted keys in
// std::sort's order (run-weighted batches: keys and weights; exact batches,
// whose weights are all 1 and sum exactly: the zero group's first key).
// keys_in/weight_in hold each feature's runs (exact: entries) in row order
// before the sort; elem_w and weight_in are free for an exact feature's runs.
__global__ __launch_bounds__(kTieThreads) void k_tie_order(const uint32_t* __restrict__ table,
                                                            const SkFeature* __restrict__ features,
                                                            const SkStats* __restrict__ stats,
                                                            const uint32_t* __restrict__ key_begin,
                                                            const uint32_t* __restrict__ key_end,
                                                            const uint32_t* __restrict__ run_start,
                                                            const uint32_t* __restrict__ keys_in,
                                                            uint32_t* __restrict__ weight_in, uint32_t* __restrict__ elem_w,
                                                            uint32_t* __restrict__ keys, uint32_t* __restrict__ wts) {
  __shared__ uint32_t s_flag;
  __shared__ uint32_t lds_key[kTieLdsRuns], lds_w[kTieLdsRuns];
  const uint32_t c = table[2 * blockIdx.x], b = table[2 * blockIdx.x + 1];
  const SkFeature fe = features[c];
  const SkStats st = stats[c];
  const uint32_t kb = key_begin[blockIdx.x], size = key_end[blockIdx.x] - kb;
  if (threadIdx.x == 0) s_flag = 0;
  __syncthreads();
  for (uint32_t i = 1 + threadIdx.x; i < size; i += blockDim.x) {
    const uint32_t ka = keys[kb + i - 1], kz = keys[kb + i];
    if (key_value(ka) != key_value(kz)) continue;
    if (ka != kz || (!fe.exact && wts[kb + i - 1] != wts[kb + i])) s_flag = 1;
  }
  __syncthreads();
  if (!s_flag || threadIdx.x != 0) return;
  // The batch's runs in row order.
  const uint64_t rb = (uint64_t)b * 2 * fe.limit;
  const uint32_t n = (uint32_t)std::min<uint64_t>(2ull * fe.limit, st.runs - rb);
  const uint32_t base = (uint32_t)fe.base;
  TieRuns r;
  if (n <= kTieLdsRuns) {
    r.key = lds_key;
    r.weight = lds_w;
  } else if (fe.exact) {
    r.key = elem_w + base + rb;
    r.weight = weight_in + base + rb;
  } else {
    r.key = keys + kb;  // this batch's sorted output, overwritten in place
    r.weight = wts + kb;
  }
  for (uint32_t j = 0; j < n; ++j) {
    const uint32_t run = (uint32_t)rb + j;
    if (fe.exact) {
      const uint32_t s0 = run_start[base + run];
      const uint32_t s1 = run + 1 < st.runs ? run_start[base + run + 1] : st.elements;
      r.key[j] = keys_in[base + s0];
      r.weight[j] = s1 - s0;  // a run length (the weights of exact features are never summed as floats)
    } else {
      r.key[j] = keys_in[base + run];
      r.weight[j] = weight_in[base + run];
    }
  }
  tie_std_sort(r, n);
  if (!fe.exact) {
    if (r.key != keys + kb)
      for (uint32_t j = 0; j < n; ++j) { keys[kb + j] = r.key[j]; wts[kb + j] = r.weight[j]; }
    return;
  }
  // Exact batch: the zero group keeps its counts; its first key becomes the
  // zero std::sort puts first.
  uint32_t first_zero = 0xffffffffu;
  for (uint32_t j = 0; j < n; ++j)
    if (key_value(r.key[j]) == 0.0f) { first_zero = r.key[j]; break; }
  if (first_zero == 0xffffffffu) return;
  uint32_t z0 = 0xffffffffu, z1 = 0;
  for (uint32_t i = 0; i < size; ++i)
    if (key_value(keys[kb + i]) == 0.0f) {
      if (z0 == 0xffffffffu) z0 = i;
      if (keys[kb + i] == first_zero) z1 = i;
    }
  if (z0 != 0xffffffffu && keys[kb + z0] != first_zero) {
    const uint32_t t = keys[kb + z0];
    keys[kb + z0] = keys[kb + z1];
    keys[kb + z1] = t;
  }
}

// Level 0 of every feature's tree: one workgroup per batch summarizes the
// batch's sorted runs into the feature's work area and prunes the summary to
// `limit` entries (the serial rule's first step for each batch,
// kernels/quantile.metal.h:317-352).
__global__ __launch_bounds__(kMergeThreads) void k_level0(const uint32_t* __restrict__ table,
                                                           const SkFeature* __restrict__ features,
                                                           const SkStats* __restrict__ stats,
                                                           const uint32_t* __restrict__ key_begin,
                                                           const uint32_t* __restrict__ key_end,
                                                           const uint32_t* __restrict__ keys,
                                                           const float* __restrict__ wts, SkEntry* __restrict__ work,
                                                           SkEntry* __restrict__ tree, uint32_t* __restrict__ scratch,
                                                           uint32_t* __restrict__ node_count) {
  __shared__ MergeLds<kMergeThreads> L;
  const uint32_t c = table[2 * blockIdx.x], b = table[2 * blockIdx.x + 1];
  const SkFeature fe = features[c];
  const uint32_t kb = key_begin[blockIdx.x], size = key_end[blockIdx.x] - kb;
  // The batch's summary takes the work area of its runs (16 bytes each); it
  // has at most one entry per run.
  const uint64_t rb = (uint64_t)b * 2 * fe.limit;
  const uint32_t runs = (uint32_t)std::min<uint64_t>(2ull * fe.limit, stats[c].runs - rb);
  SkEntry* summary = work + fe.base + rb;
  SkEntry* pruned = tree + fe.tree + (uint64_t)b * fe.limit;
  uint32_t m;
  if (fe.exact) {
    // Sorted entries of weight 1: values and weight prefixes (at most
    // 2 runs + 1 words) instead of 16-byte entries.
    float* value = reinterpret_cast<float*>(summary);
    uint32_t* prefix = reinterpret_cast<uint32_t*>(summary) + runs;
    const uint32_t n = summarize_exact(keys + kb, nullptr, size, value, prefix, L.scan);
    m = prune(ExactSummary{value, prefix}, n, fe.limit, pruned, L);
  } else {
    const uint32_t n = summarize(keys + kb, wts + kb, size, summary,
                                 scratch + fe.scratch + (uint64_t)b * (2 * fe.limit + 2), L.scan);
    m = prune(EntryArray{summary}, n, fe.limit, pruned, L);
  }
  if (threadIdx.x == 0) node_count[fe.node_base + b] = m;
}

// Level `level` >= 1: node k merges nodes 2k + 1 and 2k of the level below
// (the serial rule's merge of a new summary into an occupied level) and
// prunes the merge to `limit`.  A merge of at most `limit` entries stays at
// its level in the serial rule instead of moving up, so the tree no longer
// matches it: the feature is marked for the serial rebuild.
template <uint32_t kThreads>
__global__ __launch_bounds__(kThreads) void k_level_up(uint32_t level, const uint32_t* __restrict__ table,
                                                             const SkFeature* __restrict__ features,
                                                             SkEntry* __restrict__ work, SkEntry* __restrict__ tree,
                                                             uint32_t* __restrict__ node_count,
                                                             uint32_t* __restrict__ serial) {
  __shared__ MergeLds<kThreads> L;
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
                             nb, merged, L);
  if (n <= fe.limit) {
    if (threadIdx.x == 0) atomicOr(&serial[c], 1u);
    return;
  }
  const uint32_t m = prune(EntryArray{merged}, n, fe.limit, tree + fe.tree + (uint64_t)(here + k) * fe.limit, L);
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
                                                           SkEntry* __restrict__ fin,
                                                           uint32_t f0, uint32_t max_bin, uint32_t* __restrict__ picks,
                                                           float* __restrict__ cuts,
                                                           uint32_t* __restrict__ counts) {
  __shared__ uint32_t level_count[64];
  __shared__ uint32_t s_scan[kSketchThreads / kWave + 1];
  __shared__ uint32_t s_stop;
  extern __shared__ __align__(16) uint8_t s_dynamic[];
  MergeLds<kSketchThreads>& L = *reinterpret_cast<MergeLds<kSketchThreads>*>(s_dynamic);
  const uint32_t c = blockIdx.x;
  const SkFeature fe = features[c];
  const uint32_t limit = fe.limit, batches = fe.batches;
  const uint64_t buf = 2ull * fe.final_cap + 2;
  SkEntry* cur = fin + fe.fin;
  SkEntry* oth = cur + buf;
  SkEntry* lvl = oth + buf;  // the serial stack: (levels + 1) x limit
  uint32_t n = 0;
  if (batches && !serial[c]) {
    for (uint32_t level = 0; level < fe.levels && level < 32; ++level) {
      if ((batches >> level) & 1u) {
        const uint32_t node = level_first(batches, level) + (batches >> level) - 1;
        n = combine(cur, n, tree + fe.tree + (uint64_t)node * limit, node_count[fe.node_base + node], oth, L);
        SkEntry* t = cur; cur = oth; oth = t;
      }
      n = prune(EntryArray{cur}, n, fe.final_cap, oth, L);
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
          n = combine(cur, n, lvl + (uint64_t)level * limit, m, oth, L);
          SkEntry* t = cur; cur = oth; oth = t;
        }
        __syncthreads();
        if (threadIdx.x == 0) level_count[level] = 0;
        __syncthreads();
        if (n <= limit) break;
        ++level;
        n = prune(EntryArray{cur}, n, limit, oth, L);
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
        n = combine(cur, n, lvl + (uint64_t)level * limit, m, oth, L);
        SkEntry* t = cur; cur = oth; oth = t;
      }
      n = prune(EntryArray{cur}, n, fe.final_cap, oth, L);
      SkEntry* t = cur; cur = oth; oth = t;
    }
  }
  n = prune(EntryArray{cur}, n, fe.budget, oth, L);
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
  // Rank queries in parallel: query i (1 <= i < max_bin) picks entry c_i.
  // The serial pass that follows (kernels/quantile.metal.h:371-396) emits,
  // while it can, e_i = c_i's value if it exceeds the last one emitted, else
  // the next entry above it.  Entry values strictly increase, so in indexes
  // k_i = max(c_i, k_{i-1} + 1) with k_0 = 0, i.e. k_i = i + max(0, max over
  // j <= i of (c_j - j)) -- a prefix maximum -- and the pass stops after the
  // first k_i = size - 1 (no entry is left above it).
  uint32_t* pick = picks + (uint64_t)c * max_bin;
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
    pick[i] = cursor + ((isnan(boundary) || rank >= (double)boundary) ? 1u : 0u);
  }
  if (threadIdx.x == 0) s_stop = max_bin;
  __syncthreads();
  // Thread t takes queries 1 + kCutsPer t .. kCutsPer (t + 1), in order; the
  // offset keeps c_j - j + kMaxBinSketch >= 0 for the unsigned maximum.
  constexpr uint32_t kCutsPer = (kMaxBinSketch + kSketchThreads - 1) / kSketchThreads;
  uint32_t k[kCutsPer];
  uint32_t local = 0;
#pragma unroll
  for (uint32_t u = 0; u < kCutsPer; ++u) {
    const uint32_t i = 1 + kCutsPer * threadIdx.x + u;
    if (i < max_bin) {
      const uint32_t d = pick[i] + kMaxBinSketch - i;
      local = d > local ? d : local;
    }
  }
  uint32_t all;
  uint32_t run = block_exclusive_max_u32(local, s_scan, &all);
#pragma unroll
  for (uint32_t u = 0; u < kCutsPer; ++u) {
    const uint32_t i = 1 + kCutsPer * threadIdx.x + u;
    k[u] = 0;
    if (i < max_bin) {
      const uint32_t d = pick[i] + kMaxBinSketch - i;
      run = d > run ? d : run;
      k[u] = i + (run > kMaxBinSketch ? run - kMaxBinSketch : 0u);
      if (k[u] == size - 1) atomicMin(&s_stop, i);
    }
  }
  __syncthreads();
  const uint32_t emitted = s_stop < max_bin ? s_stop : max_bin - 1;
#pragma unroll
  for (uint32_t u = 0; u < kCutsPer; ++u) {
    const uint32_t i = 1 + kCutsPer * threadIdx.x + u;
    if (i <= emitted) out[i - 1] = cur[k[u]].value;
  }
  if (threadIdx.x == 0) {
    const float tail = cur[size - 1].value;
    out[emitted] = tail + (fabsf(tail) + 1e-5f);
    counts[f] = emitted + 1;
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

uint64_t g_group_entries = 0;  // mgb_sketch_group_entries; 0: from the free device memory

// Entries per group of features: the set value, else what a quarter of the
// free device memory holds at kGroupBytesPerEntry.
uint64_t group_entries() {
  if (g_group_entries) return std::min(g_group_entries, kMaxGroupEntries);
  size_t free_bytes = 0, total_bytes = 0;
  if (hipMemGetInfo(&free_bytes, &total_bytes) != hipSuccess) {
    (void)hipGetLastError();
    return uint64_t(1) << 27;
  }
  return std::clamp<uint64_t>(free_bytes / 4 / kGroupBytesPerEntry, uint64_t(1) << 20, kMaxGroupEntries);
}

// Device memory of one sketch pass from the library's allocator, in order on
// the library stream: a free is queued behind the kernels that use the
// buffer instead of waiting for the device, and the allocator keeps it for
// the next pass.
struct StreamBuffer {
  void* p = nullptr;
  StreamBuffer() = default;
  StreamBuffer(const StreamBuffer&) = delete;
  StreamBuffer& operator=(const StreamBuffer&) = delete;
  ~StreamBuffer() {
    if (p) (void)mgb_free(p);
  }
  int alloc(size_t bytes) { return mgb_malloc(&p, bytes ? bytes : 16); }
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
// load_entry for the meaning of row_of and weights.
int sketch_group(const float* vals, const std::vector<uint64_t>& seg, const uint32_t* row_of, uint32_t nf, uint32_t f0,
                 const float* weights, uint32_t max_bin, float* cuts, uint32_t* counts) {
  hipStream_t s = stream();
  const uint64_t total = seg[nf];
  // Positions are 32-bit and the segmented sort counts in int.
  if (total >= (1ull << 31)) { set_error("sketch: more than 2^31 - 1 entries in one group"); return -1; }
  // The run passes' work list: each feature's blocks of kBlockEntries
  // entries, stored feature after feature (block_off), and its workgroups of
  // up to kRunBlocks consecutive blocks (items).
  std::vector<uint32_t> block_off(nf + 1, 0);
  std::vector<SkRunItem> items;
  for (uint32_t c = 0; c < nf; ++c) {
    const uint32_t nblocks = (uint32_t)((seg[c + 1] - seg[c] + kBlockEntries - 1) / kBlockEntries);
    block_off[c + 1] = block_off[c] + nblocks;
    for (uint32_t b = 0; b < nblocks; b += kRunBlocks) items.push_back(SkRunItem{c, b, block_off[c], 0u});
  }
  if (items.empty()) items.push_back(SkRunItem{0u, 0u, 0u, 0u});  // no entries: one idle workgroup
  const uint64_t E = total ? total : 1;
  Arena a1;
  const uint64_t o_seg = a1.stage(seg);
  const uint64_t o_block_off = a1.stage(block_off);
  const uint64_t o_items = a1.stage(items);
  const uint64_t o_blocks = a1.reserve((uint64_t)std::max<uint32_t>(block_off[nf], 1) * sizeof(SkBlock));
  const uint64_t o_stats = a1.reserve(nf * sizeof(SkStats));
  const uint64_t o_region = a1.reserve(E * 16);
  const uint64_t o_keys_out = a1.reserve(E * 4), o_weight_out = a1.reserve(E * 4);
  if (a1.commit()) return -1;
  const uint64_t* seg_d = a1.at<uint64_t>(o_seg);
  const uint32_t* block_off_d = a1.at<uint32_t>(o_block_off);
  const SkRunItem* items_d = a1.at<SkRunItem>(o_items);
  SkBlock* blocks = a1.at<SkBlock>(o_blocks);
  SkStats* stats_d = a1.at<SkStats>(o_stats);
  uint32_t* keys_out = a1.at<uint32_t>(o_keys_out);
  uint32_t* weight_out = a1.at<uint32_t>(o_weight_out);
  // One 16-byte-per-entry region: run starts, the sort's keys and payloads
  // and entry weights until the sort, then the summaries' and merges' work
  // area.
  uint32_t* run_start = a1.at<uint32_t>(o_region);
  uint32_t* keys_in = run_start + E;
  uint32_t* weight_in = keys_in + E;
  float* elem_w = reinterpret_cast<float*>(weight_in + E);
  SkEntry* work = a1.at<SkEntry>(o_region);
  const dim3 run_grid((uint32_t)items.size());
  hipLaunchKernelGGL(k_run_count, run_grid, dim3(kSketchThreads), 0, s, vals, seg_d, row_of, weights,
                     items_d, blocks);
  MGB_LAUNCH_CHECK("k_run_count");
  hipLaunchKernelGGL(k_run_scan, dim3(nf), dim3(kSketchThreads), 0, s, seg_d, block_off_d,
                     blocks, stats_d);
  MGB_LAUNCH_CHECK("k_run_scan");
  hipLaunchKernelGGL(k_run_emit, run_grid, dim3(kSketchThreads), 0, s, vals, seg_d, row_of, weights,
                     items_d, blocks, stats_d, keys_in, run_start, elem_w);
  MGB_LAUNCH_CHECK("k_run_emit");
  hipLaunchKernelGGL(k_run_weights, run_grid, dim3(kSketchThreads), 0, s, seg_d, stats_d, items_d,
                     run_start, weights ? elem_w : nullptr, reinterpret_cast<float*>(weight_in));
  MGB_LAUNCH_CHECK("k_run_weights");
  std::vector<SkStats> stats(nf);
  MGB_CHECK(hipMemcpyAsync(stats.data(), stats_d, nf * sizeof(SkStats), hipMemcpyDeviceToHost, s));
  MGB_CHECK(hipStreamSynchronize(s));

  // Batch plan (src/quantile.cpp:87-122) and tree layout.  table0 lists the
  // exact features' batches first: their entries are sorted as keys alone.
  std::vector<SkFeature> features(nf);
  std::vector<uint32_t> table0, table0_runs;
  std::vector<std::vector<uint32_t>> tables;  // levels 1, 2, ...
  uint64_t tree_total = 0, scratch_total = 0, fin_total = 0;
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
    fe.exact = exact_feature(weights != nullptr, st.elements) ? 1u : 0u;
    fe.final_cap = std::max(fe.budget, fe.limit);
    const uint32_t nodes = level_first(fe.batches, 32);
    fe.node_base = node_total;
    fe.tree = tree_total;
    fe.scratch = scratch_total;
    fe.fin = fin_total;
    node_total += nodes;
    tree_total += (uint64_t)nodes * fe.limit;
    scratch_total += (uint64_t)fe.batches * (2ull * fe.limit + 2);
    fin_total += 2 * (2ull * fe.final_cap + 2) + (uint64_t)(fe.levels + 1) * fe.limit;
    std::vector<uint32_t>& t0 = fe.exact ? table0 : table0_runs;
    for (uint32_t b = 0; b < fe.batches; ++b) {
      t0.push_back(c);
      t0.push_back(b);
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
  const uint32_t exact_batches = (uint32_t)(table0.size() / 2);
  table0.insert(table0.end(), table0_runs.begin(), table0_runs.end());
  const uint32_t batches = (uint32_t)(table0.size() / 2), run_batches = batches - exact_batches;
  size_t temp_keys = 0, temp_pairs = 0;
  if (exact_batches)
    MGB_CHECK(hipcub::DeviceSegmentedRadixSort::SortKeys(nullptr, temp_keys, keys_in, keys_out, (int)total,
                                                          (int)exact_batches, (const uint32_t*)nullptr,
                                                          (const uint32_t*)nullptr, 0, 32, s));
  if (run_batches)
    MGB_CHECK(hipcub::DeviceSegmentedRadixSort::SortPairs(nullptr, temp_pairs, keys_in, keys_out, weight_in, weight_out,
                                                           (int)total, (int)run_batches, (const uint32_t*)nullptr,
                                                           (const uint32_t*)nullptr, 0, 32, s));
  size_t temp_bytes = std::max(temp_keys, temp_pairs);
  Arena a2;
  const uint64_t o_features = a2.stage(features), o_table0 = a2.stage(table0);
  const uint64_t o_key_b = a2.reserve((uint64_t)batches * 4), o_key_e = a2.reserve((uint64_t)batches * 4);
  std::vector<uint64_t> o_tables(tables.size());
  for (size_t l = 0; l < tables.size(); ++l) o_tables[l] = a2.stage(tables[l]);
  const uint64_t o_tree = a2.reserve(tree_total * sizeof(SkEntry)), o_scratch = a2.reserve(scratch_total * 4);
  const uint64_t o_node_count = a2.reserve((uint64_t)node_total * 4), o_serial = a2.reserve(nf * 4);
  const uint64_t o_fin = a2.reserve(fin_total * sizeof(SkEntry));
  const uint64_t o_values = a2.reserve((uint64_t)nf * max_bin * 4), o_temp = a2.reserve(temp_bytes);
  if (a2.commit()) return -1;
  const SkFeature* features_d = a2.at<SkFeature>(o_features);
  SkEntry* tree = a2.at<SkEntry>(o_tree);
  uint32_t* scratch = a2.at<uint32_t>(o_scratch);
  uint32_t* node_count = a2.at<uint32_t>(o_node_count);
  uint32_t* serial = a2.at<uint32_t>(o_serial);
  MGB_CHECK(hipMemsetAsync(serial, 0, nf * 4, s));
  if (batches) {
    uint32_t* key_b = a2.at<uint32_t>(o_key_b);
    uint32_t* key_e = a2.at<uint32_t>(o_key_e);
    hipLaunchKernelGGL(k_batch_keys, dim3((batches + 255) / 256), dim3(256), 0, s, a2.at<uint32_t>(o_table0), batches,
                       features_d, stats_d, run_start, key_b, key_e);
    MGB_LAUNCH_CHECK("k_batch_keys");
    if (exact_batches)
      MGB_CHECK(hipcub::DeviceSegmentedRadixSort::SortKeys(a2.at<void>(o_temp), temp_bytes, keys_in, keys_out,
                                                            (int)total, (int)exact_batches, key_b, key_e, 0, 32, s));
    if (run_batches)
      MGB_CHECK(hipcub::DeviceSegmentedRadixSort::SortPairs(a2.at<void>(o_temp), temp_bytes, keys_in, keys_out,
                                                             weight_in, weight_out, (int)total, (int)run_batches,
                                                             key_b + exact_batches, key_e + exact_batches, 0, 32, s));
    hipLaunchKernelGGL(k_tie_order, dim3(batches), dim3(kTieThreads), 0, s, a2.at<uint32_t>(o_table0), features_d,
                       stats_d, key_b, key_e, run_start, keys_in, weight_in, reinterpret_cast<uint32_t*>(elem_w),
                       keys_out, weight_out);
    MGB_LAUNCH_CHECK("k_tie_order");
    hipLaunchKernelGGL(k_level0, dim3(batches), dim3(kMergeThreads), 0, s, a2.at<uint32_t>(o_table0), features_d,
                       stats_d, key_b, key_e, keys_out, reinterpret_cast<const float*>(weight_out), work, tree,
                       scratch, node_count);
    MGB_LAUNCH_CHECK("k_level0");
  }
  // Levels with many nodes run four 256-thread workgroups per CU; the last
  // few levels, with fewer nodes than two per CU, give each merge 1,024
  // threads instead.
  for (size_t l = 0; l < tables.size(); ++l) {
    const uint32_t nodes = (uint32_t)(tables[l].size() / 2);
    if (nodes >= kWideLevelNodes)
      hipLaunchKernelGGL(k_level_up<kMergeThreads>, dim3(nodes), dim3(kMergeThreads), 0, s, (uint32_t)(l + 1),
                         a2.at<uint32_t>(o_tables[l]), features_d, work, tree, node_count, serial);
    else
      hipLaunchKernelGGL(k_level_up<kSketchThreads>, dim3(nodes), dim3(kSketchThreads), 0, s, (uint32_t)(l + 1),
                         a2.at<uint32_t>(o_tables[l]), features_d, work, tree, node_count, serial);
    MGB_LAUNCH_CHECK("k_level_up");
  }
  const uint32_t lds_bytes = sizeof(MergeLds<kSketchThreads>);
  if (hipFuncSetAttribute((const void*)k_finish, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes) != hipSuccess) {
    set_error("hipFuncSetAttribute(k_finish LDS) failed");
    return -1;
  }
  hipLaunchKernelGGL(k_finish, dim3(nf), dim3(kSketchThreads), lds_bytes, s, features_d, tree, node_count, serial,
                     a2.at<SkEntry>(o_fin), f0, max_bin, a2.at<uint32_t>(o_values),
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
  if (max_bin < 2 || max_bin > kMaxBinSketch) { set_error("max_bin must be in [2, 4096]"); return -1; }
  if (!cols) return 0;
  if (rows >= (1u << 31)) { set_error("sketch: rows must be below 2^31"); return -1; }
  // Feature groups of at most group_entries() entries and kMaxGroupFeatures
  // features.
  if (bound_device() < 0) return -1;
  const uint32_t group = (uint32_t)std::max<uint64_t>(
      1, std::min<uint64_t>(std::min<uint64_t>(cols, kMaxGroupFeatures), group_entries() / std::max(1u, rows)));
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
  if (max_bin < 2 || max_bin > kMaxBinSketch) { set_error("max_bin must be in [2, 4096]"); return -1; }
  if (!cols) return 0;
  if (bound_device() < 0) return -1;
  (void)rows;
  std::vector<uint64_t> colptr_host(cols + 1);
  MGB_CHECK(hipMemcpyAsync(colptr_host.data(), colptr, (cols + 1) * sizeof(uint64_t), hipMemcpyDeviceToHost, stream()));
  MGB_CHECK(hipStreamSynchronize(stream()));
  // Groups of whole columns of at most group_entries() entries (a longer
  // column forms a group of its own) and kMaxGroupFeatures columns.
  const uint64_t chunk = group_entries();
  for (uint32_t f0 = 0; f0 < cols;) {
    uint32_t f1 = f0 + 1;
    while (f1 < cols && f1 - f0 < kMaxGroupFeatures && colptr_host[f1 + 1] - colptr_host[f0] <= chunk) ++f1;
    std::vector<uint64_t> seg(f1 - f0 + 1);
    for (uint32_t c = 0; c <= f1 - f0; ++c) seg[c] = colptr_host[f0 + c] - colptr_host[f0];
    const uint64_t first = colptr_host[f0];
    if (sketch_group(values + first, seg, row_of + first, f1 - f0, f0, weights, max_bin, cuts, counts)) return -1;
    f0 = f1;
  }
  return 0;
}

int mgb_tie_sort_order(const uint32_t* keys, uint32_t n, uint32_t* order) {
  if (n && (!keys || !order)) { set_error("mgb_tie_sort_order: null argument"); return -1; }
  std::vector<uint32_t> k(keys, keys + n), id(n);
  for (uint32_t i = 0; i < n; ++i) id[i] = i;
  TieRuns r{k.data(), id.data()};
  tie_std_sort(r, n);
  for (uint32_t i = 0; i < n; ++i) order[i] = id[i];
  return 0;
}

int mgb_sketch_group_entries(uint64_t entries) {
  g_group_entries = entries;
  return 0;
}

}  // extern "C"
