// Weighted quantile sketch on the GPU: the per-feature cut points of the
// reference's hist method (src/quantile.cpp:22-212, kernels/quantile.metal.h,
// XGBoost's WQSummary semantics).
//
//  1. transpose the row-major matrix to columns (coalesced reads per feature);
//  2. one workgroup per feature finds runs of equal values in row order
//     (ballot + block scan), with run weights = run length or an in-order
//     binary32 weight sum;
//  3. the host plans batches of 2*limit runs (limit = sketch budget);
//  4. one segmented radix sort orders every batch by (value, position);
//  5. one workgroup per feature summarizes each batch, prunes, merges it into
//     the level stack, and finally selects the cuts.  Summaries, prunes and
//     merges are data-parallel restatements of the serial rules: prune
//     positions come from binary searches over monotone rank sums, merges from
//     merge-path ranks, and the error fix-up from prefix maxima, so every
//     binary32 rounding step is the same operation on the same operands.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cmath>
#include <vector>

#include "device_common.hpp"

namespace mgb {
namespace {

constexpr uint32_t kSketchThreads = 1024;

struct SkEntry { float rmin, rmax, wmin, value; };
struct SkStats { uint32_t nonmissing, elements, runs, padding; };
struct SkFeature {
  uint64_t lvl_offset, work_offset, scratch_offset;  // entries / words
  uint32_t limit, budget, batches, levels;
  uint32_t exact_integer, padding;
};

__device__ __forceinline__ uint32_t order_key(float v) {
  uint32_t bits = __float_as_uint(v);
  return bits ^ ((bits & 0x80000000u) ? 0xffffffffu : 0x80000000u);
}
__device__ __forceinline__ float min_next(const SkEntry& e) { return e.rmin + e.wmin; }
__device__ __forceinline__ float max_prev(const SkEntry& e) { return e.rmax - e.wmin; }

__global__ void k_transpose(const float* __restrict__ X, uint32_t rows, uint32_t cols, float* __restrict__ Xt) {
  __shared__ float tile[32][33];
  uint32_t c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  for (uint32_t k = threadIdx.y; k < 32; k += blockDim.y) {
    uint32_t r = r0 + k, c = c0 + threadIdx.x;
    if (r < rows && c < cols) tile[k][threadIdx.x] = X[(uint64_t)r * cols + c];
  }
  __syncthreads();
  for (uint32_t k = threadIdx.y; k < 32; k += blockDim.y) {
    uint32_t c = c0 + k, r = r0 + threadIdx.x;
    if (r < rows && c < cols) Xt[(uint64_t)c * rows + r] = tile[threadIdx.x][k];
  }
}

// Runs of equal values over a feature's non-missing, nonzero-weight entries in
// row order (kernels/quantile.metal.h:19-140).  Feature f's entries are
// vals[seg[f] .. seg[f+1]) in row order: a column of the transposed dense
// matrix (row = position) or of the column-major copy of a CSR matrix (row =
// row_of[position]); entries absent from a CSR column are missing values and
// take no part, exactly like NaN entries of a dense column.
__global__ __launch_bounds__(kSketchThreads) void k_runs(const float* __restrict__ vals, const uint64_t* __restrict__ seg,
                                                         const uint32_t* __restrict__ row_of,
                                                         const float* __restrict__ weights,
                                                         float* __restrict__ run_v, float* __restrict__ run_w,
                                                         uint32_t* __restrict__ run_start, float* __restrict__ elem_w,
                                                         SkStats* __restrict__ stats) {
  __shared__ uint32_t scan[kSketchThreads / kWave + 1];
  __shared__ uint32_t wave_has[kSketchThreads / kWave];
  __shared__ float wave_last[kSketchThreads / kWave];
  __shared__ uint32_t carry_has;
  __shared__ float carry_last;
  const uint32_t f = blockIdx.x;
  const uint64_t base = seg[f];
  const uint32_t rows = (uint32_t)(seg[f + 1] - base);  // entries of this feature
  const float* col = vals + base;
  const uint32_t lane = lane_id(), wave = threadIdx.x / kWave, waves = blockDim.x / kWave;
  uint32_t elements = 0, runs = 0, nonmissing = 0;
  if (threadIdx.x == 0) { carry_has = 0; carry_last = 0; }
  __syncthreads();
  for (uint32_t t0 = 0; t0 < rows; t0 += blockDim.x) {
    const uint32_t r = t0 + threadIdx.x;
    float v = r < rows ? col[r] : __uint_as_float(0x7fc00000u);
    float w = (r < rows && weights) ? weights[row_of ? row_of[base + r] : r] : 1.0f;
    const bool present = !isnan(v);
    const bool valid = present && (__float_as_uint(w) & 0x7fffffffu) != 0;
    const uint64_t mask = __ballot(valid);
    const uint64_t below = mask & (lane ? (~0ull >> (64 - lane)) : 0ull);
    float prev = __shfl(v, below ? 63 - __clzll(below) : 0, kWave);
    bool have_prev = below != 0;
    const float last_in_wave = __shfl(v, mask ? 63 - __clzll(mask) : 0, kWave);
    if (lane == 0) {
      wave_has[wave] = mask != 0;
      wave_last[wave] = last_in_wave;
    }
    __syncthreads();
    if (!have_prev) {
      for (int k = (int)wave - 1; k >= 0; --k) {
        if (wave_has[k]) { prev = wave_last[k]; have_prev = true; break; }
      }
      if (!have_prev && carry_has) { prev = carry_last; have_prev = true; }
    }
    const bool new_run = valid && (!have_prev || v != prev);
    uint32_t total_valid, total_runs, total_present;
    const uint32_t eidx = elements + block_exclusive_u32(valid ? 1u : 0u, scan, &total_valid);
    const uint32_t ridx = runs + block_exclusive_u32(new_run ? 1u : 0u, scan, &total_runs);
    block_exclusive_u32(present ? 1u : 0u, scan, &total_present);
    if (valid && weights) elem_w[base + eidx] = w;
    if (new_run) { run_v[base + ridx] = v; run_start[base + ridx] = eidx; }
    elements += total_valid;
    runs += total_runs;
    nonmissing += total_present;
    if (threadIdx.x == 0) {
      for (int k = (int)waves - 1; k >= 0; --k)
        if (wave_has[k]) { carry_has = 1; carry_last = wave_last[k]; break; }
    }
    __syncthreads();
  }
  for (uint32_t k = threadIdx.x; k < runs; k += blockDim.x) {
    uint32_t s = run_start[base + k];
    uint32_t e = k + 1 < runs ? run_start[base + k + 1] : elements;
    float w;
    if (!weights) {
      uint32_t len = e - s;
      w = (float)(len < (1u << 24) ? len : (1u << 24));
    } else {
      w = elem_w[base + s];
      for (uint32_t i = s + 1; i < e; ++i) w = w + elem_w[base + i];
    }
    run_w[base + k] = w;
  }
  if (threadIdx.x == 0) stats[f] = SkStats{nonmissing, elements, runs, 0};
}

// One workgroup per feature: sort keys (value order, run index) of its runs.
__global__ void k_keys(const float* __restrict__ run_v, const SkStats* __restrict__ stats,
                       const uint64_t* __restrict__ seg, uint64_t* __restrict__ keys) {
  const uint32_t f = blockIdx.x;
  const uint64_t base = seg[f];
  const uint32_t runs = stats[f].runs;
  for (uint32_t k = threadIdx.x; k < runs; k += blockDim.x)
    keys[base + k] = ((uint64_t)order_key(run_v[base + k]) << 32) | k;
}

// ---------------------------------------------------------------------------
// Per-feature reduction.
// ---------------------------------------------------------------------------
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

// kernels/quantile.metal.h:192-214 (sketch_prune_serial), data-parallel.
// The serial loop walks i forward while rank_k >= rmax_{i+1} + rmin_{i+1};
// both ranks and these sums are nondecreasing, so i_k is a binary search and
// the chosen indices c_k are nondecreasing: "append if c_k != last" keeps the
// first k of each run of equal c_k.  in[0..size) -> out (out != in).
__device__ uint32_t prune(const SkEntry* in, uint32_t size, uint32_t capacity, SkEntry* out, uint32_t* scan) {
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
  if (threadIdx.x == 0) { out[0] = in[0]; s_last = 0; s_dead = 0; }
  __syncthreads();
  uint32_t carry = 0, prev_chunk = 0;
  for (uint32_t base = 1; base < n; base += blockDim.x) {
    const uint32_t k = base + threadIdx.x;
    uint32_t choice = 0;
    bool live = false;
    if (k < n) {
      const float rank = 2.0f * (((float)k * range) / (float)n + begin);
      uint32_t lo = 2, hi = size;  // first j in [2, size) with rank < rmax_j + rmin_j
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
// a[0..n) and b[0..m) -> out; out must differ from both.
__device__ uint32_t combine(const SkEntry* a, uint32_t n, const SkEntry* b, uint32_t m, SkEntry* out,
                            uint32_t* eq_prefix, uint32_t* scan) {
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
  // Equal-value pairs, indexed by a: eq_prefix[i] = #pairs with a-index < i.
  uint32_t carry = 0;
  for (uint32_t base = 0; base < n; base += blockDim.x) {
    uint32_t i = base + threadIdx.x;
    uint32_t eq = 0;
    if (i < n) {
      float x = a[i].value;
      uint32_t lo = 0, hi = m;
      while (lo < hi) { uint32_t mid = lo + (hi - lo) / 2; if (b[mid].value < x) lo = mid + 1; else hi = mid; }
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
    uint32_t lo = 0, hi = m;
    while (lo < hi) { uint32_t mid = lo + (hi - lo) / 2; if (b[mid].value < x.value) lo = mid + 1; else hi = mid; }
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
    uint32_t lo = 0, hi = n;
    while (lo < hi) { uint32_t mid = lo + (hi - lo) / 2; if (a[mid].value < y.value) lo = mid + 1; else hi = mid; }
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

// Summary of one sorted batch (kernels/quantile.metal.h:216-240).
__device__ uint32_t summarize(const uint64_t* keys, const float* run_v, const float* run_w, uint32_t size, bool exact,
                              SkEntry* out, uint32_t* scratch, uint32_t* scan) {
  if (!exact) {
    __shared__ uint32_t result;
    if (threadIdx.x == 0) {
      uint32_t n = 0;
      float total = 0;
      for (uint32_t i = 0; i < size;) {
        uint32_t k = (uint32_t)keys[i];
        float value = run_v[k], weight = run_w[k];
        uint32_t j = i + 1;
        while (j < size && run_v[(uint32_t)keys[j]] == value) weight = weight + run_w[(uint32_t)keys[j++]];
        out[n++] = SkEntry{total, total + weight, weight, value};
        total = total + weight;
        i = j;
      }
      result = n;
    }
    __syncthreads();
    return result;
  }
  // Integer weights with a total below 2^24: every binary32 partial sum is
  // exact, so a parallel prefix reproduces the serial sums bit for bit.
  uint32_t carry_w = 0, carry_s = 0;
  for (uint32_t base = 0; base < size; base += blockDim.x) {
    uint32_t i = base + threadIdx.x;
    uint32_t w = 0, start = 0;
    float v = 0;
    if (i < size) {
      uint32_t k = (uint32_t)keys[i];
      v = run_v[k];
      w = (uint32_t)run_w[k];
      start = i == 0 || run_v[(uint32_t)keys[i - 1]] != v;
    }
    uint32_t tw, ts;
    uint32_t pw = block_exclusive_u32(w, scan, &tw) + carry_w;
    uint32_t ps = block_exclusive_u32(start, scan, &ts) + carry_s;
    if (start) {
      scratch[ps] = pw;
      out[ps].value = v;
    }
    carry_w += tw;
    carry_s += ts;
  }
  if (threadIdx.x == 0) scratch[carry_s] = carry_w;
  __syncthreads();
  const uint32_t n = carry_s;
  for (uint32_t o = threadIdx.x; o < n; o += blockDim.x) {
    uint32_t p = scratch[o], q = scratch[o + 1];
    out[o].rmin = (float)p;
    out[o].rmax = (float)q;
    out[o].wmin = (float)(q - p);
  }
  __syncthreads();
  return n;
}

__global__ __launch_bounds__(kSketchThreads) void k_reduce(const uint64_t* __restrict__ keys,
                                                           const float* __restrict__ run_v,
                                                           const float* __restrict__ run_w,
                                                           const SkStats* __restrict__ stats,
                                                           const SkFeature* __restrict__ features,
                                                           const uint64_t* __restrict__ seg,
                                                           uint32_t max_bin, SkEntry* __restrict__ levels,
                                                           SkEntry* __restrict__ work, uint32_t* __restrict__ scratch_u,
                                                           float* __restrict__ cut_values, float* __restrict__ cuts,
                                                           uint32_t* __restrict__ counts) {
  __shared__ uint32_t scan[kSketchThreads / kWave + 1];
  __shared__ uint32_t level_count[64];
  const uint32_t f = blockIdx.x;
  const SkFeature fe = features[f];
  const SkStats st = stats[f];
  const uint64_t base = seg[f];
  const uint32_t limit = fe.limit;
  const uint32_t cap = 2 * limit + 2;
  SkEntry* bufA = work + fe.work_offset;
  SkEntry* bufB = bufA + cap;
  uint32_t* scratch = scratch_u + fe.scratch_offset;
  SkEntry* lvl = levels + fe.lvl_offset;
  for (uint32_t i = threadIdx.x; i < 64; i += blockDim.x) level_count[i] = 0;
  __syncthreads();
  const uint64_t capacity = 2ull * limit;
  for (uint64_t begin = 0; begin < st.runs; begin += capacity) {
    uint32_t size = (uint32_t)((st.runs - begin) < capacity ? (st.runs - begin) : capacity);
    uint32_t n = summarize(keys + base + begin, run_v + base, run_w + base, size, fe.exact_integer != 0, bufA,
                           scratch, scan);
    SkEntry* cur = bufA;
    SkEntry* oth = bufB;
    uint32_t level = 0;
    for (;;) {
      n = prune(cur, n, limit, oth, scan);
      { SkEntry* t = cur; cur = oth; oth = t; }
      uint32_t m = level_count[level];
      if (m) {
        n = combine(cur, n, lvl + (uint64_t)level * limit, m, oth, scratch, scan);
        SkEntry* t = cur; cur = oth; oth = t;
      }
      __syncthreads();
      if (threadIdx.x == 0) level_count[level] = 0;
      __syncthreads();
      if (n <= limit) break;
      ++level;
    }
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) lvl[(uint64_t)level * limit + i] = cur[i];
    __syncthreads();
    if (threadIdx.x == 0) level_count[level] = n;
    __syncthreads();
  }
  // Final combine over the levels, then prune to the budget.
  SkEntry* cur = bufA;
  SkEntry* oth = bufB;
  uint32_t n = 0;
  const uint32_t final_cap = fe.budget > limit ? fe.budget : limit;
  for (uint32_t level = 0; level < fe.levels && level < 64; ++level) {
    uint32_t m = level_count[level];
    if (m) {
      n = combine(cur, n, lvl + (uint64_t)level * limit, m, oth, scratch, scan);
      SkEntry* t = cur; cur = oth; oth = t;
    }
    n = prune(cur, n, final_cap, oth, scan);
    SkEntry* t = cur; cur = oth; oth = t;
  }
  n = prune(cur, n, fe.budget, oth, scan);
  { SkEntry* t = cur; cur = oth; oth = t; }
  // Cuts (kernels/quantile.metal.h:354-400).
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
      float tail = cur[size - 1].value;
      out[size - 1] = tail + (fabsf(tail) + 1e-5f);
      counts[f] = size;
    }
    return;
  }
  // Rank queries in parallel; the order-preserving dedup pass is serial.
  float* values = cut_values + (uint64_t)f * max_bin;
  const double total = (double)cur[size - 1].rmax, denominator = (double)max_bin;
  for (uint32_t i = 1 + threadIdx.x; i < max_bin; i += blockDim.x) {
    double rank = ((double)i * total) / denominator * 2.0;
    uint32_t lo = 1, hi = size - 1;  // cursor = #{j in [1, size-2] : rmin_j + rmax_j <= rank}
    while (lo < hi) {
      uint32_t mid = lo + (hi - lo) / 2;
      if (rank >= (double)(cur[mid].rmin + cur[mid].rmax)) lo = mid + 1;
      else hi = mid;
    }
    uint32_t cursor = lo - 1;
    float boundary = min_next(cur[cursor]) + max_prev(cur[cursor + 1]);
    values[i] = cur[cursor + ((isnan(boundary) || rank >= (double)boundary) ? 1u : 0u)].value;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float last = cur[0].value;
    uint32_t next = 1, count = 0;
    for (uint32_t i = 1; i < max_bin; ++i) {
      float value = values[i];
      if (value <= last) {
        while (next < size && cur[next].value <= last) ++next;
        if (next == size) break;
        value = cur[next].value;
      } else if (next < size && cur[next].value <= value) {
        do { ++next; } while (next < size && cur[next].value <= value);
      }
      out[count++] = value;
      last = value;
    }
    float tail = cur[size - 1].value;
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

struct DeviceBuffer {
  void* p = nullptr;
  ~DeviceBuffer() { if (p) (void)hipFree(p); }
  int alloc(size_t bytes) { return check(hipMalloc(&p, bytes ? bytes : 16), "hipMalloc(sketch)"); }
};

// Cuts of `cols` features whose entries are vals[seg[f] .. seg[f+1]) (device
// values; host and device copies of the offsets), see k_runs.
int sketch_segments(const float* vals, const std::vector<uint64_t>& seg_host, const uint32_t* row_of,
                    uint32_t cols, const float* weights, uint32_t max_bin, float* cuts, uint32_t* counts) {
  hipStream_t s = stream();
  const uint64_t total = seg_host[cols];
  // Positions are 32-bit and the segmented sort counts in int.
  if (total >= (1ull << 31)) { set_error("sketch: more than 2^31 - 1 entries"); return -1; }
  const uint64_t alloc = total ? total : 1;
  DeviceBuffer seg_d, run_v, run_w, run_start, elem_w, stats_d, keys_in, keys_out;
  if (seg_d.alloc((cols + 1) * sizeof(uint64_t)) || run_v.alloc(alloc * 4) || run_w.alloc(alloc * 4) ||
      run_start.alloc(alloc * 4) || stats_d.alloc(cols * sizeof(SkStats)) || keys_in.alloc(alloc * 8) ||
      keys_out.alloc(alloc * 8))
    return -1;
  if (weights && elem_w.alloc(alloc * 4)) return -1;
  MGB_CHECK(hipMemcpyAsync(seg_d.p, seg_host.data(), (cols + 1) * sizeof(uint64_t), hipMemcpyHostToDevice, s));
  hipLaunchKernelGGL(k_runs, dim3(cols), dim3(kSketchThreads), 0, s, vals, (const uint64_t*)seg_d.p, row_of, weights,
                     (float*)run_v.p, (float*)run_w.p, (uint32_t*)run_start.p, (float*)elem_w.p,
                     (SkStats*)stats_d.p);
  MGB_LAUNCH_CHECK("k_runs");
  std::vector<SkStats> stats(cols);
  MGB_CHECK(hipMemcpyAsync(stats.data(), stats_d.p, cols * sizeof(SkStats), hipMemcpyDeviceToHost, s));
  MGB_CHECK(hipStreamSynchronize(s));
  // Batch plan (src/quantile.cpp:87-122).
  std::vector<SkFeature> features(cols);
  std::vector<uint32_t> seg_begin, seg_end;
  uint64_t lvl_total = 0, work_total = 0, scratch_total = 0;
  for (uint32_t f = 0; f < cols; ++f) {
    const SkStats& st = stats[f];
    uint32_t limit = sketch_budget(max_bin, st.nonmissing);
    uint32_t budget = sketch_budget(max_bin, st.elements);
    uint64_t capacity = 2ull * limit;
    uint32_t batches = 0;
    for (uint64_t b = 0; b < st.runs; b += capacity) {
      uint64_t size = std::min<uint64_t>(capacity, st.runs - b);
      seg_begin.push_back((uint32_t)(seg_host[f] + b));
      seg_end.push_back((uint32_t)(seg_host[f] + b + size));
      ++batches;
    }
    uint32_t levels = bit_width(std::max(1u, batches)) + 1;
    SkFeature fe{};
    fe.lvl_offset = lvl_total;
    fe.work_offset = work_total;
    fe.limit = limit;
    fe.budget = budget;
    fe.batches = batches;
    fe.levels = levels;
    fe.exact_integer = !weights && st.elements <= (1u << 24);
    fe.scratch_offset = scratch_total;
    features[f] = fe;
    lvl_total += (uint64_t)limit * (levels + 1);
    work_total += 2 * (2ull * limit + 2);
    scratch_total += 2ull * limit + 4;
  }
  DeviceBuffer levels_d, work_d, scratch_d, feat_d, values_d, seg_b, seg_e, temp;
  if (levels_d.alloc(lvl_total * sizeof(SkEntry)) || work_d.alloc(work_total * sizeof(SkEntry)) ||
      feat_d.alloc(cols * sizeof(SkFeature)) || values_d.alloc((uint64_t)cols * max_bin * 4))
    return -1;
  if (scratch_d.alloc(scratch_total * 4)) return -1;
  MGB_CHECK(hipMemcpyAsync(feat_d.p, features.data(), cols * sizeof(SkFeature), hipMemcpyHostToDevice, s));
  if (!seg_begin.empty()) {
    hipLaunchKernelGGL(k_keys, dim3(cols), dim3(256), 0, s, (const float*)run_v.p, (const SkStats*)stats_d.p,
                       (const uint64_t*)seg_d.p, (uint64_t*)keys_in.p);
    MGB_LAUNCH_CHECK("k_keys");
    if (seg_b.alloc(seg_begin.size() * 4) || seg_e.alloc(seg_end.size() * 4)) return -1;
    MGB_CHECK(hipMemcpyAsync(seg_b.p, seg_begin.data(), seg_begin.size() * 4, hipMemcpyHostToDevice, s));
    MGB_CHECK(hipMemcpyAsync(seg_e.p, seg_end.data(), seg_end.size() * 4, hipMemcpyHostToDevice, s));
    size_t temp_bytes = 0;
    MGB_CHECK(hipcub::DeviceSegmentedRadixSort::SortKeys(nullptr, temp_bytes, (const uint64_t*)keys_in.p,
                                                          (uint64_t*)keys_out.p, (int)total, (int)seg_begin.size(),
                                                          (const uint32_t*)seg_b.p, (const uint32_t*)seg_e.p, 0, 64,
                                                          s));
    if (temp.alloc(temp_bytes)) return -1;
    MGB_CHECK(hipcub::DeviceSegmentedRadixSort::SortKeys(temp.p, temp_bytes, (const uint64_t*)keys_in.p,
                                                          (uint64_t*)keys_out.p, (int)total, (int)seg_begin.size(),
                                                          (const uint32_t*)seg_b.p, (const uint32_t*)seg_e.p, 0, 64,
                                                          s));
  }
  hipLaunchKernelGGL(k_reduce, dim3(cols), dim3(kSketchThreads), 0, s, (const uint64_t*)keys_out.p,
                     (const float*)run_v.p, (const float*)run_w.p, (const SkStats*)stats_d.p,
                     (const SkFeature*)feat_d.p, (const uint64_t*)seg_d.p, max_bin, (SkEntry*)levels_d.p,
                     (SkEntry*)work_d.p, (uint32_t*)scratch_d.p, (float*)values_d.p, cuts, counts);
  MGB_LAUNCH_CHECK("k_reduce");
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
  const uint64_t total = (uint64_t)rows * cols;
  if (total >= (1ull << 31)) { set_error("sketch: rows*cols must be below 2^31"); return -1; }
  DeviceBuffer xt;
  if (xt.alloc((total ? total : 1) * 4)) return -1;
  if (rows) {
    dim3 grid((cols + 31) / 32, (rows + 31) / 32), block(32, 8);
    hipLaunchKernelGGL(k_transpose, grid, block, 0, stream(), X, rows, cols, (float*)xt.p);
    MGB_LAUNCH_CHECK("k_transpose");
  }
  std::vector<uint64_t> seg(cols + 1);
  for (uint32_t f = 0; f <= cols; ++f) seg[f] = (uint64_t)f * rows;
  return sketch_segments((const float*)xt.p, seg, nullptr, cols, weights, max_bin, cuts, counts);
}

int mgb_sketch_cuts_csc(const float* values, const uint32_t* row_of, const uint64_t* colptr, uint32_t rows,
                        uint32_t cols, const float* weights, uint32_t max_bin, float* cuts, uint32_t* counts) {
  if (max_bin < 2) { set_error("max_bin must be at least 2"); return -1; }
  if (!cols) return 0;
  (void)rows;
  std::vector<uint64_t> seg(cols + 1);
  MGB_CHECK(hipMemcpyAsync(seg.data(), colptr, (cols + 1) * sizeof(uint64_t), hipMemcpyDeviceToHost, stream()));
  MGB_CHECK(hipStreamSynchronize(stream()));
  return sketch_segments(values, seg, row_of, cols, weights, max_bin, cuts, counts);
}

}  // extern "C"
