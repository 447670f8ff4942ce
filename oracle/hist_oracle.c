/*
 * hist_oracle.c -- CPU restatement of the reference's hist tree-boosting path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker).  Only tests/, the smoke
 * check in __graft_entry__.py and bench.py's cpu_baseline leg may load it; the
 * product library never links or calls it.
 *
 * Citations are reference-relative paths (file:line).  The reference's kernels
 * emulate binary64 in software because its GPU lacks fp64; here every such
 * step is written with native IEEE binary64/binary32 arithmetic, compiled with
 * -ffp-contract=off so that only the explicit fma() calls fuse.
 *
 * Parity pins (see tests/test_oracle.py):
 *  - end to end: three prediction SHA-256 known answers published by the
 *    reference (benchmarks/results/2026-11-12/controlled-comparison.json),
 *    produced identically by stock XGBoost 3.4.1 CPU and by the reference;
 *  - sketch/bins: invariants (sorted, strictly increasing, <= max_bin, tail
 *    sentinel) and exact closed forms for small distinct-value columns;
 *  - quantization: arbitrary-precision integer check of the scale;
 *  - histograms: brute-force integer sums;
 *  - scoring: exact-rational double-rounding constructions
 *    (tests/test_scalar_weight.py:29-71 of the reference);
 *  - tree: constructed known answers (tests/test_histogram_present.py:81).
 *  - logistic: the sigmoid is upstream XGBoost's expression over the host
 *    libm's expf, as stock XGBoost computes it (the library's device exp is
 *    checked against the same libm on all 2^32 inputs, tests/test_expf.py).
 * Parity unpinned: weighted sketches with tied values (the reference
 * emulates libc++ std::sort permutations).
 */
#include "hist_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif
#include <stddef.h>

/* ------------------------------------------------------------------------ */
/* Quantile sketch (weighted quantile summary, XGBoost WQSummary semantics)  */
/* ------------------------------------------------------------------------ */

typedef struct { float rmin, rmax, wmin, value; } SkEntry;
typedef struct { float value, weight; uint32_t order; } SkRun;

/* src/quantile.cpp:11-19 */
uint32_t oracle_sketch_budget(uint32_t bins, uint32_t count) {
  if (!count) return 1;
  double epsilon = 1.0 / (double)(bins < count ? bins : count);
  for (uint32_t level = 1; level < 32; ++level) {
    uint64_t limit = (uint64_t)ceil(level / (epsilon / 2.0)) + 1;
    if (limit > count) limit = count;
    if (((uint64_t)1 << level) * limit >= count) return (uint32_t)limit;
  }
  return count;
}

static float sk_min_next(SkEntry e) { return e.rmin + e.wmin; }   /* kernels/quantile.metal.h:14 */
static float sk_max_prev(SkEntry e) { return e.rmax - e.wmin; }   /* kernels/quantile.metal.h:15 */

/* kernels/quantile.metal.h:192-214 (sketch_prune_serial) */
static uint32_t sk_prune(SkEntry* e, uint32_t size, uint32_t capacity) {
  if (size <= capacity) return size;
  if (!capacity) return 0;
  if (capacity == 1) return 1;
  float begin = e[0].rmax, range = e[size - 1].rmin - begin;
  uint32_t n = capacity - 1, count = 1, i = 1, last = 0;
  SkEntry tail = e[size - 1], left = e[1], right = e[2];
  for (uint32_t k = 1; k < n; ++k) {
    float rank = 2.0f * (((float)k * range) / (float)n + begin);
    while (i < size - 1 && rank >= right.rmax + right.rmin) {
      ++i;
      left = right;
      if (i < size - 1) right = e[i + 1];
    }
    if (i == size - 1) break;
    if (rank < sk_min_next(left) + sk_max_prev(right)) {
      if (i != last) { e[count++] = left; last = i; }
    } else if (i + 1 != last) {
      e[count++] = right;
      last = i + 1;
    }
  }
  if (last != size - 1) e[count++] = tail;
  return count;
}

/* kernels/quantile.metal.h:266-311 (sketch_combine_serial) */
static uint32_t sk_combine(SkEntry* cur, uint32_t n, const SkEntry* other, uint32_t m, SkEntry* scratch) {
  if (!m) return n;
  if (!n) {
    memcpy(cur, other, (size_t)m * sizeof(SkEntry));
    return m;
  }
  uint32_t a = 0, b = 0, count = 0;
  float prev_a = 0, prev_b = 0;
  while (a < n && b < m) {
    SkEntry x = cur[a], y = other[b], r;
    if (x.value == y.value) {
      r.rmin = x.rmin + y.rmin; r.rmax = x.rmax + y.rmax; r.wmin = x.wmin + y.wmin; r.value = x.value;
      prev_a = sk_min_next(x); prev_b = sk_min_next(y);
      ++a; ++b;
    } else if (x.value < y.value) {
      r.rmin = x.rmin + prev_b; r.rmax = x.rmax + sk_max_prev(y); r.wmin = x.wmin; r.value = x.value;
      prev_a = sk_min_next(x);
      ++a;
    } else {
      r.rmin = y.rmin + prev_a; r.rmax = y.rmax + sk_max_prev(x); r.wmin = y.wmin; r.value = y.value;
      prev_b = sk_min_next(y);
      ++b;
    }
    scratch[count++] = r;
  }
  float tail_a = cur[n - 1].rmax, tail_b = other[m - 1].rmax;
  while (a < n) {
    SkEntry x = cur[a++];
    SkEntry r = {x.rmin + prev_b, x.rmax + tail_b, x.wmin, x.value};
    scratch[count++] = r;
  }
  while (b < m) {
    SkEntry y = other[b++];
    SkEntry r = {y.rmin + prev_a, y.rmax + tail_a, y.wmin, y.value};
    scratch[count++] = r;
  }
  float prev_min = 0, prev_max = 0;
  for (uint32_t i = 0; i < count; ++i) {
    SkEntry e = scratch[i];
    if (e.rmin < prev_min) e.rmin = prev_min;
    else prev_min = e.rmin;
    if (e.rmax < prev_max) e.rmax = prev_max;
    if (e.rmax < sk_min_next(e)) e.rmax = sk_min_next(e);
    prev_max = e.rmax;
    cur[i] = e;
  }
  return count;
}

/* std::sort as libstdc++ implements it (GCC 11, bits/stl_algo.h and
 * bits/stl_heap.h), restated for an array of `size`-byte elements ordered by
 * `less`: introsort with a depth limit of 2 floor(log2 n), the median of the
 * second, middle and last elements moved to the front as the pivot, an
 * unguarded partition, heap sort when the depth runs out, and a final
 * insertion sort (the first 16 elements guarded, the rest unguarded).
 * Elements that compare equal end in the order these steps leave them: the
 * order stock XGBoost's x86-64 build merges equal sketch values in
 * (tests/golden/sort_ties_libstdcxx.json, written by this image's g++, pins
 * it). */
typedef int (*sk_less_fn)(const void* a, const void* b);
typedef struct {
  char* base;
  size_t size;
  sk_less_fn less;
  uint64_t* heap_sorts; /* heap-sort fallbacks taken (a test statistic; may be NULL) */
} SkSort;
#define SK_AT(s, i) ((s)->base + (size_t)(i) * (s)->size)

static void sk_swap(const SkSort* s, size_t a, size_t b) {
  char t[16];
  memcpy(t, SK_AT(s, a), s->size);
  memcpy(SK_AT(s, a), SK_AT(s, b), s->size);
  memcpy(SK_AT(s, b), t, s->size);
}

/* __move_median_to_first */
static void sk_median_to_first(const SkSort* s, size_t result, size_t a, size_t b, size_t c) {
  if (s->less(SK_AT(s, a), SK_AT(s, b))) {
    if (s->less(SK_AT(s, b), SK_AT(s, c))) sk_swap(s, result, b);
    else if (s->less(SK_AT(s, a), SK_AT(s, c))) sk_swap(s, result, c);
    else sk_swap(s, result, a);
  } else if (s->less(SK_AT(s, a), SK_AT(s, c))) {
    sk_swap(s, result, a);
  } else if (s->less(SK_AT(s, b), SK_AT(s, c))) {
    sk_swap(s, result, c);
  } else {
    sk_swap(s, result, b);
  }
}

/* __unguarded_partition */
static size_t sk_unguarded_partition(const SkSort* s, size_t first, size_t last, size_t pivot) {
  for (;;) {
    while (s->less(SK_AT(s, first), SK_AT(s, pivot))) ++first;
    --last;
    while (s->less(SK_AT(s, pivot), SK_AT(s, last))) --last;
    if (!(first < last)) return first;
    sk_swap(s, first, last);
    ++first;
  }
}

/* __adjust_heap with __push_heap, over elements [first, first + len) */
static void sk_adjust_heap(const SkSort* s, size_t first, ptrdiff_t hole, ptrdiff_t len, const char* value) {
  const ptrdiff_t top = hole;
  ptrdiff_t child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (s->less(SK_AT(s, first + child), SK_AT(s, first + child - 1))) --child;
    memcpy(SK_AT(s, first + hole), SK_AT(s, first + child), s->size);
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    memcpy(SK_AT(s, first + hole), SK_AT(s, first + child - 1), s->size);
    hole = child - 1;
  }
  ptrdiff_t parent = (hole - 1) / 2;
  while (hole > top && s->less(SK_AT(s, first + parent), value)) {
    memcpy(SK_AT(s, first + hole), SK_AT(s, first + parent), s->size);
    hole = parent;
    parent = (hole - 1) / 2;
  }
  memcpy(SK_AT(s, first + hole), value, s->size);
}

/* __partial_sort(first, last, last): __make_heap then __sort_heap */
static void sk_heap_sort(const SkSort* s, size_t first, size_t last) {
  char value[16];
  const ptrdiff_t len = (ptrdiff_t)(last - first);
  if (s->heap_sorts) ++*s->heap_sorts;
  if (len < 2) return;
  for (ptrdiff_t parent = (len - 2) / 2;; --parent) {
    memcpy(value, SK_AT(s, first + parent), s->size);
    sk_adjust_heap(s, first, parent, len, value);
    if (parent == 0) break;
  }
  for (size_t end = last; end - first > 1;) {
    --end;
    memcpy(value, SK_AT(s, end), s->size);
    memcpy(SK_AT(s, end), SK_AT(s, first), s->size);
    sk_adjust_heap(s, first, 0, (ptrdiff_t)(end - first), value);
  }
}

/* __introsort_loop */
static void sk_introsort(const SkSort* s, size_t first, size_t last, int depth) {
  while (last - first > 16) {
    if (depth == 0) {
      sk_heap_sort(s, first, last);
      return;
    }
    --depth;
    const size_t mid = first + (last - first) / 2;
    sk_median_to_first(s, first, first + 1, mid, last - 1);
    const size_t cut = sk_unguarded_partition(s, first + 1, last, first);
    sk_introsort(s, cut, last, depth);
    last = cut;
  }
}

/* __unguarded_linear_insert */
static void sk_linear_insert(const SkSort* s, size_t last) {
  char value[16];
  memcpy(value, SK_AT(s, last), s->size);
  size_t next = last - 1;
  while (s->less(value, SK_AT(s, next))) {
    memcpy(SK_AT(s, last), SK_AT(s, next), s->size);
    last = next;
    --next;
  }
  memcpy(SK_AT(s, last), value, s->size);
}

/* __insertion_sort */
static void sk_insertion_sort(const SkSort* s, size_t first, size_t last) {
  char value[16];
  for (size_t i = first + 1; i < last; ++i) {
    if (s->less(SK_AT(s, i), SK_AT(s, first))) {
      memcpy(value, SK_AT(s, i), s->size);
      memmove(SK_AT(s, first + 1), SK_AT(s, first), (i - first) * s->size);
      memcpy(SK_AT(s, first), value, s->size);
    } else {
      sk_linear_insert(s, i);
    }
  }
}

static void sk_std_sort(void* base, size_t n, size_t size, sk_less_fn less, uint64_t* heap_sorts) {
  if (n < 2) return;
  const SkSort s = {(char*)base, size, less, heap_sorts};
  int lg = 0;
  while (((size_t)2 << lg) <= n) ++lg; /* std::__lg(n): floor(log2 n) */
  sk_introsort(&s, 0, n, 2 * lg);
  if (n > 16) {
    sk_insertion_sort(&s, 0, 16);
    for (size_t i = 16; i < n; ++i) sk_linear_insert(&s, i);
  } else {
    sk_insertion_sort(&s, 0, n);
  }
}

/* The sketch entries' order: the value alone (upstream WQSummary's entries
 * compare values; -0 and +0 are equal). */
static int sk_run_less(const void* a, const void* b) { return ((const SkRun*)a)->value < ((const SkRun*)b)->value; }

typedef struct { uint32_t key, id; } SkKeyed;
static int sk_keyed_less(const void* a, const void* b) { return ((const SkKeyed*)a)->key < ((const SkKeyed*)b)->key; }

/* Test hook: the ids 0..n-1 of elements with the given keys, in the order the
 * restated std::sort leaves them; returns the heap-sort fallbacks taken. */
uint64_t oracle_std_sort_order(const uint32_t* keys, uint32_t n, uint32_t* order) {
  SkKeyed* v = (SkKeyed*)malloc(sizeof(SkKeyed) * (n ? n : 1));
  for (uint32_t i = 0; i < n; ++i) { v[i].key = keys[i]; v[i].id = i; }
  uint64_t heap_sorts = 0;
  sk_std_sort(v, n, sizeof(SkKeyed), sk_keyed_less, &heap_sorts);
  for (uint32_t i = 0; i < n; ++i) order[i] = v[i].id;
  free(v);
  return heap_sorts;
}

/* kernels/quantile.metal.h:216-240 (sketch_summarize_ordered) over a batch of
 * runs in row order: they are sorted by value with std::sort (libstdc++'s
 * steps, above) and equal values are merged in the order it leaves them --
 * the first one's value (the sign of a zero) and the weights added in that
 * order, as stock XGBoost's x86-64 build merges them (upstream
 * WQSummary::Queue::MakeSummary).  The reference reproduces libc++'s order
 * the same way for its macOS builds (kernels/sketch_sort.metal.h). */
static uint32_t sk_summarize(SkRun* runs, uint32_t size, uint32_t limit, SkEntry* out) {
  sk_std_sort(runs, size, sizeof(SkRun), sk_run_less, NULL);
  uint32_t n = 0;
  float total = 0;
  for (uint32_t i = 0; i < size;) {
    float value = runs[i].value, weight = runs[i].weight;
    uint32_t j = i + 1;
    while (j < size && runs[j].value == value) weight = weight + runs[j++].weight;
    SkEntry e = {total, total + weight, weight, value};
    out[n++] = e;
    total = total + weight;
    i = j;
  }
  return sk_prune(out, n, limit);
}

/* kernels/quantile.metal.h:354-400 (sketch_cuts_serial), numeric features. */
static uint32_t sk_cuts(const SkEntry* e, uint32_t size, uint32_t numeric_bins, float* out) {
  uint32_t count = 0;
  if (!size) { out[0] = 1e-5f; return 1; }
  if (size <= numeric_bins) {
    float last = e[0].value;
    for (uint32_t i = 1; i < size; ++i) {
      float value = e[i].value;
      if (last < value) { out[count++] = value; last = value; }
    }
  } else {
    float last = e[0].value;
    uint32_t next = 1, cursor = 0;
    double total = (double)e[size - 1].rmax, denominator = (double)numeric_bins;
    for (uint32_t i = 1; i < numeric_bins; ++i) {
      double rank = ((double)i * total) / denominator * 2.0;
      while (cursor < size - 2 && rank >= (double)(e[cursor + 1].rmin + e[cursor + 1].rmax)) ++cursor;
      float boundary = sk_min_next(e[cursor]) + sk_max_prev(e[cursor + 1]);
      float value = e[cursor + (uint32_t)(isnan(boundary) || rank >= (double)boundary)].value;
      if (value <= last) {
        while (next < size && e[next].value <= last) ++next;
        if (next == size) break;
        value = e[next].value;
      } else if (next < size && e[next].value <= value) {
        do { ++next; } while (next < size && e[next].value <= value);
      }
      out[count++] = value;
      last = value;
    }
  }
  float tail = e[size - 1].value;
  out[count++] = tail + (fabsf(tail) + 1e-5f);
  return count;
}

static uint32_t bit_width_u32(uint32_t v) { return v ? 32u - (uint32_t)__builtin_clz(v) : 0u; }

/* One numeric feature: src/quantile.cpp:22-212 with the serial kernels
 * sketch_input_* (runs in row order, quantile.metal.h:19-140),
 * sketch_summarize (:242-252), sketch_reduce_serial (:317-352), sketch_cuts. */
static void sk_feature(const float* X, uint32_t rows, uint32_t cols, uint32_t f, const float* weights,
                       uint32_t max_bin, float* cuts, uint32_t* count_out) {
  SkRun* runs = (SkRun*)malloc((size_t)(rows ? rows : 1) * sizeof(SkRun));
  uint32_t nonmissing = 0, elements = 0, nruns = 0;
  int have_prev = 0;
  float prev = 0;
  for (uint32_t r = 0; r < rows; ++r) {
    float v = X[(size_t)r * cols + f];
    if (isnan(v)) continue;
    ++nonmissing;
    float w = weights ? weights[r] : 1.0f;
    uint32_t wb;
    memcpy(&wb, &w, 4);
    if (!(wb & 0x7fffffffu)) continue;
    ++elements;
    if (have_prev && v == prev) {
      runs[nruns - 1].weight = weights ? runs[nruns - 1].weight + w : runs[nruns - 1].weight;
      runs[nruns - 1].order += weights ? 0u : 1u; /* unit weights: run length in `order` */
    } else {
      SkRun run = {v, w, weights ? nruns : 1u};
      runs[nruns++] = run;
    }
    prev = v;
    have_prev = 1;
  }
  if (!weights) {
    /* kernels/quantile.metal.h:137: a unit-weight run weighs min(length, 2^24). */
    for (uint32_t i = 0; i < nruns; ++i) {
      uint32_t length = runs[i].order;
      runs[i].weight = (float)(length < (1u << 24) ? length : (1u << 24));
      runs[i].order = i;
    }
  }
  uint32_t limit = oracle_sketch_budget(max_bin, nonmissing);
  uint32_t budget = oracle_sketch_budget(max_bin, elements);
  uint64_t capacity = 2ull * limit;
  uint32_t batches = nruns ? (uint32_t)((nruns + capacity - 1) / capacity) : 0;
  uint32_t levels = bit_width_u32(batches > 1 ? batches : 1) + 1;
  SkEntry* resident = (SkEntry*)calloc((size_t)limit * (levels + 1), sizeof(SkEntry));
  uint32_t counts[64] = {0};
  size_t work = 4 * (size_t)limit + capacity + 4;
  SkEntry* current = (SkEntry*)malloc(work * sizeof(SkEntry));
  SkEntry* scratch = (SkEntry*)malloc(work * sizeof(SkEntry));
  for (uint64_t begin = 0; begin < nruns; begin += capacity) {
    uint32_t size = (uint32_t)((nruns - begin) < capacity ? (nruns - begin) : capacity);
    uint32_t n = sk_summarize(runs + begin, size, limit, current);
    uint32_t level = 0;
    for (;;) {
      n = sk_prune(current, n, limit);
      n = sk_combine(current, n, resident + (size_t)level * limit, counts[level], scratch);
      counts[level] = 0;
      if (n <= limit) break;
      ++level;
    }
    counts[level] = n;
    memcpy(resident + (size_t)level * limit, current, (size_t)n * sizeof(SkEntry));
  }
  uint32_t n = 0;
  uint32_t cap = budget > limit ? budget : limit;
  for (uint32_t level = 0; level < levels; ++level) {
    n = sk_combine(current, n, resident + (size_t)level * limit, counts[level], scratch);
    n = sk_prune(current, n, cap);
  }
  n = sk_prune(current, n, budget);
  *count_out = sk_cuts(current, n, max_bin, cuts);
  free(runs);
  free(resident);
  free(current);
  free(scratch);
}

int oracle_sketch_cuts(const float* X, uint32_t rows, uint32_t cols, const float* weights, uint32_t max_bin,
                       float* cuts, uint32_t* counts, float* minima) {
  if (max_bin < 2) return -1;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t f = 0; f < (int64_t)cols; ++f) {
    float* out = cuts + (size_t)f * max_bin;
    for (uint32_t i = 0; i < max_bin; ++i) out[i] = 0;
    sk_feature(X, rows, cols, (uint32_t)f, weights, max_bin, out, &counts[f]);
    minima[f] = -INFINITY; /* kernels/quantile.metal.h:367 */
  }
  return 0;
}

/* kernels/boost.metal:476-499 (quantize): bin = min(#{cuts <= v}, count-1). */
void oracle_quantize(const float* X, uint32_t rows, uint32_t cols, const float* cuts, const uint32_t* counts,
                     uint32_t max_bin, uint16_t* bins) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < (int64_t)rows; ++r) {
    for (uint32_t f = 0; f < cols; ++f) {
      float v = X[(size_t)r * cols + f];
      uint32_t count = counts[f];
      const float* column = cuts + (size_t)f * max_bin;
      uint16_t bin = 0xFFFF;
      if (!isnan(v) && count) {
        uint32_t lo = 0, hi = count;
        while (lo < hi) {
          uint32_t mid = lo + (hi - lo) / 2;
          if (v >= column[mid]) lo = mid + 1;
          else hi = mid;
        }
        bin = (uint16_t)(lo < count - 1 ? lo : count - 1);
      }
      bins[(size_t)r * cols + f] = bin;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Gradients, base score and fixed-point quantization                       */
/* ------------------------------------------------------------------------ */

/* Upstream XGBoost's Sigmoid (src/common/math.h), which stock XGBoost's
 * binary:logistic gradient and prediction transform call:
 * expf(std::min(-x, 88.7f)) + 1 + 1e-16f, inverted; std::min keeps -x when it
 * is NaN.  The reference's gradient kernel omits the clamp
 * (kernels/boost.metal:50) and restates the clamped form elsewhere
 * (kernels/distributions.metal.h:250); they differ only for x < -88.7. */
float oracle_sigmoid(float x) {
  float neg = -x;
  float arg = 88.7f < neg ? 88.7f : neg;
  return 1.0f / (expf(arg) + 1.0f + 1e-16f);
}

/* binary:logistic's prediction transform over an array. */
void oracle_sigmoid_array(const float* in, float* out, uint64_t count) {
  for (uint64_t i = 0; i < count; ++i) out[i] = oracle_sigmoid(in[i]);
}

/* kernels/boost.metal:553-601 (gradients), objectives 0, 1 and 2. */
void oracle_gradients(int32_t objective, const float* margin, const float* labels, const float* weights,
                      uint32_t rows, float scale_pos_weight, float* grad, float* hess) {
  for (uint32_t r = 0; r < rows; ++r) {
    float pred = margin[r], label = labels[r];
    float weight = weights ? weights[r] : 1.0f;
    float g = pred - label, h = 1.0f;
    if (objective == ORACLE_OBJ_LOGISTIC || objective == ORACLE_OBJ_LOGITRAW) {
      float prob = oracle_sigmoid(pred);
      weight *= label == 1.0f ? scale_pos_weight : 1.0f;
      g = prob - label;
      h = fmaxf(prob * (1.0f - prob), 1.0e-16f);
    }
    grad[r] = g * weight;
    hess[r] = h * weight;
  }
}

/* src/learner.cpp:316-333 with kernels/boost.metal:356-423: the weighted label
 * mean in extended precision, rounded once to binary32.  Products of two
 * binary32 values are exact in binary64; the sum is compensated (Neumaier).
 * A logistic objective whose scale_pos_weight is not 1 takes each term as the
 * binary32 product y * w (the reweighted intercept, boost.metal:379-381). */
float oracle_base_score(int32_t objective, const float* labels, const float* weights, uint32_t rows,
                        float scale_pos_weight) {
  const int logistic = objective == ORACLE_OBJ_LOGISTIC || objective == ORACLE_OBJ_LOGITRAW;
  const int float_product = logistic && fabsf(scale_pos_weight - 1.0f) > 1.0e-6f;
  double s = 0, c = 0, ws = 0, wc = 0;
  for (uint32_t r = 0; r < rows; ++r) {
    float w = weights ? weights[r] : 1.0f;
    float y = labels[r];
    if (logistic) w *= y == 1 ? scale_pos_weight : 1;
    const float product = y * w;
    double term = float_product ? (double)product : (double)y * (double)w;
    double t = s + term;
    c += fabs(s) >= fabs(term) ? (s - t) + term : (term - t) + s;
    s = t;
    double tw = ws + (double)w;
    wc += fabs(ws) >= fabs((double)w) ? (ws - tw) + (double)w : ((double)w - tw) + ws;
    ws = tw;
  }
  double value = s + c, weight = ws + wc;
  if (!(weight > 0)) return objective == ORACLE_OBJ_SQUARED_ERROR && rows == 0 ? 0.0f : 0.5f;
  return (float)(value / weight);
}

/* src/objectives.cpp:17-31 (score_margins). */
float oracle_base_margin(int32_t objective, float base_score) {
  /* Only the logistic score maps to a margin; logitraw's score is its margin. */
  if (objective == ORACLE_OBJ_LOGISTIC) {
    float v = base_score < 1.0e-6f ? 1.0e-6f : (base_score > 1 - 1.0e-6f ? 1 - 1.0e-6f : base_score);
    return -logf(1.0f / v - 1.0f);
  }
  return base_score;
}

/* kernels/gradient_quantization.metal.h:4-67: exact sum of |value| in units
 * of 2^-149 (ten 32-bit limbs); scale = 2^(62 - max(0, bitlen - 149)). */
float oracle_gradient_scale(const float* values, uint32_t rows) {
  uint32_t limb[10] = {0};
  for (uint32_t r = 0; r < rows; ++r) {
    uint32_t bits;
    memcpy(&bits, &values[r], 4);
    bits &= 0x7fffffffu;
    uint32_t e = bits >> 23;
    uint64_t m = bits & 0x7fffffu;
    uint32_t shift = 0;
    if (e) { m |= 0x800000u; shift = e - 1; }
    uint32_t word = shift / 32;
    uint64_t v = m << (shift % 32);
    uint64_t carry = 0;
    for (uint32_t w = word; w < 10; ++w) {
      uint64_t add = (w == word ? (v & 0xffffffffu) : (w == word + 1 ? (v >> 32) : 0)) + carry;
      uint64_t sum = (uint64_t)limb[w] + add;
      limb[w] = (uint32_t)sum;
      carry = sum >> 32;
      if (!carry && w > word) break;
    }
  }
  int exponent = 0;
  for (int w = 9; w >= 0; --w) {
    if (limb[w]) {
      int bitlen = w * 32 + 32 - __builtin_clz(limb[w]);
      exponent = bitlen - 149 > 0 ? bitlen - 149 : 0;
      break;
    }
  }
  uint32_t sbits = (uint32_t)(62 - exponent + 127) << 23;
  float scale;
  memcpy(&scale, &sbits, 4);
  return scale;
}

/* kernels/boost.metal:605-616 (quantize_gradients). */
void oracle_quantize_gradients(const float* grad, const float* hess, uint32_t rows, float scale_g, float scale_h,
                               int64_t* qg, int64_t* qh) {
  for (uint32_t r = 0; r < rows; ++r) {
    qg[r] = (int64_t)rintf(grad[r] * scale_g);
    qh[r] = (int64_t)rintf(hess[r] * scale_h);
  }
}

/* ------------------------------------------------------------------------ */
/* Histograms                                                               */
/* ------------------------------------------------------------------------ */

/* kernels/boost.metal:700-733 (histogram): exact int64 sums modulo 2^64 per
 * (feature, bin); bin max_bin collects missing values. */
void oracle_histogram(const uint16_t* bins, uint32_t cols, uint32_t max_bin, const uint32_t* rows, uint32_t count,
                      const int64_t* qg, const int64_t* qh, int64_t* hist) {
  size_t stride = (size_t)(max_bin + 1) * 2;
  memset(hist, 0, (size_t)cols * stride * sizeof(int64_t));
  for (uint32_t i = 0; i < count; ++i) {
    uint32_t r = rows[i];
    for (uint32_t f = 0; f < cols; ++f) {
      uint32_t bin = bins[(size_t)r * cols + f];
      if (bin == 0xFFFF) bin = max_bin;
      uint64_t* h = (uint64_t*)(hist + f * stride + (size_t)bin * 2);
      h[0] += (uint64_t)qg[r];
      h[1] += (uint64_t)qh[r];
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Split scoring                                                            */
/* ------------------------------------------------------------------------ */

static int scale_exponent(float scale) { int e; frexpf(scale, &e); return e - 1; }
/* kernels/split_statistics.metal.h:107-119: RN64(integer) * 2^-k. */
static double stat_value(int64_t v, float scale) { return ldexp((double)v, -scale_exponent(scale)); }

/* kernels/scalar_gain.metal.h:56-82 and split_statistics.metal.h:124-140:
 * w = RN32(RN64(-ThresholdL1(G, alpha) / (H + lambda))), clamped. */
float oracle_weight(double G, double H, const OracleParams* p) {
  if (!(H > 0)) return 0.0f;
  double alpha = fabs((double)p->reg_alpha);
  double g = G;
  if (fabs(g) <= alpha) g = 0;
  else g = g + (g < 0 ? alpha : -alpha);
  double den = H + (double)p->reg_lambda;
  float w = (float)(-g / den);
  float limit = fabsf(p->max_delta_step);
  if (limit != 0 && fabsf(w) > limit) w = copysignf(limit, w);
  return w;
}

/* kernels/scalar_gain.metal.h:91-103: RN32(-(2G*w + (H+lambda)*RN32(w*w) + 2*alpha*|w|))
 * with the two products fused into binary64 multiply-adds when fma_contract. */
float oracle_gain(double G, double H, float w, const OracleParams* p) {
  if (!(H > 0)) return 0.0f;
  double wd = (double)w;
  double square = (double)(w * w);
  double quadratic = (H + (double)p->reg_lambda) * square;
  double alpha2 = (double)p->reg_alpha + (double)p->reg_alpha;
  double sum;
  if (p->fma_contract) {
    sum = fma(G + G, wd, quadratic);
    sum = fma(alpha2, fabs(wd), sum);
  } else {
    sum = (G + G) * wd + quadratic;
    sum = alpha2 * fabs(wd) + sum;
  }
  return (float)(-sum);
}

/* kernels/scalar_gain.metal.h:79-80, split_statistics.metal.h:35-36: the
 * weight clamped to the node's monotone bounds [lower, upper]. */
static float bounded_weight(double G, double H, const OracleParams* p, float lower, float upper) {
  float w = oracle_weight(G, H, p);
  if (w < lower) w = lower;
  if (upper < w) w = upper;
  return w;
}

static int valid_hessian(double H, float min_child_weight) {
  return H > 0 && H >= (double)fabsf(min_child_weight);
}

/* kernels/boost.metal:902-920 (consider_split): child weights clamped to
 * the node's bounds; a monotone feature rejects a split whose left weight is
 * above (increasing) or below (decreasing) its right weight. */
static void consider(OracleSplit* best, int64_t lg, int64_t lh, int64_t rg, int64_t rh, float sg, float sh,
                     float threshold, uint32_t default_left, int32_t feature, uint32_t bin, float parent_gain,
                     const OracleParams* p, int monotone, float lower, float upper) {
  double GL = stat_value(lg, sg), HL = stat_value(lh, sh);
  double GR = stat_value(rg, sg), HR = stat_value(rh, sh);
  if (!valid_hessian(HL, p->min_child_weight) || !valid_hessian(HR, p->min_child_weight)) return;
  float lw = bounded_weight(GL, HL, p, lower, upper), rw = bounded_weight(GR, HR, p, lower, upper);
  if ((monotone > 0 && !(lw <= rw)) || (monotone < 0 && !(lw >= rw))) return;
  float gain = (oracle_gain(GL, HL, lw, p) + oracle_gain(GR, HR, rw, p)) - parent_gain;
  if (gain > best->gain) {
    best->gain = gain;
    best->threshold = threshold;
    best->feature = feature;
    best->default_left = default_left;
    best->bin = bin;
    best->left_h = (float)HL;
    best->right_h = (float)HR;
    best->left_weight = lw;
    best->right_weight = rw;
    best->left_g = lg; best->left_hs = lh;
    best->right_g = rg; best->right_hs = rh;
  }
}

/* kernels/boost.metal:921-1005 (evaluate_feature), numeric features:
 * forward scan (missing right), then backward scan when missing != 0; the
 * node's weight and every child weight clamped to [lower, upper]. */
static void evaluate_feature(const int64_t* fh, uint32_t count, const float* cuts, float minimum, int64_t total_g,
                             int64_t total_h, float scale_g, float scale_h, const OracleParams* p, int32_t feature,
                             int monotone, float lower, float upper, OracleSplit* out) {
  uint64_t pg = 0, ph = 0;
  for (uint32_t b = 0; b < count; ++b) { pg += (uint64_t)fh[2 * b]; ph += (uint64_t)fh[2 * b + 1]; }
  int64_t miss_g = (int64_t)((uint64_t)total_g - pg), miss_h = (int64_t)((uint64_t)total_h - ph);
  double G = stat_value(total_g, scale_g), H = stat_value(total_h, scale_h);
  float w = bounded_weight(G, H, p, lower, upper);
  OracleSplit best;
  memset(&best, 0, sizeof(best));
  best.gain = -INFINITY;
  best.feature = -1;
  best.left_weight = best.right_weight = w;
  best.total_g = (float)G;
  best.total_h = (float)H;
  best.parent_weight = w;
  float parent_gain = oracle_gain(G, H, w, p);
  uint64_t lg = 0, lh = 0;
  for (uint32_t b = 0; b < count; ++b) {
    lg += (uint64_t)fh[2 * b];
    lh += (uint64_t)fh[2 * b + 1];
    consider(&best, (int64_t)lg, (int64_t)lh, (int64_t)((uint64_t)total_g - lg), (int64_t)((uint64_t)total_h - lh),
             scale_g, scale_h, cuts[b], 0, feature, b, parent_gain, p, monotone, lower, upper);
  }
  if (miss_g != 0 || miss_h != 0) {
    uint64_t rg = 0, rh = 0;
    for (int64_t b = (int64_t)count - 1; b >= 0; --b) {
      rg += (uint64_t)fh[2 * b];
      rh += (uint64_t)fh[2 * b + 1];
      float threshold = b == 0 ? minimum : cuts[b - 1];
      consider(&best, (int64_t)((uint64_t)total_g - rg), (int64_t)((uint64_t)total_h - rh), (int64_t)rg, (int64_t)rh,
               scale_g, scale_h, threshold, 1, feature, (uint32_t)b, parent_gain, p, monotone, lower, upper);
    }
  }
  *out = best;
}

void oracle_evaluate_feature(const int64_t* fh, uint32_t count, const float* cuts, float minimum, int64_t total_g,
                             int64_t total_h, float scale_g, float scale_h, const OracleParams* p, int32_t feature,
                             OracleSplit* out) {
  evaluate_feature(fh, count, cuts, minimum, total_g, total_h, scale_g, scale_h, p, feature, 0, -FLT_MAX, FLT_MAX,
                   out);
}

/* ------------------------------------------------------------------------ */
/* Depthwise tree growth                                                    */
/* ------------------------------------------------------------------------ */

uint32_t oracle_max_nodes(int32_t max_depth) { return (2u << (uint32_t)max_depth) - 1u; }

typedef struct {
  uint32_t id, begin, count;
  int64_t sum_g, sum_h;
  float lower, upper;  /* monotone bounds of the node's weight (src/tree.cpp:1083-1086) */
} Frontier;

typedef struct {
  const uint16_t* bins;      /* row-major */
  const uint16_t* bins_cm;   /* feature-major copy for the histogram loop */
  uint32_t rows, cols, max_bin;
  const float* cuts;
  const uint32_t* counts;
  const float* minima;
  int dense;
} Quantized;

/* Histogram of one node, parallel over features (results are exact integers
 * and independent of the thread count).  The node's fixed-point pairs are
 * gathered once into `pairs` (2 x count words) in row-list order, so each
 * feature reads them in sequence. */
static void node_histogram(const Quantized* q, const uint32_t* rows, uint32_t count, const int64_t* qg,
                           const int64_t* qh, int64_t* pairs, int64_t* hist) {
  size_t stride = (size_t)(q->max_bin + 1) * 2;
#pragma omp parallel
  {
#pragma omp for schedule(static)
    for (int64_t i = 0; i < (int64_t)count; ++i) {
      pairs[2 * i] = qg[rows[i]];
      pairs[2 * i + 1] = qh[rows[i]];
    }
#pragma omp for schedule(dynamic, 1)
    for (int64_t f = 0; f < (int64_t)q->cols; ++f) {
      uint64_t* h = (uint64_t*)(hist + (size_t)f * stride);
      memset(h, 0, stride * sizeof(int64_t));
      const uint16_t* column = q->bins_cm + (size_t)f * q->rows;
      for (uint32_t i = 0; i < count; ++i) {
        uint32_t bin = column[rows[i]];
        if (bin == 0xFFFF) bin = q->max_bin;
        h[2 * bin] += (uint64_t)pairs[2 * i];
        h[2 * bin + 1] += (uint64_t)pairs[2 * i + 1];
      }
    }
  }
}

/* Ordered binary64 sum of a bin range (kernels/scalar_root.metal.h:1-105). */
static void ordered_sum(const int64_t* fh, uint32_t first, uint32_t steps, int reverse, uint32_t count,
                        float sg, float sh, double* g, double* h) {
  double a = 0, b = 0;
  for (uint32_t s = 0; s < steps; ++s) {
    uint32_t bin = reverse ? count - s - 1 : first + s;
    a += stat_value(fh[2 * bin], sg);
    b += stat_value(fh[2 * bin + 1], sh);
  }
  *g = a;
  *h = b;
}

/* One tree: src/tree.cpp:291-349 (host driver), :1031-1104 (pop/apply),
 * :1663-1717 (replay), kernels/scalar_root.metal.h:107-186 (dense root),
 * kernels/boost.metal:1245-1265 (select_splits). */
static uint32_t grow_tree(const Quantized* q, const OracleParams* p, const int64_t* qg, const int64_t* qh,
                          float sg, float sh, uint32_t* row_buf, uint32_t* tmp_buf, int64_t* hist,
                          OracleNode* nodes, const uint8_t* allowed, uint32_t* leaf_of_row) {
  uint32_t max_nodes = oracle_max_nodes(p->max_depth);
  size_t stride = (size_t)(q->max_bin + 1) * 2;
  for (uint32_t i = 0; i < max_nodes; ++i) {
    OracleNode n = {-1, -1, -1, -1, 0, 0, 0, 0, 0, 0};
    nodes[i] = n;
  }
  uint32_t node_count = 1;
  for (uint32_t r = 0; r < q->rows; ++r) row_buf[r] = r;
  Frontier* frontier = (Frontier*)malloc(sizeof(Frontier) * (max_nodes + 1));
  Frontier* next = (Frontier*)malloc(sizeof(Frontier) * (max_nodes + 1));
  OracleSplit* cands = (OracleSplit*)malloc(sizeof(OracleSplit) * (q->cols ? q->cols : 1));
  int64_t* pairs = (int64_t*)malloc(sizeof(int64_t) * 2 * (q->rows ? q->rows : 1));
  uint32_t nf = 1;
  frontier[0].id = 0; frontier[0].begin = 0; frontier[0].count = q->rows;
  frontier[0].sum_g = frontier[0].sum_h = 0;
  frontier[0].lower = -FLT_MAX;  /* kernels/tree_sample_columns.metal.h tree_init_bounds */
  frontier[0].upper = FLT_MAX;
  for (int32_t depth = 0; nf > 0; ++depth) {
    uint32_t nn = 0;
    for (uint32_t k = 0; k < nf; ++k) {
      Frontier* fr = &frontier[k];
      uint32_t id = fr->id;
      if (depth >= p->max_depth) {
        for (uint32_t i = 0; i < fr->count; ++i) leaf_of_row[row_buf[fr->begin + i]] = id;
        continue;
      }
      node_histogram(q, row_buf + fr->begin, fr->count, qg, qh, pairs, hist);
      int64_t total_g = fr->sum_g, total_h = fr->sum_h;
      if (depth == 0) {
        /* Root: present + missing of feature 0 (equal for every feature). */
        uint64_t a = 0, b = 0;
        for (uint32_t bin = 0; bin <= q->max_bin; ++bin) { a += (uint64_t)hist[2 * bin]; b += (uint64_t)hist[2 * bin + 1]; }
        total_g = (int64_t)a; total_h = (int64_t)b;
      }
      /* Every feature's best candidate (in parallel: each is a function of
       * its own histogram row), then the first strictly greater gain in
       * feature order. */
#pragma omp parallel for schedule(dynamic, 1)
      for (int64_t f = 0; f < (int64_t)q->cols; ++f) {
        evaluate_feature(hist + (size_t)f * stride, q->counts[f], q->cuts + (size_t)f * q->max_bin, q->minima[f],
                         total_g, total_h, sg, sh, p, (int32_t)f, p->monotone ? p->monotone[f] : 0, fr->lower,
                         fr->upper, &cands[f]);
        if (allowed && !allowed[f]) {
          /* A feature outside the tree's sample offers no split. */
          cands[f].gain = -INFINITY;
          cands[f].feature = -1;
        }
      }
      OracleSplit best;
      memset(&best, 0, sizeof(best));
      for (uint32_t f = 0; f < q->cols; ++f)
        if (f == 0 || cands[f].gain > best.gain) best = cands[f];
      float applied_weight = 0, applied_hessian = 0;
      float parent_weight = best.parent_weight, total_h_f = best.total_h;
      if (depth == 0 && q->dense) {
        uint32_t c0 = q->counts[0];
        double tg, th;
        ordered_sum(hist, 0, c0, 0, c0, sg, sh, &tg, &th);
        parent_weight = bounded_weight(tg, th, p, fr->lower, fr->upper);
        total_h_f = (float)th;
        if (best.feature >= 0) {
          uint32_t f = (uint32_t)best.feature, count = q->counts[f];
          const float* column = q->cuts + (size_t)f * q->max_bin;
          uint32_t lo = 0, hi = count;
          while (lo < hi) {
            uint32_t mid = lo + (hi - lo) / 2;
            if (column[mid] < best.threshold) lo = mid + 1;
            else hi = mid;
          }
          uint32_t steps = lo + 1;
          if (best.default_left) {
            uint32_t bin = best.threshold == q->minima[f] ? 0 : lo + 1;
            steps = count - bin;
          }
          double cg, ch;
          ordered_sum(hist + (size_t)f * stride, 0, steps, (int)best.default_left, count, sg, sh, &cg, &ch);
          double og = tg - cg, oh = th - ch;
          double ag = cg + og, ah = ch + oh;
          applied_weight = bounded_weight(ag, ah, p, fr->lower, fr->upper);
          applied_hessian = (float)ah;
        }
      } else if (best.feature >= 0) {
        double ag = stat_value(best.left_g, sg) + stat_value(best.right_g, sg);
        double ah = stat_value(best.left_hs, sh) + stat_value(best.right_hs, sh);
        applied_weight = bounded_weight(ag, ah, p, fr->lower, fr->upper);
        applied_hessian = (float)ah;
      }
      OracleNode* node = &nodes[id];
      node->cover = total_h_f;
      if (id == 0) {
        node->base_weight = parent_weight;
        node->leaf = parent_weight * p->eta;
      }
      int expand = best.feature >= 0 && best.gain > 1.0e-6f && best.gain >= p->min_split_loss && depth < p->max_depth;
      if (!expand) {
        for (uint32_t i = 0; i < fr->count; ++i) leaf_of_row[row_buf[fr->begin + i]] = id;
        continue;
      }
      uint32_t left = node_count, right = left + 1;
      node_count += 2;
      node->left = (int32_t)left;
      node->right = (int32_t)right;
      node->feature = best.feature;
      node->threshold = best.threshold;
      node->default_left = best.default_left;
      node->gain = best.gain;
      node->base_weight = applied_weight;
      node->cover = applied_hessian;
      OracleNode l = {-1, -1, (int32_t)id, -1, 0, best.left_weight * p->eta, best.left_h, 0, 0, 0};
      OracleNode r = {-1, -1, (int32_t)id, -1, 0, best.right_weight * p->eta, best.right_h, 0, 0, 0};
      l.base_weight = l.leaf;
      r.base_weight = r.leaf;
      nodes[left] = l;
      nodes[right] = r;
      /* Stable partition: value < threshold <=> bin <= b (forward) or
       * bin <= b-1 (backward); missing follows default_left. */
      uint32_t f = (uint32_t)best.feature;
      int64_t last_left_bin = best.default_left ? (int64_t)best.bin - 1 : (int64_t)best.bin;
      const uint16_t* column = q->bins_cm + (size_t)f * q->rows;
      uint32_t nl = 0, nr = 0;
      for (uint32_t i = 0; i < fr->count; ++i) {
        uint32_t row = row_buf[fr->begin + i];
        uint32_t bin = column[row];
        int go_left = bin == 0xFFFF ? (int)best.default_left : (int64_t)bin <= last_left_bin;
        if (go_left) row_buf[fr->begin + nl++] = row;
        else tmp_buf[nr++] = row;
      }
      memcpy(row_buf + fr->begin + nl, tmp_buf, (size_t)nr * sizeof(uint32_t));
      /* Children's bounds (src/tree.cpp:1083-1086): the midpoint of the two
       * child weights caps the left child from above and the right from below
       * (increasing), or the reverse (decreasing); std::min/std::max order. */
      Frontier a = {left, fr->begin, nl, best.left_g, best.left_hs, fr->lower, fr->upper};
      Frontier b = {right, fr->begin + nl, nr, best.right_g, best.right_hs, fr->lower, fr->upper};
      int mono = p->monotone ? p->monotone[f] : 0;
      float middle = (best.left_weight + best.right_weight) * 0.5f;
      if (mono > 0) {
        if (middle < a.upper) a.upper = middle;
        if (b.lower < middle) b.lower = middle;
      } else if (mono < 0) {
        if (a.lower < middle) a.lower = middle;
        if (middle < b.upper) b.upper = middle;
      }
      next[nn++] = a;
      next[nn++] = b;
    }
    Frontier* t = frontier;
    frontier = next;
    next = t;
    nf = nn;
  }
  free(frontier);
  free(next);
  free(cands);
  free(pairs);
  return node_count;
}

/* ---------------------------------------------------------------------------
 * Sampling.
 * MT19937: the published generator (Matsumoto and Nishimura, ACM TOMACS 8(1),
 * 1998) with the C++ standard's seeding (std::mersenne_twister_engine::seed:
 * x[i] = 1812433253 (x[i-1] ^ (x[i-1] >> 30)) + i) -- block twist of all
 * 624 words, then tempering.  The standard fixes the 10000th output of a
 * default-seeded (5489) engine at 4123659995.
 * ------------------------------------------------------------------------- */
void oracle_mt_seed(OracleMT* g, uint32_t seed) {
  g->state[0] = seed;
  for (uint32_t i = 1; i < 624; ++i) g->state[i] = 1812433253u * (g->state[i - 1] ^ (g->state[i - 1] >> 30)) + i;
  g->next = 624;
}

uint32_t oracle_mt_next(OracleMT* g) {
  if (g->next >= 624) {
    for (uint32_t i = 0; i < 624; ++i) {
      uint32_t y = (g->state[i] & 0x80000000u) | (g->state[(i + 1) % 624] & 0x7fffffffu);
      g->state[i] = g->state[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
    }
    g->next = 0;
  }
  uint32_t y = g->state[g->next++];
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

/* kernels/sampling.metal.h:1-30: the row's engine state is the round seed
 * times 16807^(row+1) modulo 2^63 (a multiplicative generator stepped row+1
 * times); the row is kept when the canonical binary64 draw
 * RN53(state - 1) / 2^63 (libc++ bernoulli_distribution over a 63-bit engine)
 * is below subsample.  For subsample < 2^-39 the comparison is made in
 * binary32, as the reference does. */
int oracle_sample_row(uint32_t seed, uint32_t row, float subsample) {
  const uint64_t mask = 0x7fffffffffffffffull;
  uint64_t state = seed ? seed : 1u, factor = 16807u;
  for (uint64_t e = (uint64_t)row + 1; e; e >>= 1) {
    if (e & 1) state = (state * factor) & mask;
    factor = (factor * factor) & mask;
  }
  uint64_t numerator = state - 1;
  /* Round to 53 significant bits, ties to even (the int -> binary64 conversion). */
  double rounded = (double)numerator;
  float limit = subsample * 0x1p63f;
  if (limit < 0x1p24f) return (float)rounded < limit;
  return rounded < (double)limit;
}

/* Uniform integer in [0, range), 2 <= range <= 2^32, as libstdc++'s
 * std::uniform_int_distribution draws it from a 32-bit engine (GCC 11 and
 * later): Lemire's multiply-shift with rejection ("Fast Random Integer
 * Generation in an Interval", ACM TOMACS 29(1), 2019). */
static uint32_t uniform_libstdcxx(OracleMT* g, uint64_t range) {
  uint32_t r32 = (uint32_t)range;
  uint64_t product = (uint64_t)oracle_mt_next(g) * r32;
  uint32_t low = (uint32_t)product;
  if (low < r32) {
    uint32_t threshold = (uint32_t)(0u - r32) % r32;
    while (low < threshold) {
      product = (uint64_t)oracle_mt_next(g) * r32;
      low = (uint32_t)product;
    }
  }
  return (uint32_t)(product >> 32);
}

static void swap_u32(uint32_t* v, uint64_t a, uint64_t b) {
  uint32_t t = v[a];
  v[a] = v[b];
  v[b] = t;
}

/* std::shuffle(v, v + n, mt19937) of either standard library.
 * libstdc++ (model 0; x86-64 Linux, stock XGBoost's wheels): position i from
 * 1 upwards swaps with a uniform position in [0, i]; while n^2 < 2^32 the
 * draws are paired: an even n first swaps position 1 with a draw over
 * {0, 1}, then positions i, i + 1 share one draw x over [0, (i+1)(i+2)) and
 * swap with x / (i+2) and x % (i+2).
 * libc++ (model 1; the reference's macOS builds): position pos from 0
 * swaps with pos + u, u uniform in [0, n - pos) from one engine output masked
 * to the bit width of n - pos - 1, values >= n - pos rejected. */
void oracle_std_shuffle(uint32_t* v, uint32_t n, OracleMT* g, int32_t model) {
  if (n < 2) return;
  if (model == 1) {
    for (uint32_t pos = 0; pos + 1 < n; ++pos) {
      uint32_t range = n - pos;
      uint32_t width = 32u - (uint32_t)__builtin_clz(range - 1u);
      uint32_t mask = width >= 32 ? 0xffffffffu : (1u << width) - 1u;
      uint32_t u;
      do u = oracle_mt_next(g) & mask; while (u >= range);
      swap_u32(v, pos, pos + u);
    }
    return;
  }
  if (0xffffffffull / n >= n) {
    uint64_t i = 1;
    if (n % 2 == 0) {
      swap_u32(v, 1, uniform_libstdcxx(g, 2));
      i = 2;
    }
    for (; i < n; i += 2) {
      uint64_t b1 = i + 2;
      uint32_t x = uniform_libstdcxx(g, (i + 1) * b1);
      swap_u32(v, i, x / b1);
      swap_u32(v, i + 1, x % b1);
    }
    return;
  }
  for (uint64_t i = 1; i < n; ++i) swap_u32(v, i, uniform_libstdcxx(g, i + 1));
}

/* src/tree.cpp:28-45: a fresh engine seeded with `seed` shuffles the n
 * features (std::shuffle of the given model); the first
 * max(1, floor(n * fraction)) (binary32 product) are kept, sorted. */
uint32_t oracle_sample_columns(uint32_t n, float fraction, uint32_t seed, int32_t model, uint32_t* out) {
  for (uint32_t i = 0; i < n; ++i) out[i] = i;
  if (!(fraction < 1.0f) || n == 0) return n;
  float scaled = floorf((float)n * fraction);
  uint32_t keep = scaled < 1.0f ? 1u : (uint32_t)scaled;
  if (keep > n) keep = n;
  OracleMT g;
  oracle_mt_seed(&g, seed);
  oracle_std_shuffle(out, n, &g, model);
  /* Sort the kept prefix (insertion sort; n is a feature count). */
  for (uint32_t i = 1; i < keep; ++i) {
    uint32_t v = out[i], j = i;
    while (j > 0 && out[j - 1] > v) { out[j] = out[j - 1]; --j; }
    out[j] = v;
  }
  return keep;
}

static int has_nan(const float* X, size_t n) {
  for (size_t i = 0; i < n; ++i) if (isnan(X[i])) return 1;
  return 0;
}

int oracle_train(const float* X, uint32_t rows, uint32_t cols, const float* labels, const float* weights,
                 const OracleParams* p, uint32_t rounds, const float* custom_grad, const float* custom_hess,
                 OracleNode* trees, uint32_t* tree_sizes, float* margin, float* base_score_out, float* cuts_out,
                 uint32_t* cut_counts_out) {
  if (p->max_bin < 2 || p->max_depth < 0 || p->max_depth > 20 || cols == 0) return -1;
#ifdef _OPENMP
  if (p->nthread > 0) omp_set_num_threads(p->nthread);
#endif
  uint32_t max_bin = (uint32_t)p->max_bin;
  uint32_t hist_bins = rows < max_bin ? (rows ? rows : 1) : max_bin; /* src/data.cpp:1231 */
  float* cuts = (float*)calloc((size_t)cols * hist_bins, sizeof(float));
  uint32_t* counts = (uint32_t*)calloc(cols, sizeof(uint32_t));
  float* minima = (float*)calloc(cols, sizeof(float));
  /* The sketch writes up to max_bin cuts; histogram_bins caps them. */
  float* cuts_full = (float*)calloc((size_t)cols * max_bin, sizeof(float));
  oracle_sketch_cuts(X, rows, cols, weights, max_bin, cuts_full, counts, minima);
  for (uint32_t f = 0; f < cols; ++f)
    memcpy(cuts + (size_t)f * hist_bins, cuts_full + (size_t)f * max_bin,
           (size_t)(counts[f] < hist_bins ? counts[f] : hist_bins) * sizeof(float));
  if (cuts_out) memcpy(cuts_out, cuts_full, (size_t)cols * max_bin * sizeof(float));
  if (cut_counts_out) memcpy(cut_counts_out, counts, cols * sizeof(uint32_t));
  free(cuts_full);
  uint16_t* bins = (uint16_t*)malloc((size_t)rows * cols * sizeof(uint16_t));
  oracle_quantize(X, rows, cols, cuts, counts, hist_bins, bins);
  uint16_t* bins_cm = (uint16_t*)malloc((size_t)rows * cols * sizeof(uint16_t));
  for (uint32_t r = 0; r < rows; ++r)
    for (uint32_t f = 0; f < cols; ++f) bins_cm[(size_t)f * rows + r] = bins[(size_t)r * cols + f];
  Quantized q = {bins, bins_cm, rows, cols, hist_bins, cuts, counts, minima, !has_nan(X, (size_t)rows * cols)};

  float base_score = p->has_base_score ? p->base_score
                                       : oracle_base_score(p->objective, labels, weights, rows, p->scale_pos_weight);
  if (!p->has_base_score && p->objective == ORACLE_OBJ_LOGITRAW) {
    /* logitraw's default score is the logit of the clamped label mean
     * (kernels/boost.metal:405-423 base_finalize). */
    const float v = base_score < 1.0e-6f ? 1.0e-6f : (base_score > 1 - 1.0e-6f ? 1 - 1.0e-6f : base_score);
    base_score = logf(v / (1 - v));
  }
  if (base_score_out) *base_score_out = base_score;
  float base_margin = oracle_base_margin(p->objective, base_score);
  for (uint32_t r = 0; r < rows; ++r) margin[r] = base_margin;

  float* grad = (float*)malloc((size_t)rows * sizeof(float) + 4);
  float* hess = (float*)malloc((size_t)rows * sizeof(float) + 4);
  int64_t* qg = (int64_t*)malloc((size_t)rows * sizeof(int64_t) + 8);
  int64_t* qh = (int64_t*)malloc((size_t)rows * sizeof(int64_t) + 8);
  uint32_t* row_buf = (uint32_t*)malloc((size_t)rows * sizeof(uint32_t) + 4);
  uint32_t* tmp_buf = (uint32_t*)malloc((size_t)rows * sizeof(uint32_t) + 4);
  uint32_t* leaf_of_row = (uint32_t*)malloc((size_t)rows * sizeof(uint32_t) + 4);
  int64_t* hist = (int64_t*)malloc((size_t)cols * (hist_bins + 1) * 2 * sizeof(int64_t));
  uint32_t max_nodes = oracle_max_nodes(p->max_depth);
  /* The learner's engine: default state (seed 5489) unless a nonzero seed
   * parameter reseeds it (src/learner.cpp:94-103). */
  OracleMT rng;
  oracle_mt_seed(&rng, p->seed ? p->seed : 5489u);
  /* Row sampling runs when floor(float(rows) * subsample) < rows (src/learner.cpp:679). */
  double subsample = p->subsample > 0 ? (double)p->subsample : 1.0;
  int sampling = (uint64_t)((double)(float)rows * subsample) < (uint64_t)rows;
  int colsample = p->colsample_bytree > 0 && p->colsample_bytree < 1.0f;
  uint8_t* allowed = colsample ? (uint8_t*)malloc(cols) : NULL;
  uint32_t* features = colsample ? (uint32_t*)malloc((size_t)cols * sizeof(uint32_t)) : NULL;
  for (uint32_t t = 0; t < rounds; ++t) {
    /* src/learner.cpp:668: seed_per_iteration reseeds with the round count. */
    if (p->seed_per_iteration) oracle_mt_seed(&rng, p->seed * 127u + t);
    if (custom_grad) {
      memcpy(grad, custom_grad + (size_t)t * rows, (size_t)rows * sizeof(float));
      memcpy(hess, custom_hess + (size_t)t * rows, (size_t)rows * sizeof(float));
    } else {
      oracle_gradients(p->objective, margin, labels, weights, rows, p->scale_pos_weight, grad, hess);
    }
    if (sampling) {
      /* src/sampling.cpp:11-74: one engine draw seeds the round; dropped rows
       * carry a zero gradient pair (and so add nothing to any histogram). */
      uint32_t seed = oracle_mt_next(&rng);
      for (uint32_t r = 0; r < rows; ++r)
        if (!oracle_sample_row(seed, r, p->subsample)) grad[r] = hess[r] = 0.0f;
    }
    if (colsample) {
      uint32_t keep = oracle_sample_columns(cols, p->colsample_bytree, oracle_mt_next(&rng), p->std_shuffle, features);
      memset(allowed, 0, cols);
      for (uint32_t i = 0; i < keep; ++i) allowed[features[i]] = 1;
    }
    float sg = oracle_gradient_scale(grad, rows), sh = oracle_gradient_scale(hess, rows);
    oracle_quantize_gradients(grad, hess, rows, sg, sh, qg, qh);
    OracleNode* nodes = trees + (size_t)t * max_nodes;
    tree_sizes[t] = grow_tree(&q, p, qg, qh, sg, sh, row_buf, tmp_buf, hist, nodes, allowed, leaf_of_row);
    /* Prediction-cache update: kernels/boost.metal:1738-1763, one float add per row. */
    for (uint32_t r = 0; r < rows; ++r) margin[r] = margin[r] + nodes[leaf_of_row[r]].leaf;
  }
  free(allowed); free(features);
  free(grad); free(hess); free(qg); free(qh); free(row_buf); free(tmp_buf); free(leaf_of_row); free(hist);
  free(bins); free(bins_cm); free(cuts); free(counts); free(minima);
  return 0;
}

/* kernels/boost.metal:1325-1329 (split_left) and :1738-1763 (predict). */
void oracle_predict_margin(const float* X, uint32_t rows, uint32_t cols, const OracleNode* trees,
                           const uint32_t* tree_sizes, uint32_t rounds, uint32_t stride, float base_margin,
                           float* out) {
  for (uint32_t r = 0; r < rows; ++r) {
    float sum = base_margin;
    const float* row = X + (size_t)r * cols;
    for (uint32_t t = 0; t < rounds; ++t) {
      const OracleNode* nodes = trees + (size_t)t * stride;
      uint32_t id = 0;
      (void)tree_sizes;
      while (nodes[id].left >= 0) {
        float v = row[nodes[id].feature];
        int left = isnan(v) ? (int)nodes[id].default_left : v < nodes[id].threshold;
        id = (uint32_t)(left ? nodes[id].left : nodes[id].right);
      }
      sum = sum + nodes[id].leaf;
    }
    out[r] = sum;
  }
}

/* ---- evaluation metrics ------------------------------------------------- */
/* kernels/boost.metal:51: log(1 + x) with the rounding of 1 + x compensated. */
static float log1p_compensated(float x) {
  float y = 1.0f + x;
  return y == 1.0f ? x : logf(y) * x / (y - 1.0f);
}

/* kernels/boost.metal:2245-2264 (per-row loss). */
static float metric_loss(uint32_t kind, float pred, float label, float parameter) {
  switch (kind) {
    case 0: { float d = pred - label; return d * d; }
    case 1: return fabsf(pred - label);
    case 2: { float d = log1p_compensated(pred) - log1p_compensated(label); return d * d; }
    case 3: return -label * logf(fmaxf(pred, 1.0e-16f)) - (1.0f - label) * logf(fmaxf(1.0f - pred, 1.0e-16f));
    case 6: return pred > parameter ? 1.0f - label : label;
    case 7: return fabsf((pred - label) / label);
    case 8: { float z = (pred - label) / parameter; return parameter * parameter * (sqrtf(1.0f + z * z) - 1.0f); }
    case 9: return lgammaf(label + 1.0f) + pred - label * logf(fmaxf(pred, 1.0e-16f));
    case 10: { float r = label / pred; return 2.0f * (-logf(r) + r - 1.0f); }
    case 11:
      return -label * powf(pred, 1.0f - parameter) / (1.0f - parameter) +
             powf(pred, 2.0f - parameter) / (2.0f - parameter);
    case 12: return label / pred + logf(pred);
  }
  return 0.0f;
}

/* The threadgroup tree of kernels/boost.metal:2267-2272 / 2286-2290:
 * v[t] += v[t + d] for d = 128 .. 1 over 256 pairs; the result is v[0]. */
static void tree256(float* gx, float* gy) {
  for (uint32_t d = 128; d; d >>= 1)
    for (uint32_t t = 0; t < d; ++t) {
      gx[t] = gx[t] + gx[t + d];
      gy[t] = gy[t] + gy[t + d];
    }
}

void oracle_metric_sum(const float* pred, const float* labels, const float* weights, uint32_t rows, uint32_t kind,
                       float parameter, float out[2]) {
  const uint32_t blocks = (uint32_t)(((uint64_t)rows + 255) / 256);
  float* px = (float*)calloc(blocks ? blocks : 1, sizeof(float));
  float* py = (float*)calloc(blocks ? blocks : 1, sizeof(float));
  float vx[256], vy[256];
  /* metric_partial (:2225-2275): one 256-row block per workgroup. */
  for (uint32_t b = 0; b < blocks; ++b) {
    for (uint32_t t = 0; t < 256; ++t) {
      uint64_t i = (uint64_t)b * 256 + t;
      vx[t] = vy[t] = 0.0f;
      if (i < rows) {
        float w = weights ? weights[i] : 1.0f;
        vx[t] = w * metric_loss(kind, pred[i], labels[i], parameter);
        vy[t] = w;
      }
    }
    tree256(vx, vy);
    px[b] = vx[0];
    py[b] = vy[0];
  }
  /* metric_reduce (:2276-2295): thread t sums blocks t, t + 256, ... with
   * compensation, then the tree. */
  for (uint32_t t = 0; t < 256; ++t) {
    float sx = 0.0f, sy = 0.0f, cx = 0.0f, cy = 0.0f;
    for (uint32_t i = t; i < blocks; i += 256) {
      float yx = px[i] - cx, yy = py[i] - cy;
      float nx = sx + yx, ny = sy + yy;
      cx = (nx - sx) - yx;
      cy = (ny - sy) - yy;
      sx = nx;
      sy = ny;
    }
    vx[t] = sx;
    vy[t] = sy;
  }
  tree256(vx, vy);
  out[0] = vx[0];
  out[1] = vy[0];
  free(px);
  free(py);
}

/* Descending prediction order as ascending uint32 keys; +0 and -0 tie
 * (kernels/radix_sort.metal.h:20-23). */
static uint32_t descending_key(float p) {
  uint32_t b;
  memcpy(&b, &p, 4);
  if ((b & 0x7fffffffu) == 0) b = 0;
  uint32_t ascending = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ~ascending;
}

typedef struct {
  uint32_t key, row;
} KeyRow;

static int key_row_cmp(const void* a, const void* b) {
  const KeyRow *x = (const KeyRow*)a, *y = (const KeyRow*)b;
  if (x->key != y->key) return x->key < y->key ? -1 : 1;
  return x->row < y->row ? -1 : (x->row > y->row);
}

/* 1 - log(1 + u) / u for 0 < u <= 1/4 by its alternating series. */
static double one_minus_log1p_ratio(double u) {
  double term = u, sum = 0.0;
  for (int k = 1; k <= 40; ++k) {
    double add = term / (double)(k + 1);
    sum = (k & 1) ? sum + add : sum - add;
    term *= u;
  }
  return sum;
}

/* kernels/radix_sort.metal.h:354-398 (auc_pr_segment_d64): precision
 * integrated over the recall rise of one step, precision linear in (TP, FP)
 * between the step's end points. */
static double pr_step_area(double prev_tp, double prev_fp, double tp, double fp, double positives) {
  if (tp == 0.0 || positives == 0.0) return 0.0;
  double mass = tp + fp;
  if (mass == 0.0) return 0.0;
  double rise = tp / positives, q = tp / mass;
  double cumulative = prev_tp + prev_fp;
  if (cumulative == 0.0) return rise * q;
  double r = prev_tp / cumulative, retained, added;
  if (mass <= cumulative) {
    double u = mass / cumulative;
    if (u <= 0.25) {
      added = one_minus_log1p_ratio(u);
      retained = 1.0 - added;
    } else {
      retained = log1p(u) / u;
      added = 1.0 - retained;
    }
  } else {
    double v = cumulative / mass;
    retained = v == 0.0 ? 0.0 : v * (log1p(v) - log(v));
    added = 1.0 - retained;
  }
  return rise * (r * retained + q * added);
}

void oracle_metric_auc(const float* pred, const float* labels, const float* weights, uint32_t rows, int pr,
                       double out[3]) {
  out[0] = out[1] = out[2] = 0.0;
  if (!rows) return;
  KeyRow* order = (KeyRow*)malloc(sizeof(KeyRow) * rows);
  double positives = 0.0, negatives = 0.0;
  for (uint32_t r = 0; r < rows; ++r) {
    order[r].key = descending_key(pred[r]);
    order[r].row = r;
    float w = weights ? weights[r] : 1.0f;
    positives += (double)fabsf(labels[r] * w);
    negatives += (double)fabsf((1.0f - labels[r]) * w);
  }
  qsort(order, rows, sizeof(KeyRow), key_row_cmp);
  double tp_before = 0.0, fp_before = 0.0, area = 0.0;
  for (uint32_t i = 0; i < rows;) {
    double tp = 0.0, fp = 0.0;
    uint32_t j = i;
    for (; j < rows && order[j].key == order[i].key; ++j) {
      uint32_t r = order[j].row;
      float w = weights ? weights[r] : 1.0f;
      tp += (double)fabsf(labels[r] * w);
      fp += (double)fabsf((1.0f - labels[r]) * w);
    }
    /* ROC: trapezoid under the step (kernels/radix_sort.metal.h:740-744). */
    area += pr ? pr_step_area(tp_before, fp_before, tp, fp, positives) : fp * (2.0 * tp_before + tp) * 0.5;
    tp_before += tp;
    fp_before += fp;
    i = j;
  }
  out[0] = area;
  out[1] = positives;
  out[2] = negatives;
  free(order);
}

void oracle_cv_folds(uint32_t rows, int nfold, uint32_t seed, int shuffle, int stratified, const float* labels,
                     int32_t model, int32_t* fold) {
  uint32_t* order = (uint32_t*)malloc(sizeof(uint32_t) * (rows ? rows : 1));
  for (uint32_t r = 0; r < rows; ++r) order[r] = r;
  if (shuffle && rows > 1) {
    /* std::shuffle with mt19937(seed) (src/c_api.cpp:1018-1110), with
     * libstdc++'s draws (model 0, an x86-64 build) or libc++'s (model 1, the
     * reference's macOS builds). */
    OracleMT g;
    oracle_mt_seed(&g, seed);
    oracle_std_shuffle(order, rows, &g, model);
  }
  if (stratified) {
    /* Stable insertion sort by label (test sizes are small). */
    for (uint32_t i = 1; i < rows; ++i) {
      uint32_t v = order[i], j = i;
      while (j > 0 && labels[order[j - 1]] > labels[v]) { order[j] = order[j - 1]; --j; }
      order[j] = v;
    }
    for (uint32_t pos = 0; pos < rows; ++pos) fold[order[pos]] = (int32_t)(pos % (uint32_t)nfold);
  } else {
    uint32_t pos = 0;
    for (int k = 0; k < nfold; ++k) {
      uint32_t chunk = rows / (uint32_t)nfold + ((uint32_t)k < rows % (uint32_t)nfold ? 1u : 0u);
      for (uint32_t j = 0; j < chunk; ++j) fold[order[pos++]] = k;
    }
  }
  free(order);
}
