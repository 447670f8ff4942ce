/*
 * mgb_kernels.h -- thin C ABI between the C++ host (learner, tree grower,
 * XGBoost C API) and the HIP kernels for gfx950.
 *
 * Every entry point takes plain device pointers, sizes and POD parameter
 * blocks, returns 0 on success or -1 on failure (message in
 * mgb_last_error()), and enqueues its work on the library's single HIP
 * stream.  It replaces the reference's Metal runtime and dispatch layer:
 *   src/runtime.mm:37-455, include/metalgb/runtime.hpp:14-114
 *   (Buffer, Runtime, Command::dispatch/zero/commit/wait).
 * The POD layouts replace include/metalgb/shared.h:18-168 for this path.
 */
#ifndef MGB_KERNELS_H
#define MGB_KERNELS_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime: device, stream, memory (src/runtime.mm:37-199) ---------- */
int mgb_init(int device);
const char* mgb_last_error(void);
int mgb_device_count(int* count);
/* Device memory ordered on the library's one stream.  A freed buffer is kept
 * by the library (up to 8 GiB) for the next request of about its size and
 * only returned to HIP when an allocation would otherwise fail; mgb_free
 * takes only pointers from mgb_malloc. */
int mgb_malloc(void** ptr, size_t bytes);
int mgb_free(void* ptr);
int mgb_memcpy_h2d(void* dst, const void* src, size_t bytes);
int mgb_memcpy_d2h(void* dst, const void* src, size_t bytes);
int mgb_memcpy_d2d(void* dst, const void* src, size_t bytes);
/* Enqueued host-to-device copy; returns once src may be reused (pageable
 * memory is staged before the call returns). */
int mgb_memcpy_h2d_async(void* dst, const void* src, size_t bytes);
int mgb_memset(void* dst, int value, size_t bytes);
int mgb_synchronize(void);
/* Event timing on the library stream (src/runtime.mm:203-280 profiler). */
int mgb_event_record(int slot);
int mgb_event_elapsed_ms(int begin_slot, int end_slot, float* ms);
/* Per-kernel-class timing: when enabled, every launch of the classes below is
 * bracketed by HIP events on the library stream; mgb_profile_collect waits
 * for the stream and adds the elapsed times (src/runtime.mm:203-280). */
enum {
  MGB_PROF_GRADIENT = 0, MGB_PROF_HISTOGRAM = 1, MGB_PROF_SPLIT = 2, MGB_PROF_CONTROL = 3,
  MGB_PROF_PARTITION = 4, MGB_PROF_PREDICT = 5, MGB_PROF_REDUCE = 6, MGB_PROF_KINDS = 7
};
int mgb_profile_enable(int on);
int mgb_profile_collect(void);
int mgb_profile_read(double* ms, uint64_t* launches, int kinds);
int mgb_profile_reset(void);
/* Plain device copy (dst, src 16-byte aligned); the bandwidth reference for
 * the roofline and the calibration kernel for HBM counters. */
int mgb_stream_copy(void* dst, const void* src, size_t bytes);

/* ---- POD layouts ------------------------------------------------------ */

/* Bin matrix of bin_bytes = 1 (u8) or 2 (u16) codes.  Features form groups
 * of group_features (4, 8 or 16; the last group padded with missing codes);
 * the code of (row, f) is at
 *   bins + (f / group_features) * group_stride + row * row_stride
 *        + (f % group_features) * bin_bytes.
 * Row-major: row_stride = groups * group_features * bin_bytes and
 * group_stride = group_features * bin_bytes (a row's codes are contiguous).
 * Group-major: row_stride = group_features * bin_bytes and group_stride =
 * rows * row_stride (each feature group's codes are contiguous over rows), so
 * a workgroup that histograms one group streams only that group's bytes.
 * missing_code marks a missing value: 0xFF / 0xFFFF when the matrix has
 * missing values, 0xFFFFFFFF (matches no code) when it has none, so a dense
 * matrix keeps u8 codes for all 256 bins. */
typedef struct {
  uint32_t rows, cols, row_stride, bin_bytes;
  uint32_t max_bin;         /* histogram bins per feature; slot max_bin holds missing */
  uint32_t cut_stride;      /* floats per feature in the cut array */
  uint32_t missing_code;
  uint32_t group_features;
  uint64_t group_stride;    /* bytes */
} MgbMatrix;

/* Per-round gradient statistics (replaces GradientParams/GradCert,
 * include/metalgb/shared.h:58-62, :110-113, and the uniform-sampling part of
 * SamplingParams, :63-67).  subsample < 1 keeps a row iff its draw from the
 * round's sample_seed is below subsample; dropped rows get (0, 0). */
typedef struct {
  uint32_t rows, objective, has_weight, sample_seed;
  float scale_pos_weight, subsample, padding1, padding2;
} MgbGradParams;

/* Split regularisation (replaces SplitParams, include/metalgb/shared.h:114-119).
 * inject_status: a test hook -- its bits are reported in the tree's status
 * word (see mgb_grow_tree) as if the device had detected them, while every
 * kernel runs normally; 0 in normal use. */
typedef struct {
  float reg_lambda, reg_alpha, min_child_weight, max_delta_step;
  float min_split_loss, eta;
  uint32_t max_depth, fma_contract;
  uint32_t inject_status, padding;
} MgbSplitParams;

/* Tree status bits (the second word at mgb_grow_tree's node_count), set by
 * the device when a tree's control state is inconsistent, as the reference's
 * tree driver sets its error word (kernels/tree_driver.metal.h:56-70).  The
 * level that finds it stops expanding and writes nothing out of range; the
 * host refuses the tree (src/tree.cpp:1664-1665). */
enum {
  MGB_TREE_STATUS_NODE_ID = 1u,    /* a frontier node's id is outside the tree's node table */
  MGB_TREE_STATUS_CAPACITY = 2u,   /* children would lie beyond the node table or the frontier */
  MGB_TREE_STATUS_TASKS = 4u,      /* a level's histogram or partition tasks exceed the workspace */
  MGB_TREE_STATUS_PARTITION = 8u   /* a child's row count exceeds its parent's */
};

/* One tree node as the host model consumes it (include/metalgb/shared.h:27-31
 * plus base_weights). */
typedef struct {
  int32_t left, right, parent, feature;
  float threshold, leaf, cover, gain;
  uint32_t default_left;
  float base_weight;
} MgbTreeNode;

/* Device-side tree workspace sizes; see mgb_tree_workspace_bytes.
 * column_levels: levels (from the root) whose histograms read the
 * column-major codes passed to mgb_grow_tree instead of the bin matrix; the
 * rows of shallow nodes are dense enough that one feature column per load
 * beats partial rows of the row-major matrix (0: never). */
typedef struct {
  uint32_t rows, cols, max_bin, max_depth;  /* rows below 2^31, max_depth 1..16 */
  uint32_t rows_per_tile, features_per_group, unit_hessian, dense;
  uint32_t column_levels;
  uint32_t sparse;  /* 1: the workspace is for mgb_grow_tree_csr (no per-tile partial histograms) */
  /* Rows per histogram tile at the root (0: rows_per_tile).  The root reads
   * every row in order, so longer tiles cost no locality and leave fewer
   * per-tile partial histograms for the split kernel to sum. */
  uint32_t root_rows_per_tile;
  /* 1: rows whose quantized gradient pair is (0, 0) -- the rows a subsample
   * drops -- leave the tree's row list before the root
   * (kernels/tree_sample_columns.metal.h:4-31 tree_rows_compact_sampled):
   * histograms and partitions see only the kept rows, and the dropped rows
   * get their leaf added to the margin by a walk of the finished tree.
   * mgb_grow_tree only (0 for the CSR driver). */
  uint32_t compact_sampled;
  /* 1: the row partition is stable -- inside each child the rows keep their
   * order in the parent's row list (kernels/boost.metal:1550-1614) -- at the
   * cost of one more launch per level (a counting pass that keeps each row
   * tile's directions and left count; the scatter takes every tile's
   * positions from the counts of its node's tiles).  0: tiles claim
   * their ranges with atomics, so the order inside a child follows arrival.
   * Histograms are exact integer sums, so the trees are identical either way. */
  uint32_t stable_partition;
} MgbTreeShape;

/* ---- data: quantile cuts and bin matrix ------------------------------- */
/* Weighted-quantile-sketch cuts of a row-major float matrix
 * (src/quantile.cpp:22-212, kernels/quantile.metal.h:19-412).
 * cuts: cols*max_bin floats, counts: cols.  weights may be NULL.  Allocates
 * its temporary device memory and synchronises the stream (one-time set-up). */
int mgb_sketch_cuts(const float* X, uint32_t rows, uint32_t cols, const float* weights, uint32_t max_bin,
                    float* cuts, uint32_t* counts);
/* Largest number of entries (present values) the sketch processes as one
 * group of features; 0 (the default) sizes groups from the free device
 * memory, about 64 bytes of temporaries per entry within a quarter of it.
 * Smaller groups bound the sketch's memory at the cost of fewer features in
 * flight per launch; the cuts are the same for any size.  No counterpart in
 * the reference (its sketch runs on the host). */
int mgb_sketch_group_entries(uint64_t entries);
/* Host only (no device work), a test hook: the ids 0..n-1 of elements with
 * these keys in the order the sketch's tie sort leaves them -- the device
 * code that re-sorts a batch whose equal values carry different zero signs
 * or weights, with libstdc++'s std::sort steps (stock XGBoost's x86-64
 * build merges equal sketch values in that order; the reference restates
 * libc++'s, kernels/sketch_sort.metal.h).  Keys compare as the binary32
 * values of sketch order keys (unsigned compare for keys below 2^31). */
int mgb_tie_sort_order(const uint32_t* keys, uint32_t n, uint32_t* order);
/* bin = min(#{cuts <= v}, count-1); NaN -> missing code
 * (kernels/boost.metal:476-499, src/data.cpp:1210-1306).  Sets *any_missing. */
int mgb_quantize_bins(const float* X, const float* cuts, const uint32_t* counts, const MgbMatrix* m, void* bins,
                      uint32_t* any_missing);
/* mgb_quantize_bins that also writes the codes column-major, code (r, f) at
 * columns[f * rows + r] (bin_bytes each), from the same pass over X. */
int mgb_quantize_bins_columns(const float* X, const float* cuts, const uint32_t* counts, const MgbMatrix* m,
                              void* bins, void* columns, uint32_t* any_missing);

/* ---- gradients -------------------------------------------------------- */
/* Words of the gradient-mass scratch of mgb_gradients / mgb_gradient_mass:
 * per-workgroup exact partial sums of |g| and |h| and a completion counter.
 * Zero it once; every call leaves the counter zeroed again. */
#define MGB_MASS_WORDS 5640
/* Objective gradients (kernels/boost.metal:553-601) written as float2 (g, h),
 * the exact |g|, |h| mass (kernels/gradient_quantization.metal.h:4-24) and,
 * from it, the power-of-two fixed-point scales[2]
 * (kernels/gradient_quantization.metal.h:26-67), in one launch. */
int mgb_gradients(const MgbGradParams* p, const float* margin, const float* labels, const float* weights,
                  float* grad, uint64_t* mass, float* scales);
/* Row sampling (p->subsample < 1, applied in place), mass and scales of
 * caller-provided gradients (custom objectives); p->objective and
 * p->has_weight are not used. */
int mgb_gradient_mass(const MgbGradParams* p, float* grad, uint64_t* mass, float* scales);
/* Scales from 2 x 256 u64 mantissa sums per binary32 exponent (|g| then |h|)
 * in mass[0..511]; clears them. */
int mgb_gradient_scales(uint64_t* mass, float* scales);
/* Weighted label mean (src/learner.cpp:316-333): out[0] = binary32 mean. */
int mgb_base_score(const float* labels, const float* weights, uint32_t rows, uint32_t objective,
                   float scale_pos_weight, float* out);
/* margin[r] = value for all rows. */
int mgb_fill_f32(float* data, uint64_t count, float value);
/* *flag (device) |= 1 if any of count floats is NaN. */
int mgb_any_missing(const float* data, uint64_t count, uint32_t* flag);
/* Output transform of margins: objective 1 (logistic) maps x -> 1/(1+exp(-x)). */
int mgb_transform(float* data, uint64_t count, uint32_t objective);

/* Host only (no device work): checks one tree's node records as the host
 * publishes them (src/learner.cpp:36-61 checks the emitted table against the
 * host replay, src/tree.cpp:1663-1717): status 0; 1 <= count <= max_nodes;
 * node 0 the root (parent -1); every split node's children are the next two
 * unused ids in node-id order (left = 2k + 1 for the k-th split node), both
 * name it as their parent and come after it; leaves have no children and no
 * feature; split features are below cols and leaf values finite.  Returns 0,
 * or -1 with the first violation in mgb_last_error(). */
int mgb_validate_tree(const MgbTreeNode* nodes, uint32_t count, uint32_t status, uint32_t max_nodes, uint32_t cols);

/* Host only (no device work): the permutation std::shuffle(0..n-1) draws over
 * std::mt19937(seed) in the column sample (src/tree.cpp:28-45), with
 * libstdc++'s draws (model 0, x86-64 builds) or libc++'s (model 1, the
 * reference's macOS builds); *next_draw (if not NULL) receives the engine's
 * next output.  Returns -1 for another model. */
int mgb_std_shuffle(uint32_t seed, uint32_t n, uint32_t model, uint32_t* order, uint32_t* next_draw);

/* ---- one depthwise tree ---------------------------------------------- */
size_t mgb_tree_workspace_bytes(const MgbTreeShape* shape);
/* Grows one depthwise tree on the device and adds its leaves to margin
 * (src/tree.cpp:455-1029 GPU-driven tree + replay :1663-1717 and the
 * prediction-cache update kernels/boost.metal:1738-1763).  Nothing is
 * synchronised; nodes (2^(max_depth+1)-1 records) and node_count are device
 * pointers filled by the time the stream drains.  node_count holds two
 * words: [0] the number of nodes, [1] the tree's status (0, or
 * MGB_TREE_STATUS_* bits: the tree is not valid).  features (device, cols
 * flags, may be NULL for all) restricts the split search to the tree's
 * column sample (src/tree.cpp:179-180).  monotone (device, cols int32 of -1, 0
 * or 1, may be NULL for none) applies monotone constraints
 * (src/tree.cpp:15-26, :1083-1086; kernels/boost.metal:902-920): each node
 * carries bounds on its weight, every weight is clamped to them, a split on an
 * increasing (decreasing) feature needs left weight <= (>=) right weight,
 * and the children's bounds meet at the midpoint of their weights.  columns (device, may be NULL) holds
 * the same codes column-major, code(row, f) at columns + (f * rows + row) *
 * bin_bytes: the row partition then reads its split feature's codes from one
 * column instead of one cache line of the row-major matrix per row. */
int mgb_grow_tree(const MgbTreeShape* shape, const MgbMatrix* m, const void* bins, const void* columns, const float* cuts,
                  const uint32_t* counts, const float* grad, const float* scales, const MgbSplitParams* sp,
                  const uint32_t* features, const int32_t* monotone, void* workspace, size_t workspace_bytes,
                  float* margin, MgbTreeNode* nodes, uint32_t* node_count);

/* mgb_grow_tree without a workspace argument and without allocating: no
 * counterpart in the reference.  For callers that cannot allocate device
 * memory (tight serving or online-update loops, harnesses that forbid
 * hipMalloc).  The work is queued on the library's own stream, so a HIP graph
 * capture that the caller begins on another stream does not record it (the
 * kernels run eagerly, outside the caller's graph).  The workspace is a static 64 MiB
 * device array of the library (one per device, held until the process
 * ends); shapes whose mgb_tree_workspace_bytes exceeds it are rejected with
 * an error, as is a call while per-kernel timing is on (its events are
 * created on demand).  Every call on a device shares and overwrites that
 * device's scratch: the library enqueues all calls on its single stream,
 * which orders them; calls that ran concurrently on one device would race.
 * Nothing in the scratch needs to start at zero: each tree initialises its
 * own state.  Other arguments and results as for mgb_grow_tree. */
int mgb_grow_tree_noalloc(const MgbTreeShape* shape, const MgbMatrix* m, const void* bins, const void* columns,
                          const float* cuts, const uint32_t* counts, const float* grad, const float* scales,
                          const MgbSplitParams* sp, const uint32_t* features, const int32_t* monotone, float* margin,
                          MgbTreeNode* nodes, uint32_t* node_count);

/* ---- CSR input (src/data.cpp:721-870 Matrix::sparse) ----------------- *
 * indptr holds rows+1 offsets into indices/values; column indices are
 * strictly increasing within a row; absent entries are missing values. */
typedef struct {
  uint32_t rows, cols, max_bin, cut_stride;
  uint32_t bin_bytes, missing_code;  /* codes per nonzero: u8 or u16; NaN values carry missing_code */
  uint64_t nnz;
} MgbCsrMatrix;

/* Column-major copy of a CSR matrix: colptr (cols+1 offsets) and, grouped by
 * column in row order, every nonzero's row and value (and its column in
 * csc_cols unless NULL).  Synchronises. */
int mgb_csr_to_csc(const uint64_t* indptr, const uint32_t* indices, const float* values, uint32_t rows, uint32_t cols,
                   uint64_t nnz, uint64_t* colptr, uint32_t* csc_rows, float* csc_values, uint32_t* csc_cols);
/* Quantile cuts from the column-major copy: the cuts mgb_sketch_cuts gives
 * for the dense matrix with NaN at the absent entries (src/quantile.cpp:22-212
 * over the present values of each column).  Synchronises. */
int mgb_sketch_cuts_csc(const float* values, const uint32_t* row_of, const uint64_t* colptr, uint32_t rows,
                        uint32_t cols, const float* weights, uint32_t max_bin, float* cuts, uint32_t* counts);
/* Bin code of every nonzero with the dense bin rule; NaN -> missing_code
 * (kernels/sparse_data.metal.h:460-498 sparse_quantize_csr). */
int mgb_quantize_csr(const uint32_t* indices, const float* values, uint64_t nnz, const float* cuts,
                     const uint32_t* counts, uint32_t cut_stride, uint32_t bin_bytes, uint32_t missing_code,
                     void* codes);
/* mgb_grow_tree over a CSR bin matrix (codes per nonzero, see
 * mgb_quantize_csr): histograms of the nonzeros with 64-bit device atomics
 * and each feature's missing slot as the node total minus its present bins
 * (kernels/histogram_csr.metal.h:22-153), the partition looking up the split
 * feature in each row (:155-262).  The root, which holds every row, builds
 * its histogram from the column-major codes instead (colptr, csc_rows as
 * from mgb_csr_to_csc, csc_codes its columns' codes): a few features per
 * workgroup in LDS and plain stores, no device atomics.  The shape must have
 * sparse = 1; features and monotone as for mgb_grow_tree. */
int mgb_grow_tree_csr(const MgbTreeShape* shape, const MgbCsrMatrix* m, const uint64_t* indptr,
                      const uint32_t* indices, const void* codes, const uint64_t* colptr, const uint32_t* csc_rows,
                      const void* csc_codes, const float* cuts, const uint32_t* counts,
                      const float* grad, const float* scales, const MgbSplitParams* sp, const uint32_t* features,
                      const int32_t* monotone, void* workspace, size_t workspace_bytes, float* margin,
                      MgbTreeNode* nodes, uint32_t* node_count);
/* mgb_predict over a CSR matrix of raw values. */
int mgb_predict_csr(const uint64_t* indptr, const uint32_t* indices, const float* values, uint32_t rows,
                    const MgbTreeNode* nodes, const uint32_t* tree_offsets, uint32_t trees, float* margin);

/* Rows and nodes whose histograms each level built directly (not by
 * subtraction), from the last mgb_grow_tree on this workspace; synchronises. */
int mgb_tree_level_stats(const MgbTreeShape* shape, const void* workspace, uint64_t* rows_built,
                         uint32_t* nodes_built, uint32_t levels);
/* Rows the partition of each level of the last mgb_grow_tree on this
 * workspace handled: rows of the nodes that split there (moved into their
 * children's segments; at the last level given the child's leaf) and rows of
 * the nodes that stopped there (their leaf added to the margin);
 * synchronises.  The partition's algorithmic bytes per level follow from
 * them; a diagnostic, no counterpart in the reference. */
int mgb_tree_partition_stats(const MgbTreeShape* shape, const void* workspace, uint32_t* rows_split,
                             uint32_t* rows_leaf, uint32_t levels);
/* Copies to host memory the row list (shape->rows words) that level `depth`
 * of the last mgb_grow_tree on this workspace read: each node's rows form one
 * segment of it.  Valid for the last two levels of a tree (the list of level
 * d is overwritten by the partition of level d + 1); synchronises.  A
 * diagnostic for the partition's row order, no counterpart in the reference. */
int mgb_tree_row_list(const MgbTreeShape* shape, const void* workspace, uint32_t depth, uint32_t* rows);

/* ---- kernel-level entry points used by parity tests and the profiler --- */
/* Histogram of rows [0, count) of row list `rows` (NULL = identity) into
 * hist[cols][max_bin+1][2] int64 (kernels/boost.metal:700-733). */
int mgb_histogram(const MgbTreeShape* shape, const MgbMatrix* m, const void* bins, const uint32_t* rows,
                  uint32_t count, const float* grad, const float* scales, int64_t* hist, void* workspace,
                  size_t workspace_bytes);
/* Prediction: margin[r] += leaf of each tree (kernels/boost.metal:1738-1763). */
int mgb_predict(const float* X, uint32_t rows, uint32_t cols, const MgbTreeNode* nodes, const uint32_t* tree_offsets,
                uint32_t trees, float* margin);

/* ---- leaf indices and feature contributions -------------------------- *
 * (src/learner.cpp:455-560 Learner::predict types 6 and 2-5.)  Rows are
 * dense (X: rows x cols floats, indptr NULL) or CSR (X holds the values,
 * indptr rows+1 offsets, indices strictly increasing column ids a row;
 * absent entries are missing); trees [tree_offsets[0], ...) of `nodes`.
 * mgb_predict_leaf: out[r * trees + t] = the leaf node id row r reaches in
 * tree t.  mgb_predict_contribs: out[r * (cols + 1) + f] = feature f's
 * contribution to row r's margin, out[r * (cols + 1) + cols] = the bias
 * (base[r], or base_value when base is NULL, plus every tree's root mean);
 * node_means holds each node's cover-weighted mean leaf value at the node's
 * index in `nodes`.  approximate = 0: exact path-dependent TreeSHAP (trees of
 * depth <= 16, max_depth the deepest tree's); 1: each split's feature gets the
 * change of the node mean along the row's path.  interactions = 1: each row
 * is a (cols + 1) x (cols + 1) matrix at out + r * (cols + 1)^2 -- exact: SHAP
 * interaction values (off the diagonal half the change of feature j's value
 * between feature i always present and always absent, on it feature i's
 * value less its interactions); approximate: the approximate values on the
 * diagonal -- with the bias in the last element (types 4 and 5). */
int mgb_predict_leaf(const float* X, const uint64_t* indptr, const uint32_t* indices, uint32_t rows, uint32_t cols,
                     const MgbTreeNode* nodes, const uint32_t* tree_offsets, uint32_t trees, float* out);
int mgb_predict_contribs(const float* X, const uint64_t* indptr, const uint32_t* indices, uint32_t rows,
                         uint32_t cols, const MgbTreeNode* nodes, const float* node_means,
                         const uint32_t* tree_offsets, uint32_t trees, uint32_t max_depth, uint32_t approximate,
                         uint32_t interactions, const float* base, float base_value, float* out);

/* ---- evaluation metrics (src/metrics.cpp:8-159) ------------------------- */
/* Elementwise metric kinds, numbered as the reference's metric table
 * (src/metrics.cpp:13-16). */
enum {
  MGB_METRIC_RMSE = 0, MGB_METRIC_MAE = 1, MGB_METRIC_RMSLE = 2, MGB_METRIC_LOGLOSS = 3, MGB_METRIC_ERROR = 6,
  MGB_METRIC_MAPE = 7, MGB_METRIC_MPHE = 8, MGB_METRIC_POISSON = 9, MGB_METRIC_GAMMA_DEVIANCE = 10,
  MGB_METRIC_TWEEDIE = 11, MGB_METRIC_GAMMA_NLOGLIK = 12
};
/* Scratch bytes mgb_metric_sum and mgb_metric_auc need for `rows`. */
size_t mgb_metric_workspace_bytes(uint32_t rows);
/* (sum of weight * loss, sum of weight) over rows into out[2] (host), with
 * the reference's summation order: a 256-element pairwise tree per block,
 * compensated sums over blocks, a final tree (kernels/boost.metal:2225-2295).
 * weights NULL = 1; parameter = error threshold, huber slope or tweedie
 * power.  Synchronises. */
int mgb_metric_sum(const float* pred, const float* labels, const float* weights, uint32_t rows, uint32_t kind,
                   float parameter, float* out, void* workspace, size_t workspace_bytes);
/* ROC-AUC area (pr = 0) or PR-AUC area (pr = 1) in binary64 over the rows
 * sorted by descending prediction, tied predictions forming one step; out =
 * {area, positive weight, negative weight} on the host
 * (kernels/radix_sort.metal.h:427-790).  Synchronises. */
int mgb_metric_auc(const float* pred, const float* labels, const float* weights, uint32_t rows, int pr, double* out,
                   void* workspace, size_t workspace_bytes);

#ifdef __cplusplus
}
#endif
#endif
