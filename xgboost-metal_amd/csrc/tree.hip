// One depthwise tree on gfx950: per level
//   plan (smaller child of each sibling pair) -> clear multi-tile histograms
//   -> LDS-private integer histograms (row tiles x feature groups)
//   -> fused sibling subtraction + wave64 prefix-scan split evaluation
//   -> select/apply (argmax over features, node records, child ids)
//   -> ballot+prefix row partition with the margin update fused in: stable
//      (a counting pass first, then each child keeps its parent's row order)
//      or, with one launch fewer, tiles claiming their ranges by atomics (the
//      order inside a child follows arrival; the trees are the same).
// All control lives on the device: kernels read work counts written by the
// previous kernel, so the host enqueues a whole tree without a wait
// (the reference's GPU-driven tree, src/tree.cpp:455-1029, uses indirect
// dispatch for the same purpose).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstring>
#include <mutex>

#include "device_common.hpp"

// Tree workspace of mgb_grow_tree_noalloc, for callers that cannot allocate:
// one copy per device, from module load until the process ends.  Host code
// never uses this name as an address: the device address comes from
// hipGetSymbolAddress (scratch_address below).
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace mgb {
namespace {

// Rows per partition task (Tree::part_tile): 2048 for the stable partition
// of a dense matrix (10M x 128: partition 1.66 -> 1.55 ms per round against
// 1024; 512: 2.06 ms), else 1024 (262,144 x 64 with claims: 38.0 against
// 38.6 ms per fit at 2048; 1M x 2000 CSR, whose row test is a search in the
// row: 0.37 against 0.44 ms per round).  The partition kernels take the rows
// per thread (part_tile / kPartThreads) as a template argument.
constexpr uint32_t kPartTileWide = 2048, kPartTileNarrow = 1024;
constexpr uint32_t kPartThreads = 256;    // partition (and select bookkeeping) workgroup
constexpr uint32_t kSelectThreads = 256;
constexpr uint32_t kHistThreads = 1024;
constexpr int kHistUnroll = 2;          // rows per thread per histogram batch

enum : uint32_t { kOpNone = 0, kOpLeaf = 1, kOpSplit = 2, kOpFinal = 3 };

constexpr uint32_t kMaxLevels = 32;
// Features per node from which the split kernel reads a node's best key
// before offering its own (see score_node).
constexpr uint32_t kContendedFeatures = 512;
// Independent one-wave split items packed into one workgroup (8: C3's
// rounds 1.6 % slower, C2 unchanged; 16: C2 3 % and C3 11 % slower).
constexpr uint32_t kSplitPack = 4;
// Stable partition: levels of at most this many nodes are planned by the
// select bookkeeping from the counting pass's left counts (no k_plan).
constexpr uint32_t kPlanNodes = 2048;

struct LevelState {
  uint32_t n_nodes;       // frontier size of the current level
  uint32_t n_hist_tasks;
  uint32_t n_zero;
  uint32_t n_part[2];     // partition tasks of the levels of each parity (banked: the
                          // apply kernel of one level plans the next while it runs)
  uint32_t node_count;    // tree nodes allocated so far
  uint32_t error;
  uint32_t kept, dropped;  // row compaction: rows kept (row list [0, kept)) and dropped
                           // (stored from the end of the list down)
  uint32_t padding[7];
  // Per level: rows and nodes whose histograms were built directly.
  uint64_t rows_built[kMaxLevels];
  uint32_t nodes_built[kMaxLevels];
  // Per level: rows of the nodes that split there and of those that stopped
  // (the partition's work: moved rows, margin updates).
  uint32_t rows_split[kMaxLevels];
  uint32_t rows_leaf[kMaxLevels];
};

struct Frontier {
  int32_t id;             // tree node id
  uint32_t begin, count;  // segment of this level's row buffer
  uint32_t parent_slot;   // parent's slot in the previous level's histogram bank
  int64_t sum_g, sum_h;   // node integer totals (the parent's chosen child sums)
  uint32_t built;         // histogram built directly (1) or by subtraction (0)
  uint32_t first_task;    // built nodes: first histogram task (row tile)
  uint32_t ntiles;        // built nodes: number of row tiles
  float leaf;             // the node's leaf value if it does not split
  float lower, upper;     // monotone bounds of the node's weight (src/tree.cpp:1083-1086)
  uint32_t padding[2];
};

struct Cand {
  float gain;
  int32_t feature;
  uint32_t bin, default_left;
  float threshold, left_w, right_w, left_h, right_h;
  float parent_w, total_h;
  uint32_t padding;
  int64_t lg, lh, rg, rh;
};

// Per (node, feature): the feature's best candidate, rebuilt in full by the
// select kernel for the node's winning feature only.
struct SplitRec {
  float gain;
  uint32_t order;   // b (missing right) or 2*count-1-b (missing left)
  int64_t lg, lh;   // left child sums
};

struct NodeOp {
  uint32_t op, feature;
  int32_t last_left_bin;
  uint32_t default_left;
  float leaf, left_leaf, right_leaf;
  uint32_t child_slot;
};

struct HistTask { uint32_t slot, begin, end, single; };

// Per-node best-feature key: (gain order << 32) | a low word that falls as the
// feature rises, so the maximum is the largest gain and, among equal gains,
// the lowest feature -- the serial first-strictly-greater scan over features
// (kernels/boost.metal:1245-1265).  +0 and -0 map to one key; 0 means no
// valid candidate.  Up to kKeyFeatures features the low word is
// (kKeyFeatures - feature) << 16 | backward << 15 | bin: the partition reads
// a split's feature, bin and direction off the key, with no load of the
// feature's record after it; with more features it is ~feature.  A feature
// offers one candidate per node, so the bin bits never decide between keys.
constexpr uint32_t kKeyFeatures = 65535;
__device__ __forceinline__ uint64_t best_key(float gain, uint32_t feature, uint32_t order, uint32_t count,
                                             uint32_t cols) {
  const uint32_t bits = gain == 0.0f ? 0u : __float_as_uint(gain);
  const uint32_t rank = bits ^ ((bits & 0x80000000u) ? 0xffffffffu : 0x80000000u);
  uint32_t low = ~feature;
  if (cols <= kKeyFeatures) {
    const uint32_t backward = order >= count ? 1u : 0u;
    const uint32_t bin = backward ? 2 * count - 1 - order : order;  // < 2^15 (max_bin <= 4096)
    low = ((kKeyFeatures - feature) << 16) | (backward << 15) | bin;
  }
  return ((uint64_t)rank << 32) | (uint64_t)low;
}
__device__ __forceinline__ uint32_t key_feature(uint64_t key, uint32_t cols) {
  return cols <= kKeyFeatures ? kKeyFeatures - (uint32_t)((key >> 16) & 0xffffu) : ~(uint32_t)key;
}
// The gain a key was made from (-0 comes back as +0).
__device__ __forceinline__ float key_gain(uint64_t key) {
  const uint32_t rank = (uint32_t)(key >> 32);
  return __uint_as_float((rank & 0x80000000u) ? rank ^ 0x80000000u : ~rank);
}
struct PartTask { uint32_t slot, begin, end, padding; };

// Device pointers of one tree workspace.
struct Tree {
  LevelState* state;
  uint32_t* rows[2];
  // Gradient pairs in row-list order: gh[d & 1][i] = grad[rows[d & 1][i]]
  // for the levels whose histograms gather rows (the partition moves each
  // row's pair with its id), so the histogram reads them in order instead of
  // one gathered line per row and feature group.
  float2* gh[2];
  int64_t* hist[2];
  Frontier* frontier[2];
  SplitRec* recs;             // per (frontier slot, feature): the feature's best candidate
  unsigned long long* best;   // per frontier slot, see best_key
  HistTask* hist_tasks;
  uint32_t* zero_list;        // built nodes with several row tiles (reduced from partials)
  int64_t* partials;          // per (task, feature group): G x (max_bin+1) (g, h) partial histograms
  PartTask* part_tasks;       // two banks of max_part_tasks, by level parity
  uint32_t* cursors;          // per split node: next left position, end of the free right range
  // Stable partition only (NULL otherwise): per partition task, the ballot
  // masks of its left rows and its left count.
  uint64_t* part_masks;
  uint32_t* part_left;
  uint32_t* final_order;      // stable partition: the last level's tasks by row range, then 9 XCD list offsets
  // Inputs.
  const void* bins;
  const void* columns;        // column-major codes for the partition (NULL: read bins)
  const uint64_t* csr_indptr; // CSR bin matrix (mgb_grow_tree_csr; NULL for a dense matrix)
  const uint32_t* csr_indices;
  const void* csr_codes;
  const uint64_t* csc_colptr; // its column-major copy, for the root histogram (NULL: atomics at the root too)
  const uint32_t* csc_rows;
  const void* csc_codes;
  const float* cuts;
  const uint32_t* counts;
  const uint32_t* allowed;    // per feature: nonzero if in the tree's column sample (NULL: all)
  const int32_t* monotone;    // per feature -1, 0 or 1: monotone constraint (NULL: none)
  const float2* grad;
  const float* scales;
  float* margin;
  MgbTreeNode* nodes;
  int32_t* split_bins;        // per tree node id: the split's last left bin (the walk of dropped rows)
  uint32_t* node_count_out;
  // The tree's status word (node_count_out + 1; NULL for the histogram-only
  // entry point): MGB_TREE_STATUS_* bits of inconsistencies the bookkeeping
  // found, OR-ed in; the tree's set-up starts it at sp.inject_status.
  uint32_t* status;
  // Shape.
  uint32_t rows_n, cols, max_bin, bins1;     // bins1 = max_bin + 1
  uint32_t row_stride, bin_bytes, missing_code, cut_stride;
  uint32_t max_depth, slots, rows_per_tile, groups;
  uint32_t root_tile;                        // rows per histogram tile at the root
  uint32_t features_per_group, unit_hessian, dense, max_hist_tasks;
  uint32_t max_part_tasks;
  uint32_t column_levels;                    // histogram levels that read `columns`
  uint32_t select_plans;                     // unit Hessians, dense: the select bookkeeping plans the next level
  uint32_t sparse;                           // CSR: missing slots from node totals, no partials
  uint32_t compact;                          // the root's rows are the kept rows of a subsample
  uint32_t fused_level0;                     // the root histogram's workgroup 0 runs level0_setup
  uint32_t stable;                           // stable partition (k_part_count before k_apply)
  uint32_t part_tile;                        // rows per partition task
  uint64_t hist_entry;                       // int64 words per node histogram
  uint64_t group_stride;                     // bytes between feature groups' codes (see MgbMatrix)
  MgbSplitParams sp;
};

// Per-level banks, by depth parity: the apply kernel of level d reads level
// d's partition tasks, cursors and best keys while its bookkeeping workgroup
// writes level d+1's.
__device__ __forceinline__ PartTask* part_bank(const Tree& t, uint32_t depth) {
  return t.part_tasks + (uint64_t)(depth & 1) * t.max_part_tasks;
}
__device__ __forceinline__ uint32_t* cursor_bank(const Tree& t, uint32_t depth) {
  return t.cursors + (uint64_t)(depth & 1) * 2 * t.slots;
}
// A node's best key is spread over kKeyWays words, one 64-byte line: feature
// f offers into word f mod kKeyWays (below kContendedFeatures features; see
// offer_best), and the node's key is the words' maximum.  One word for all
// of a node's features serialized their atomics (262,144 x 64: 32.8 -> 32.0
// ms per 100 rounds with eight words).
constexpr uint32_t kKeyWays = 8;
__device__ __forceinline__ unsigned long long* best_bank(const Tree& t, uint32_t depth) {
  return t.best + (uint64_t)(depth & 1) * t.slots * kKeyWays;
}
__device__ __forceinline__ uint64_t node_key(const unsigned long long* words) {
  uint64_t key = 0;
#pragma unroll
  for (uint32_t i = 0; i < kKeyWays; ++i) key = words[i] > key ? words[i] : key;
  return key;
}

__host__ __device__ inline uint32_t div_up(uint64_t a, uint32_t b) { return (uint32_t)((a + b - 1) / b); }

// Index of the batch item that owns task j: the last k < nitems with
// off[k] <= j, where off holds the items' ascending exclusive task offsets in
// LDS (items without tasks share their successor's offset).
__device__ __forceinline__ uint32_t owner_of(const uint32_t* off, uint32_t nitems, uint32_t j) {
  uint32_t lo = 0, hi = nitems;
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) / 2;
    if (off[mid] <= j) lo = mid;
    else hi = mid;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// Scoring arithmetic (native binary64 restatement of the reference's
// software-binary64 scorer).
// ---------------------------------------------------------------------------
__device__ __forceinline__ double stat_value(int64_t v, int exponent) { return ldexp((double)v, -exponent); }

__device__ __forceinline__ int scale_exponent(float scale) {
  return (int)((__float_as_uint(scale) >> 23) & 255) - 127;
}

// kernels/scalar_gain.metal.h:56-82, split_statistics.metal.h:124-140.
__device__ __forceinline__ float calc_weight(double G, double H, const MgbSplitParams& p) {
  if (!(H > 0)) return 0.0f;
  double alpha = fabs((double)p.reg_alpha);
  double g = G;
  if (fabs(g) <= alpha) g = 0;
  else g = g + (g < 0 ? alpha : -alpha);
  double den = H + (double)p.reg_lambda;
  // -0/den is -0 in IEEE arithmetic, but the device's binary64 division
  // sequence refines the quotient with fused multiply-adds that can return +0
  // for a zero numerator; the zero case is therefore explicit (as in the
  // reference's scorer, kernels/scalar_gain.metal.h:66-77).
  float w = g == 0 ? -0.0f : (float)(-g / den);
  float limit = fabsf(p.max_delta_step);
  if (limit != 0.0f && fabsf(w) > limit) w = copysignf(limit, w);
  return w;
}

// A weight clamped to the node's monotone bounds (kernels/scalar_gain.metal.h:79-80,
// split_statistics.metal.h:35-36); the root's bounds are +-FLT_MAX.
__device__ __forceinline__ float clamp_weight(float w, float lower, float upper) {
  if (w < lower) w = lower;
  if (upper < w) w = upper;
  return w;
}

// kernels/scalar_gain.metal.h:91-103.
__device__ __forceinline__ float calc_gain(double G, double H, float w, const MgbSplitParams& p) {
  if (!(H > 0)) return 0.0f;
  double wd = (double)w;
  double square = (double)(w * w);
  double quadratic = (H + (double)p.reg_lambda) * square;
  double alpha2 = (double)p.reg_alpha + (double)p.reg_alpha;
  double sum;
  if (p.fma_contract) {
    sum = fma(G + G, wd, quadratic);
    sum = fma(alpha2, fabs(wd), sum);
  } else {
    sum = __dadd_rn(__dmul_rn(G + G, wd), quadratic);
    sum = __dadd_rn(__dmul_rn(alpha2, fabs(wd)), sum);
  }
  return (float)(-sum);
}

// ---------------------------------------------------------------------------
// Level 0 set-up: root frontier, root histogram tasks, root tree record.
// ---------------------------------------------------------------------------
__device__ void level0_setup(const Tree& t) {
  LevelState* st = t.state;
  // The root's rows: [0, N), or the kept rows k_compact_rows listed.  The
  // root histogram streams every row in order either way: a dropped row's
  // gradient pair is (0, 0) and adds nothing, and whole columns read faster
  // than the kept rows gathered through the list.
  const uint32_t n_root = t.compact ? st->kept : t.rows_n;
  uint32_t tiles = t.rows_n ? div_up(t.rows_n, t.root_tile) : 0;
  if (t.best)
    for (uint32_t i = threadIdx.x; i < 2 * t.slots * kKeyWays; i += blockDim.x) t.best[i] = 0;
  for (uint32_t i = threadIdx.x; i < tiles; i += blockDim.x) {
    uint32_t begin = i * t.root_tile;
    uint32_t end = begin + t.root_tile < t.rows_n ? begin + t.root_tile : t.rows_n;
    t.hist_tasks[i] = HistTask{0u, begin, end, tiles == 1 ? 1u : 0u};
  }
  // The root's partition tasks (row tiles of [0, n_root)) and cursors.
  const uint32_t ptiles = n_root ? div_up(n_root, t.part_tile) : 0;
  if (t.part_tasks)
    for (uint32_t i = threadIdx.x; i < ptiles; i += blockDim.x) {
      const uint32_t b = i * t.part_tile;
      t.part_tasks[i] = PartTask{0u, b, b + t.part_tile < n_root ? b + t.part_tile : n_root, 0u};
    }
  if (threadIdx.x == 0) {
    st->rows_built[0] = n_root;
    st->nodes_built[0] = 1;
    st->n_nodes = 1;
    st->n_hist_tasks = tiles;
    st->n_zero = tiles == 1 ? 0u : 1u;
    st->n_part[0] = ptiles;
    st->n_part[1] = 0;
    t.cursors[0] = 0;
    t.cursors[1] = n_root;
    st->node_count = 1;
    st->error = 0;
    if (t.status) *t.status = t.sp.inject_status;
    t.zero_list[0] = 0;
    Frontier root;
    root.id = 0; root.begin = 0; root.count = n_root; root.parent_slot = 0;
    root.sum_g = 0; root.sum_h = 0; root.built = 1; root.first_task = 0; root.ntiles = tiles; root.leaf = 0.0f;
    root.lower = -FLT_MAX; root.upper = FLT_MAX;  // tree_init_bounds
    root.padding[0] = root.padding[1] = 0;
    t.frontier[0][0] = root;
    MgbTreeNode n;
    n.left = -1; n.right = -1; n.parent = -1; n.feature = -1;
    n.threshold = 0; n.leaf = 0; n.cover = 0; n.gain = 0; n.default_left = 0; n.base_weight = 0;
    if (t.nodes) t.nodes[0] = n;  // the histogram-only entry point has no tree
  }
}

__global__ void k_level0(Tree t) { level0_setup(t); }

// Row tile i of the root (the tasks level0_setup lists), for the root's
// histogram launch, which may run level0_setup itself in one workgroup.
__device__ __forceinline__ HistTask root_task(const Tree& t, uint32_t i) {
  const uint32_t tiles = t.rows_n ? div_up(t.rows_n, t.root_tile) : 0;
  const uint32_t begin = i * t.root_tile;
  const uint32_t end = begin + t.root_tile < t.rows_n ? begin + t.root_tile : t.rows_n;
  return HistTask{0u, begin, end, tiles == 1 ? 1u : 0u};
}

// ---------------------------------------------------------------------------
// Sampled-row compaction (kernels/tree_sample_columns.metal.h:4-31
// tree_rows_compact_sampled, launched at src/tree.cpp:746-750): a row stays
// in the tree's row list iff its quantized gradient pair is not (0, 0), the
// rows a subsample drops having zero gradients.  Kept rows fill the list
// from the front, dropped rows from the back; each workgroup claims its two
// ranges with one atomic on each counter, so the order of rows within each
// range depends on scheduling -- nothing downstream depends on it (the
// histograms are exact integer sums, the margin update is per row).
// ---------------------------------------------------------------------------
constexpr uint32_t kCompactThreads = 256;
constexpr uint32_t kCompactChunks = 64;  // chunks of kCompactThreads rows per workgroup
constexpr uint32_t kCompactRows = kCompactThreads * kCompactChunks;

__global__ void k_compact_reset(Tree t) {
  if (threadIdx.x == 0) {
    t.state->kept = 0;
    t.state->dropped = 0;
  }
}

// One workgroup per kCompactRows consecutive rows, in two passes: the keep
// bits of every (chunk, wave) go to LDS as ballot masks and are counted, the
// workgroup claims its ranges with one atomic per counter (few workgroups, so
// little contention on the two counters), then every row's rank comes from
// the masks.
__global__ __launch_bounds__(kCompactThreads) void k_compact_rows(Tree t) {
  constexpr uint32_t kWaves = kCompactThreads / kWave;
  __shared__ uint64_t masks[kCompactChunks][kWaves];
  __shared__ uint32_t wave_count[kWaves];
  __shared__ uint32_t base_kept, base_dropped;
  const uint32_t lane = lane_id(), wave = threadIdx.x / kWave;
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
  const float sg = t.scales[0], sh = t.scales[1];
  const uint32_t first = blockIdx.x * kCompactRows;
  const uint32_t rows = (t.rows_n - first < kCompactRows ? t.rows_n - first : kCompactRows);  // grid: first < N
  uint32_t kept = 0;
  for (uint32_t c = 0; c < kCompactChunks; ++c) {
    const uint32_t i = c * kCompactThreads + threadIdx.x;
    bool keep = false;
    if (i < rows) {
      const float2 v = t.grad[first + i];
      keep = (int64_t)rintf(v.x * sg) != 0 || (int64_t)rintf(v.y * sh) != 0;
    }
    const uint64_t m = __ballot(keep);
    if (lane == 0) masks[c][wave] = m;
    kept += (uint32_t)__popcll(m);  // uniform over the wave
  }
  if (lane == 0) wave_count[wave] = kept;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t total = 0;
    for (uint32_t q = 0; q < kWaves; ++q) total += wave_count[q];
    base_kept = total ? atomicAdd(&t.state->kept, total) : 0u;
    base_dropped = rows > total ? atomicAdd(&t.state->dropped, rows - total) : 0u;
  }
  __syncthreads();
  uint32_t done_kept = 0;  // kept rows of earlier chunks
  for (uint32_t c = 0; c < kCompactChunks; ++c) {
    const uint32_t i = c * kCompactThreads + threadIdx.x;
    uint32_t wk = 0, ck = 0;
#pragma unroll
    for (uint32_t q = 0; q < kWaves; ++q) {
      const uint32_t n = (uint32_t)__popcll(masks[c][q]);
      if (q < wave) wk += n;
      ck += n;
    }
    if (i < rows) {
      const uint64_t m = masks[c][wave];
      const uint32_t rank = (uint32_t)__popcll(m & below);
      // Rows before this one in the workgroup's range: i (all of them are
      // present, the range being consecutive rows); kept among them:
      // done_kept + wk + rank.
      const uint32_t kept_before = done_kept + wk + rank;
      if ((m >> lane) & 1u) {
        t.rows[0][base_kept + kept_before] = first + i;
        t.gh[0][base_kept + kept_before] = t.grad[first + i];
      } else {
        t.rows[0][t.rows_n - 1 - (base_dropped + (i - kept_before))] = first + i;
      }
    }
    done_kept += ck;
  }
}

// Level d >= 1: build the smaller child of every sibling pair (ties build the
// left child, kernels/boost.metal:661-698); the other comes from subtraction.
__global__ __launch_bounds__(kSelectThreads) void k_plan(Tree t, uint32_t depth) {
  __shared__ uint32_t scan[kSelectThreads / kWave + 1];
  __shared__ uint32_t s_off[kSelectThreads], s_slot[kSelectThreads], s_begin[kSelectThreads], s_end[kSelectThreads];
  __shared__ uint32_t scan_right[kSelectThreads];
  LevelState* st = t.state;
  Frontier* fr = t.frontier[depth & 1];
  uint32_t pairs = st->n_nodes / 2;
  __shared__ uint32_t s_status;  // MGB_TREE_STATUS_* bits found by this plan
  if (threadIdx.x == 0) s_status = 0;
  __syncthreads();
  const uint32_t* parent_cursors = cursor_bank(t, depth - 1);
  uint32_t* cursors = cursor_bank(t, depth);
  unsigned long long* best = best_bank(t, depth);
  PartTask* ptasks = part_bank(t, depth);
  uint32_t carry_tasks = 0, carry_zero = 0, carry_rows = 0, carry_part = 0;
  for (uint32_t base = 0; base < pairs; base += blockDim.x) {
    uint32_t p = base + threadIdx.x;
    uint32_t tiles = 0, zero = 0, built = 0, count = 0, begin = 0;
    uint32_t lbegin = 0, c0 = 0, c1 = 0;
    if (p < pairs) {
      // Child segments from the partition's cursor: the left child holds the
      // rows below the parent's final left cursor, the right child the rest.
      Frontier& lf = fr[2 * p];
      Frontier& rf = fr[2 * p + 1];
      const uint32_t total = lf.count;
      c0 = parent_cursors[2 * lf.parent_slot] - lf.begin;
      if (c0 > total) {  // the partition left more rows than the parent holds
        atomicOr(&s_status, (uint32_t)MGB_TREE_STATUS_PARTITION);
        c0 = total;
      }
      c1 = total - c0;
      lbegin = lf.begin;
      lf.count = c0;
      rf.begin = lf.begin + c0;
      rf.count = c1;
      // This level's partition cursors and best-feature keys.
      cursors[4 * p] = lbegin;
      cursors[4 * p + 1] = lbegin + c0;
      cursors[4 * p + 2] = lbegin + c0;
      cursors[4 * p + 3] = lbegin + total;
      for (uint32_t i = 0; i < 2 * kKeyWays; ++i) best[2 * p * kKeyWays + i] = 0;
      built = c0 <= c1 ? 2 * p : 2 * p + 1;
      fr[built].built = 1;
      fr[built ^ 1u].built = 0;
      count = fr[built].count;
      begin = fr[built].begin;
      tiles = div_up(count, t.rows_per_tile);
      zero = tiles != 1;
    }
    uint32_t total_tasks, total_zero, total_rows;
    uint32_t off = block_exclusive_u32(tiles, scan, &total_tasks) + carry_tasks;
    uint32_t zoff = block_exclusive_u32(zero, scan, &total_zero) + carry_zero;
    block_exclusive_u32(count, scan, &total_rows);
    carry_rows += total_rows;
    // Row tiles of this batch's built nodes, written by the whole block.
    s_off[threadIdx.x] = off - carry_tasks;
    s_slot[threadIdx.x] = built;
    s_begin[threadIdx.x] = begin;
    s_end[threadIdx.x] = begin + count;
    __syncthreads();
    const uint32_t nitems = pairs - base < blockDim.x ? pairs - base : blockDim.x;
    if (threadIdx.x == 0 && (uint64_t)carry_tasks + total_tasks > t.max_hist_tasks)
      atomicOr(&s_status, (uint32_t)MGB_TREE_STATUS_TASKS);
    for (uint32_t j = threadIdx.x; j < total_tasks && carry_tasks + j < t.max_hist_tasks; j += blockDim.x) {
      const uint32_t k = owner_of(s_off, nitems, j);
      const uint32_t b = s_begin[k] + (j - s_off[k]) * t.rows_per_tile;
      const uint32_t e = b + t.rows_per_tile < s_end[k] ? b + t.rows_per_tile : s_end[k];
      const uint32_t ntiles = (k + 1 < nitems ? s_off[k + 1] : total_tasks) - s_off[k];
      t.hist_tasks[carry_tasks + j] = HistTask{s_slot[k], b, e, ntiles == 1 ? 1u : 0u};
    }
    if (p < pairs) {
      fr[built].first_task = off;
      fr[built].ntiles = tiles;
    }
    if (zero && zoff < 2 * t.slots) t.zero_list[zoff] = built;
    carry_tasks += total_tasks;
    carry_zero += total_zero;
    // Partition tasks of both children, in slot order.
    const uint32_t pl = p < pairs ? div_up(c0, t.part_tile) : 0, pr = p < pairs ? div_up(c1, t.part_tile) : 0;
    uint32_t total_part;
    const uint32_t poff = block_exclusive_u32(pl + pr, scan, &total_part);
    __syncthreads();
    s_off[threadIdx.x] = poff;
    s_slot[threadIdx.x] = pl;
    s_begin[threadIdx.x] = lbegin;
    s_end[threadIdx.x] = c0;  // left count
    scan_right[threadIdx.x] = c1;
    __syncthreads();
    if (threadIdx.x == 0 && (uint64_t)carry_part + total_part > t.max_part_tasks)
      atomicOr(&s_status, (uint32_t)MGB_TREE_STATUS_TASKS);
    for (uint32_t j = threadIdx.x; j < total_part && carry_part + j < t.max_part_tasks; j += blockDim.x) {
      const uint32_t k = owner_of(s_off, nitems, j);
      const uint32_t q = j - s_off[k];
      const bool left = q < s_slot[k];
      const uint32_t cb = left ? s_begin[k] : s_begin[k] + s_end[k];
      const uint32_t ce = left ? s_begin[k] + s_end[k] : s_begin[k] + s_end[k] + scan_right[k];
      const uint32_t b = cb + (left ? q : q - s_slot[k]) * t.part_tile;
      ptasks[carry_part + j] = PartTask{2 * (base + k) + (left ? 0u : 1u), b, b + t.part_tile < ce ? b + t.part_tile : ce, 0u};
    }
    carry_part += total_part;
    __syncthreads();
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    st->n_part[depth & 1] = carry_part;
    st->n_hist_tasks = carry_tasks;
    st->n_zero = carry_zero;
    if (depth < kMaxLevels) {
      st->rows_built[depth] = carry_rows;
      st->nodes_built[depth] = pairs;
    }
    if (s_status) {  // the tree is refused: this and the deeper levels get no work
      st->error |= s_status;
      if (t.status) atomicOr(t.status, s_status);
      st->n_part[depth & 1] = 0;
      st->n_hist_tasks = 0;
      st->n_zero = 0;
      st->n_nodes = 0;
    }
  }
}

// Single-histogram entry point (mgb_histogram) on a caller's row list: the
// gradient pairs of list 0 in list order (the histogram reads them so).
__global__ void k_gather_pairs(Tree t, uint32_t count) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (uint64_t)gridDim.x * blockDim.x)
    t.gh[0][i] = t.grad[t.rows[0][i]];
}

// Single-histogram entry point (mgb_histogram): sum the row-tile partials of
// a multi-tile node into its histogram slot (the tree's split kernel sums the
// partials of its built nodes itself, see built_pair): entry
// e = f * (max_bin+1) + b of the node adds partial[task][e] over
// the node's tasks (exact integers mod 2^64, so any order gives the same
// bits).  A block takes 64 consecutive entries of one node; its four waves
// take every fourth tile each, four loads in flight per lane, and combine in
// LDS.
constexpr uint32_t kReduceWaves = 4;
__global__ __launch_bounds__(kReduceWaves * kWave) void k_reduce_hist(Tree t, uint32_t depth) {
  __shared__ uint64_t part[kReduceWaves][kWave][2];
  const LevelState* st = t.state;
  const uint32_t n = st->n_zero;
  const uint32_t E = t.cols * t.bins1;
  const uint32_t eblocks = div_up(E, kWave);
  const Frontier* fr = t.frontier[depth & 1];
  int64_t* bank = t.hist[depth & 1];
  const uint64_t stride = (uint64_t)t.groups * t.features_per_group * t.bins1 * 2;  // int64 words per task
  const uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  for (uint32_t blk = blockIdx.x; blk < n * eblocks; blk += gridDim.x) {
    const uint32_t slot = t.zero_list[blk / eblocks];
    const uint32_t e = (blk % eblocks) * kWave + lane;
    const uint32_t first = fr[slot].first_task, ntiles = fr[slot].ntiles;
    uint64_t g = 0, h = 0;
    if (e < E) {
      const int64_t* src = t.partials + (uint64_t)first * stride + (uint64_t)e * 2;
      for (uint32_t k = wave; k < ntiles; k += 4 * kReduceWaves) {
        int4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t kk = k + u * kReduceWaves;
          v[u] = kk < ntiles ? *reinterpret_cast<const int4*>(src + kk * stride) : make_int4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          g += (uint64_t)(uint32_t)v[u].x | ((uint64_t)(uint32_t)v[u].y << 32);
          h += (uint64_t)(uint32_t)v[u].z | ((uint64_t)(uint32_t)v[u].w << 32);
        }
      }
    }
    part[wave][lane][0] = g;
    part[wave][lane][1] = h;
    __syncthreads();
    if (wave == 0 && e < E) {
      for (uint32_t q = 1; q < kReduceWaves; ++q) { g += part[q][lane][0]; h += part[q][lane][1]; }
      int64_t* dst = bank + (uint64_t)slot * E * 2 + (uint64_t)e * 2;
      *reinterpret_cast<int4*>(dst) = make_int4((int)(uint32_t)g, (int)(uint32_t)(g >> 32), (int)(uint32_t)h,
                                                (int)(uint32_t)(h >> 32));
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Histogram build (kernels/boost.metal:700-773, histogram_tiled.metal.h).
// One workgroup owns one (row tile, feature group): an LDS-private
// [max_bin+1 bins][G features] int64 gradient histogram plus a u32 row count
// (unit Hessians) or an int64 Hessian histogram, accumulated with LDS
// integer atomics.  Lanes rotate through the group's features so the 64
// lanes of a wave hit different features at once; with the bin-major,
// feature-minor layout a feature's entries all sit in the same LDS banks, so
// at G = 16 the 64 lanes of an atomic spread exactly evenly over the banks
// whatever the bins are (a feature-major layout leaves the banks to the
// data, about twice the conflict cycles).  Gradients are quantized
// on the fly: q = (int64) rint(g * scale), exactly as a stored int64 pair.
// The flush is a plain store: into the node's histogram when the tile is the
// node's only tile, else into the tile's own partial histogram, which the
// split kernel sums (no device-scope atomics across XCDs).
// ---------------------------------------------------------------------------
template <typename BinT, int G>
struct Codes {
  static constexpr int kBytes = G * (int)sizeof(BinT);
  static constexpr int kWords = (kBytes + 7) / 8;
  uint64_t w[kWords];
  __device__ __forceinline__ void load(const uint8_t* p) {
    if constexpr (kBytes >= 16) {
#pragma unroll
      for (int i = 0; i < kBytes / 16; ++i) {
        uint4 v = reinterpret_cast<const uint4*>(p)[i];
        w[2 * i] = (uint64_t)v.x | ((uint64_t)v.y << 32);
        w[2 * i + 1] = (uint64_t)v.z | ((uint64_t)v.w << 32);
      }
    } else if constexpr (kBytes == 8) {
      uint2 v = *reinterpret_cast<const uint2*>(p);
      w[0] = (uint64_t)v.x | ((uint64_t)v.y << 32);
    } else if constexpr (kBytes == 4) {
      w[0] = *reinterpret_cast<const uint32_t*>(p);
    } else if constexpr (kBytes == 2) {
      w[0] = *reinterpret_cast<const uint16_t*>(p);
    } else {
      w[0] = *p;
    }
  }
  // Codes of G features of one row from the column-major copy (column j at
  // col0 + j * stride).  Only the columns in gmask (the group's features in
  // the tree's column sample) are accumulated; the others read column
  // `other` (one of gmask's, so no extra lines) instead: the loads stay
  // unconditional and the waits exact.
  __device__ __forceinline__ void load_cols(const BinT* col0, uint64_t stride, uint32_t row, uint32_t gmask,
                                            uint32_t other) {
    constexpr uint32_t bits = 8 * sizeof(BinT);
    constexpr uint32_t per_word = 64 / bits;
#pragma unroll
    for (int i = 0; i < kWords; ++i) w[i] = 0;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const uint32_t jj = (gmask >> j) & 1u ? (uint32_t)j : other;
      const uint64_t code = col0[jj * stride + row];
      w[j / per_word] |= code << ((j % per_word) * bits);
    }
  }
  // The G codes rotated by r features: feature (k + r) mod G lands at
  // position k, read with a constant shift.  One rotation per row replaces a
  // lane-dependent select and 64-bit shift per feature: dword moves by the
  // bits of r's dword offset (bit selects under per-lane masks, made once),
  // then a funnel shift.
  static constexpr int kBits = 8 * (int)sizeof(BinT);
  static constexpr int kDwords = (G * kBits + 31) / 32;
  static constexpr int kSteps = kDwords >= 8 ? 3 : kDwords >= 4 ? 2 : kDwords >= 2 ? 1 : 0;
  struct Rotation {
    uint32_t mask[kSteps > 0 ? kSteps : 1];
    uint32_t bits;
  };
  struct Rotated {
    uint32_t d[kDwords];
    __device__ __forceinline__ uint32_t get(int k) const {
      return (d[k * kBits / 32] >> (k * kBits % 32)) & ((1u << kBits) - 1u);
    }
  };
  static __device__ __forceinline__ Rotation rotation(uint32_t r) {
    Rotation m;
    const uint32_t sh = r * kBits;
    m.bits = sh % 32;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      m.mask[s] = ((sh / 32) >> (kSteps - 1 - s)) & 1u ? ~0u : 0u;
      // Kept as a lane value for the bit selects below.
      asm volatile("" : "+v"(m.mask[s]));
    }
    return m;
  }
  __device__ __forceinline__ Rotated rotate(const Rotation& m) const {
    Rotated out;
    if constexpr (G == 1) {
      out.d[0] = (uint32_t)w[0];
    } else if constexpr (G * kBits < 32) {  // 16 bits: u8 codes, G = 2
      const uint32_t x = (uint32_t)w[0] & 0xFFFFu;
      out.d[0] = (x | (x << 16)) >> m.bits;
    } else {
      uint32_t in[kDwords];
#pragma unroll
      for (int i = 0; i < kDwords; ++i) in[i] = (uint32_t)(w[i / 2] >> (32 * (i % 2)));
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
        const int step = 1 << (kSteps - 1 - s);
        uint32_t t[kDwords];
#pragma unroll
        for (int i = 0; i < kDwords; ++i) {
          // v_bfi_b32: (mask & moved) | (~mask & kept), one op per dword.
          asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(t[i]) : "v"(m.mask[s]), "v"(in[(i + step) % kDwords]), "v"(in[i]));
        }
#pragma unroll
        for (int i = 0; i < kDwords; ++i) in[i] = t[i];
      }
#pragma unroll
      for (int i = 0; i < kDwords; ++i) out.d[i] = __builtin_amdgcn_alignbit(in[(i + 1) % kDwords], in[i], m.bits);
    }
    return out;
  }
};

// LDS atomics by byte address (the LDS aperture's 32-bit offsets), so a
// lane's per-feature base address can be kept in a register with the
// dynamic LDS base already added.
typedef __attribute__((address_space(3))) unsigned long long lds_u64_t;
typedef __attribute__((address_space(3))) uint32_t lds_u32_t;
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void lds_add(uint32_t address, unsigned long long v) {
  __hip_atomic_fetch_add((lds_u64_t*)(uintptr_t)address, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_add(uint32_t address, uint32_t v) {
  __hip_atomic_fetch_add((lds_u32_t*)(uintptr_t)address, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Whether a level histogram holds feature f (present: f is one of the
// group's columns): every feature in the tree's column sample, and at the
// root feature 0 as well, whose bins give the root's totals (and a dense
// root's ordered sums) whether or not the tree samples it.
__device__ __forceinline__ bool sampled(const Tree& t, uint32_t f, bool present, bool root) {
  return present && (!t.allowed || t.allowed[f] || (root && f == 0));
}

template <typename BinT, int G, bool UNIT, bool IDENTITY, bool COLS>
__global__ __launch_bounds__(kHistThreads) void k_histogram(Tree t, uint32_t depth) {
  constexpr int kU = kHistUnroll;
  extern __shared__ __align__(16) uint8_t smem[];
  const uint32_t B1 = t.bins1;
  unsigned long long* lg = reinterpret_cast<unsigned long long*>(smem);
  unsigned long long* lh = lg + G * B1;                        // !UNIT
  uint32_t* lc = reinterpret_cast<uint32_t*>(lg + G * B1);     // UNIT
  const LevelState* st = t.state;
  // The root's tasks are its row tiles, computed here (its level-0 set-up
  // may be running in workgroup 0 of this launch).
  const uint32_t ntasks = IDENTITY ? (t.rows_n ? div_up(t.rows_n, t.root_tile) : 0u) : st->n_hist_tasks;
  if (IDENTITY && t.fused_level0 && blockIdx.x == 0) level0_setup(t);
  const uint32_t total = ntasks * t.groups;
  const float sg = t.scales[0], sh = t.scales[1];
  const int64_t unit_q = UNIT ? (int64_t)rintf(1.0f * sh) : 0;
  // XCD-aware schedule: workgroup b runs on XCD b % 8.  Tasks are dealt
  // round-robin over the 8 XCDs and every feature group of a task runs on the
  // task's XCD, so the groups share the task's row lines in that XCD's L2.
  const uint32_t xcd = blockIdx.x % 8, local = blockIdx.x / 8, per_xcd = gridDim.x / 8;
  const uint32_t xcd_tasks = ntasks > xcd ? (ntasks - xcd + 7) / 8 : 0;
  const uint32_t xcd_items = xcd_tasks * t.groups;
  const uint32_t lane = lane_id();
  // Lanes rotate through the group's features: position k of a lane's
  // rotated codes is feature (k + lane) mod G, whose entry of bin b sits at
  // byte fa[k] + b * 8G of lg (and of lh; at fc[k] + b * 4G of lc).
  const typename Codes<BinT, G>::Rotation rot = Codes<BinT, G>::rotation(lane & (G - 1));
  uint32_t fa[G], fc[G];
  uint32_t h_offset = G * B1 * 8;  // lh after lg
  asm volatile("" : "+s"(h_offset));  // one add per entry, not folded into the bin's shift
#pragma unroll
  for (int k = 0; k < G; ++k) {
    const uint32_t j = (k + lane) & (G - 1);
    fa[k] = lds_address(lg + j);
    fc[k] = lds_address(lc + j);
    // Held in registers as computed (else the compiler rebuilds them from j
    // for every row).
    asm volatile("" : "+v"(fa[k]));
    if constexpr (UNIT) asm volatile("" : "+v"(fc[k]));
  }
  const uint32_t entries = G * B1;
  const uint32_t* rows = t.rows[depth & 1];
  int64_t* bank = t.hist[depth & 1];
  const uint8_t* bins = reinterpret_cast<const uint8_t*>(t.bins);
  (void)total;
  for (uint32_t j = local; j < xcd_items; j += per_xcd) {
    const HistTask task = IDENTITY ? root_task(t, xcd + 8 * (j / t.groups)) : t.hist_tasks[xcd + 8 * (j / t.groups)];
    const uint32_t group = j % t.groups;
    const uint32_t fbase = group * G;
    const uint32_t fcount = t.cols - fbase < (uint32_t)G ? t.cols - fbase : (uint32_t)G;
    // The group's features in the tree's column sample (bit k: feature
    // fbase + k; src/tree.cpp:179-180).  The split kernel never scores the
    // others in this tree: the root does not read their columns and no level
    // flushes their bins.  The accumulation still adds every feature of the
    // group (a per-lane feature test costs more vector work than the LDS
    // atomics it saves: 10M x 128 histograms 4.48 -> 4.59 ms per round); the
    // unsampled features' LDS bins are simply never written out.  Uniform
    // over the workgroup.  Only the column loads hold the mask through the
    // row loop (the flush reads the sample again): kept live there it pushes
    // the row-major kernels past 64 VGPRs, one 1024-thread workgroup per CU
    // instead of two (262144 x 64: +0.5 ms per 100 rounds).
    // Without a column sample the mask is the group's width (no loop on the
    // item's critical path ahead of the LDS clear).
    uint32_t gmask = fcount >= 32 ? ~0u : (1u << fcount) - 1u;
    if (t.allowed) {
      gmask = 0;
      for (uint32_t k = 0; k < fcount; ++k) gmask |= sampled(t, fbase + k, true, IDENTITY) ? 1u << k : 0u;
      if (!gmask) continue;
    }
    const uint32_t first_sampled = (uint32_t)__builtin_ctz(gmask);
    for (uint32_t i = threadIdx.x; i < entries; i += blockDim.x) {
      lg[i] = 0;
      if constexpr (UNIT) lc[i] = 0;
      else lh[i] = 0;
    }
    __syncthreads();
    const uint8_t* gbins = bins + (uint64_t)group * t.group_stride;
    const BinT* gcols = COLS ? reinterpret_cast<const BinT*>(t.columns) + (uint64_t)fbase * t.rows_n : nullptr;
    // kU rows per thread per batch, software pipelined: while a batch's LDS
    // atomics run, the next batch's gradients and codes and the row ids of
    // the one after are already in flight, so the waves of the CU (one
    // 1024-thread workgroup when the histogram fills the LDS) keep memory
    // busy instead of alternating between loading and accumulating.  More
    // rows in flight lose: the feature groups' workgroups share each row's
    // code lines through L2, and deeper queues evict them sooner (10M x 128,
    // 1024 bins, histogram per round at 1 / 2 / 3 / 4 / 6 rows per thread:
    // 4.94 / 4.56 / 4.68 / 4.72 / 4.91 ms; two batches of data ahead instead
    // of one at 4 rows: 4.82 ms).
    constexpr uint32_t kStep = kHistThreads * kU;
    // Loads are unconditional (a slot past the task's end reads the task's
    // first row instead and is skipped when accumulating): with no branch
    // around them the compiler waits for exactly the batch it consumes.
    auto fetch_rows = [&](uint32_t base, uint32_t (&row)[kU], bool (&valid)[kU]) {
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const uint32_t i = base + u * kHistThreads + threadIdx.x;
        valid[u] = base < task.end && i < task.end;
        const uint32_t at = valid[u] ? i : task.begin;
        row[u] = IDENTITY ? at : rows[at];
      }
    };
    // Gradient pairs: in row order at an identity root, else from the
    // level's list at the same positions as the row ids (no gather).
    const float2* ghl = IDENTITY ? t.grad : t.gh[depth & 1];
    auto fetch_data = [&](uint32_t base, const uint32_t (&row)[kU], const bool (&valid)[kU],
                          float2 (&gh)[kU], Codes<BinT, G> (&c)[kU]) {
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        gh[u] = ghl[valid[u] ? base + u * kHistThreads + threadIdx.x : task.begin];
        if constexpr (COLS) c[u].load_cols(gcols, t.rows_n, row[u], gmask, first_sampled);
        else c[u].load(gbins + (uint64_t)row[u] * t.row_stride);
      }
    };
    uint32_t row_a[kU], row_b[kU];
    bool valid_a[kU], valid_b[kU];
    float2 gh_a[kU];
    Codes<BinT, G> c_a[kU];
    fetch_rows(task.begin, row_a, valid_a);
    fetch_data(task.begin, row_a, valid_a, gh_a, c_a);
    fetch_rows(task.begin + kStep, row_b, valid_b);
    for (uint32_t base = task.begin; base < task.end; base += kStep) {
      float2 gh_b[kU];
      Codes<BinT, G> c_b[kU];
      fetch_data(base + kStep, row_b, valid_b, gh_b, c_b);
      uint32_t row_c[kU];
      bool valid_c[kU];
      fetch_rows(base + 2 * kStep, row_c, valid_c);
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        if (!valid_a[u]) continue;
        const unsigned long long qg = (unsigned long long)(long long)rintf(gh_a[u].x * sg);
        const unsigned long long qh = UNIT ? 0ull : (unsigned long long)(long long)rintf(gh_a[u].y * sh);
        // A (0, 0) pair adds nothing: the rows a subsample drops, which the
        // root streams with the kept ones, cost no LDS atomics.
        if (!UNIT && (qg | qh) == 0) continue;
        // A present value's code is below max_bin and the missing code
        // (0xFF / 0xFFFF) is not: the minimum sends it to the missing slot.
        const typename Codes<BinT, G>::Rotated rc = c_a[u].rotate(rot);
        if (fcount == (uint32_t)G) {  // full group (uniform): no per-feature test
#pragma unroll
          for (int k = 0; k < G; ++k) {
            const uint32_t bin = min(rc.get(k), t.max_bin);
            const uint32_t a = fa[k] + bin * (8 * G);
            lds_add(a, qg);
            if constexpr (UNIT) lds_add(fc[k] + bin * (4 * G), 1u);
            else lds_add(a + h_offset, qh);
          }
        } else {
#pragma unroll
          for (int k = 0; k < G; ++k) {
            const uint32_t j = (k + lane) & (G - 1);
            const uint32_t bin = min(rc.get(k), t.max_bin);
            if (j < fcount) {
              atomicAdd(&lg[bin * G + j], qg);
              if constexpr (UNIT) atomicAdd(&lc[bin * G + j], 1u);
              else atomicAdd(&lh[bin * G + j], qh);
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        valid_a[u] = valid_b[u];
        gh_a[u] = gh_b[u];
        c_a[u] = c_b[u];
        row_b[u] = row_c[u];
        valid_b[u] = valid_c[u];
      }
    }
    __syncthreads();
    // A node's only tile writes its histogram; tiles of larger nodes write a
    // partial that the split kernel sums (plain stores: no device-scope
    // atomics across XCDs, and the sum is independent of scheduling).
    const uint32_t task_index = xcd + 8 * (j / t.groups);
    int64_t* out = task.single ? bank + ((uint64_t)task.slot * t.cols + fbase) * B1 * 2
                               : t.partials + ((uint64_t)task_index * t.groups + group) * G * B1 * 2;
    // LDS is read in its own (bin-major) order, conflict free; each group of
    // lanes of one feature writes consecutive bins of the feature-major output.
    for (uint32_t i = threadIdx.x; i < entries; i += blockDim.x) {
      const uint32_t bin = i / G, j = i % G;
      if (!sampled(t, fbase + j, fcount > j, IDENTITY)) continue;
      int64_t g = (int64_t)lg[i];
      int64_t h = UNIT ? (int64_t)((uint64_t)lc[i] * (uint64_t)unit_q) : (int64_t)lh[i];
      reinterpret_cast<int4*>(out)[j * B1 + bin] = make_int4((int)(uint32_t)g, (int)(uint32_t)((uint64_t)g >> 32),
                                                             (int)(uint32_t)h, (int)(uint32_t)((uint64_t)h >> 32));
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// CSR histograms (kernels/histogram_csr.metal.h:22-153).  A built node's
// histogram (present entries only: the split kernel derives each feature's
// missing slot from the node total) is cleared, then every row tile of the
// node adds its nonzeros with 64-bit device atomics: the tile's rows are
// flattened into one nonzero index space (block scan of the rows' counts),
// each lane finds its entry's row by binary search over the prefix, and the
// row's fixed-point gradient pair is read from LDS.  Integer adds commute, so
// the result is independent of the order the atomics land in.
// ---------------------------------------------------------------------------
constexpr uint32_t kCsrThreads = 256;

// Root totals over every row (the dense path reads them off a feature's bins
// plus its missing slot; a CSR row may lack any feature).
__global__ __launch_bounds__(kCsrThreads) void k_root_totals(Tree t) {
  __shared__ uint64_t part[kCsrThreads / kWave][2];
  const float sg = t.scales[0], sh = t.scales[1];
  uint64_t g = 0, h = 0;
  for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < t.rows_n; r += (uint64_t)gridDim.x * blockDim.x) {
    const float2 v = t.grad[r];
    g += (uint64_t)(int64_t)rintf(v.x * sg);
    h += (uint64_t)(int64_t)rintf(v.y * sh);
  }
  g = wave_sum_u64(g);
  h = wave_sum_u64(h);
  const uint32_t wave = threadIdx.x / kWave;
  if (lane_id() == 0) { part[wave][0] = g; part[wave][1] = h; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (uint32_t k = 1; k < kCsrThreads / kWave; ++k) { g += part[k][0]; h += part[k][1]; }
    atomicAdd(reinterpret_cast<unsigned long long*>(&t.frontier[0][0].sum_g), (unsigned long long)g);
    atomicAdd(reinterpret_cast<unsigned long long*>(&t.frontier[0][0].sum_h), (unsigned long long)h);
  }
}

// Zero the histogram rows of the level's directly built nodes.
__global__ void k_zero_built(Tree t, uint32_t depth) {
  const uint32_t n = t.state->n_nodes;
  const Frontier* fr = t.frontier[depth & 1];
  int4* bank = reinterpret_cast<int4*>(t.hist[depth & 1]);
  const uint64_t per = (uint64_t)t.cols * t.bins1;  // int4 (g, h) pairs per node
  for (uint32_t slot = blockIdx.y; slot < n; slot += gridDim.y) {
    if (!fr[slot].built) continue;
    int4* row = bank + (uint64_t)slot * per;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < per; i += (uint64_t)gridDim.x * blockDim.x)
      row[i] = make_int4(0, 0, 0, 0);
  }
}

// CSR root histogram from the column-major codes: every row belongs to the
// root, so a workgroup takes up to kRootFeatures consecutive features (as many
// as fit 160 KB of LDS), accumulates
// all their nonzeros in LDS and writes the features' whole bank rows with
// plain stores -- no device atomics, which at the root would all land on one
// node's histogram from every XCD at once.
constexpr uint32_t kRootFeatures = 4;
constexpr uint32_t kRootThreads = 512;
template <typename BinT>
__global__ __launch_bounds__(kRootThreads) void k_histogram_csc_root(Tree t, uint32_t per_group) {
  extern __shared__ __align__(16) uint8_t smem[];
  unsigned long long* lh = reinterpret_cast<unsigned long long*>(smem);  // [feature][bin][g, h]
  const uint32_t B1 = t.bins1;
  const uint32_t f0 = blockIdx.x * per_group;
  const uint32_t nf = t.cols - f0 < per_group ? t.cols - f0 : per_group;
  for (uint32_t i = threadIdx.x; i < per_group * B1 * 2; i += blockDim.x) lh[i] = 0;
  uint64_t bound[kRootFeatures + 1];
#pragma unroll
  for (uint32_t j = 0; j <= kRootFeatures; ++j) bound[j] = t.csc_colptr[f0 + (j < nf ? j : nf)];
  __syncthreads();
  const float sg = t.scales[0], sh = t.scales[1];
  const BinT* codes = reinterpret_cast<const BinT*>(t.csc_codes);
  for (uint64_t i = bound[0] + threadIdx.x; i < bound[nf]; i += blockDim.x) {
    const uint32_t code = codes[i];
    if (code == t.missing_code) continue;
    uint32_t j = 0;
#pragma unroll
    for (uint32_t q = 1; q < kRootFeatures; ++q) j += i >= bound[q] && q < nf ? 1u : 0u;
    const float2 v = t.grad[t.csc_rows[i]];
    unsigned long long* p = lh + ((uint64_t)j * B1 + code) * 2;
    atomicAdd(p, (unsigned long long)(long long)rintf(v.x * sg));
    atomicAdd(p + 1, (unsigned long long)(long long)rintf(v.y * sh));
  }
  __syncthreads();
  int4* out = reinterpret_cast<int4*>(t.hist[0] + (uint64_t)f0 * B1 * 2);
  for (uint32_t k = threadIdx.x; k < nf * B1; k += blockDim.x) {
    const uint64_t g = lh[2 * k], h = lh[2 * k + 1];
    out[k] = make_int4((int)(uint32_t)g, (int)(uint32_t)(g >> 32), (int)(uint32_t)h, (int)(uint32_t)(h >> 32));
  }
}

template <typename BinT, bool IDENTITY>
__global__ __launch_bounds__(kCsrThreads) void k_histogram_csr(Tree t, uint32_t depth) {
  __shared__ uint64_t s_begin[kCsrThreads];
  __shared__ uint32_t s_off[kCsrThreads];
  __shared__ unsigned long long s_qg[kCsrThreads], s_qh[kCsrThreads];
  __shared__ uint32_t scan[kCsrThreads / kWave + 1];
  const uint32_t ntasks = t.state->n_hist_tasks;
  const uint32_t* rows = t.rows[depth & 1];
  int64_t* bank = t.hist[depth & 1];
  const float sg = t.scales[0], sh = t.scales[1];
  const uint32_t B1 = t.bins1;
  const BinT* codes = reinterpret_cast<const BinT*>(t.csr_codes);
  for (uint32_t w = blockIdx.x; w < ntasks; w += gridDim.x) {
    const HistTask task = t.hist_tasks[w];
    unsigned long long* node =
        reinterpret_cast<unsigned long long*>(bank + (uint64_t)task.slot * t.cols * B1 * 2);
    for (uint32_t base = task.begin; base < task.end; base += kCsrThreads) {
      const uint32_t i = base + threadIdx.x;
      uint32_t cnt = 0;
      if (i < task.end) {
        const uint32_t r = IDENTITY ? i : rows[i];
        const uint64_t b = t.csr_indptr[r];
        cnt = (uint32_t)(t.csr_indptr[r + 1] - b);
        s_begin[threadIdx.x] = b;
        const float2 v = IDENTITY ? t.grad[i] : t.gh[depth & 1][i];  // the pair at list position i
        s_qg[threadIdx.x] = (unsigned long long)(long long)rintf(v.x * sg);
        s_qh[threadIdx.x] = (unsigned long long)(long long)rintf(v.y * sh);
      }
      uint32_t total;
      s_off[threadIdx.x] = block_exclusive_u32(cnt, scan, &total);
      __syncthreads();
      const uint32_t nrows = task.end - base < kCsrThreads ? task.end - base : kCsrThreads;
      for (uint32_t j = threadIdx.x; j < total; j += kCsrThreads) {
        const uint32_t q = owner_of(s_off, nrows, j);
        const uint64_t k = s_begin[q] + (j - s_off[q]);
        const uint32_t code = codes[k];
        if (code == t.missing_code) continue;
        unsigned long long* p = node + ((uint64_t)t.csr_indices[k] * B1 + code) * 2;
        atomicAdd(p, s_qg[q]);
        atomicAdd(p + 1, s_qh[q]);
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------
// Split evaluation (kernels/boost.metal:902-1005, scalar_parallel.metal.h).
// One workgroup of W waves per (node pair, feature); wave c takes bins
// [64c, 64c+64) of the feature's [0, count), one bin per lane, so every load
// of the feature is in flight at once.  Each lane subtracts the built child
// from the parent (mod 2^64) and stores the sibling for the next level; wave64
// scans plus the earlier waves' chunk totals (exchanged in LDS) give exact
// int64 prefix sums of both children.  Each lane keeps its best candidate as
// (gain, order, left sums) only; the winner of the workgroup argmax rebuilds
// the full candidate.  Order is b for the forward pass (missing right) and
// 2*count-1-b for the backward pass (missing left): the maximum gain with the
// smallest order is the reference's first strictly greater candidate.  The
// sums over present bins are the node total minus the missing slot (bin
// max_bin), so one pass over the bins suffices below the root.
// ---------------------------------------------------------------------------
struct NodeEval {
  uint64_t tg, th;        // node totals (present + missing)
  uint64_t pg, ph;        // present-bin totals
  double G, H;
  float w, parent_gain;
  float lower, upper;     // monotone bounds of the node's weight
  int32_t mono;           // the item's feature's constraint (-1, 0, 1)
  bool has_missing;
  // This lane's best candidate.
  float best_gain;
  uint32_t best_order;
  uint64_t best_lg, best_lh;
};

__device__ __forceinline__ void node_begin(NodeEval& n, uint64_t tg, uint64_t th, uint64_t mg, uint64_t mh, int eg,
                                           int eh, const MgbSplitParams& p, float lower, float upper, int32_t mono) {
  n.tg = tg; n.th = th;
  n.pg = tg - mg; n.ph = th - mh;
  n.has_missing = mg != 0 || mh != 0;
  n.G = stat_value((int64_t)tg, eg);
  n.H = stat_value((int64_t)th, eh);
  n.lower = lower;
  n.upper = upper;
  n.mono = mono;
  n.w = clamp_weight(calc_weight(n.G, n.H, p), lower, upper);
  n.parent_gain = calc_gain(n.G, n.H, n.w, p);
  n.best_gain = -INFINITY;
  n.best_order = 0xffffffffu;
  n.best_lg = n.best_lh = 0;
}

__device__ __forceinline__ void try_candidate(NodeEval& n, uint64_t lg, uint64_t lh, uint32_t order, int eg, int eh,
                                              float mcw, const MgbSplitParams& p) {
  const uint64_t rg = n.tg - lg, rh = n.th - lh;
  const double GL = stat_value((int64_t)lg, eg), HL = stat_value((int64_t)lh, eh);
  const double GR = stat_value((int64_t)rg, eg), HR = stat_value((int64_t)rh, eh);
  if (!(HL > 0 && HL >= (double)mcw && HR > 0 && HR >= (double)mcw)) return;
  const float lw = clamp_weight(calc_weight(GL, HL, p), n.lower, n.upper);
  const float rw = clamp_weight(calc_weight(GR, HR, p), n.lower, n.upper);
  // A monotone feature's split keeps the left weight at most (increasing) or
  // at least (decreasing) the right one (kernels/boost.metal:909).
  if ((n.mono > 0 && !(lw <= rw)) || (n.mono < 0 && !(lw >= rw))) return;
  const float gain = (calc_gain(GL, HL, lw, p) + calc_gain(GR, HR, rw, p)) - n.parent_gain;
  if (gain > -INFINITY && (gain > n.best_gain || (gain == n.best_gain && order < n.best_order))) {
    n.best_gain = gain;
    n.best_order = order;
    n.best_lg = lg;
    n.best_lh = lh;
  }
}

// The binary32 nearest the binary64 value of a 64-bit integer, times 2^-e:
// both halves convert to binary64 exactly (the high word signed) and one
// fused multiply-add rounds their sum, so the result lies within
// 2^-24 + 2^-53 of the integer's value relatively, whatever its sign (no
// absolute value first: five vector operations against nine).
__device__ __forceinline__ float scaled_f32(uint64_t v, int e) {
  const double d = fma((double)(int32_t)(uint32_t)(v >> 32), 4294967296.0, (double)(uint32_t)v);
  return ldexpf((float)d, -e);
}

// Division-free bounds on a candidate's float gain.  With reg_alpha = 0 and
// max_delta_step = 0 the scorer's child gain is -(2Gw + (H+lambda)w^2) for the
// float weight w = -G/(H+lambda) (1+d), |d| <= 2^-24, which is exactly
// G^2/(H+lambda) (1 - d^2); after the binary64 and float roundings the
// candidate's gain lies within M * 2^-20.2 of the fp32 estimate
// GL^2/(HL+l) + GR^2/(HR+l) - parent, M = the magnitudes summed (fp32
// conversions, reciprocal and products contribute at most 2^-20.6 relative).
// The bounds below use M * 2^-17 + 2^-120, so every candidate whose gain can
// reach the best lower bound of its node is scored exactly; the rest cannot
// be the first strictly greater candidate.  lo = -inf: not certainly valid
// (it takes no part in the node's best lower bound); hi = -inf: certainly
// invalid (Hessian sums not positive or below min_child_weight).
__device__ __forceinline__ void gain_bounds(const NodeEval& n, uint64_t lg, uint64_t lh, int eg, int eh, float mcw,
                                            bool filter, float lambda, float& lo, float& hi) {
  const uint64_t rg = n.tg - lg, rh = n.th - lh;
  lo = -INFINITY;
  hi = -INFINITY;
  if ((int64_t)lh <= 0 || (int64_t)rh <= 0) return;  // HL > 0 or HR > 0 fails (the conversion keeps the sign)
  // hl, hr are within 2^-22 of HL, HR while they stay normal floats.
  const float hl = scaled_f32(lh, eh), hr = scaled_f32(rh, eh);
  constexpr float tol = 0x1p-20f;
  if (mcw > 0x1p-100f && (hl < mcw * (1.0f - tol) || hr < mcw * (1.0f - tol))) return;
  const float need = fmaxf(mcw * (1.0f + tol), 0x1p-100f);
  const bool certain = mcw == 0.0f || (hl >= need && hr >= need);
  hi = INFINITY;
  if (!filter) return;
  // Every operand a normal float away from both ends of the range, so each
  // rounding is relative; otherwise the candidate is scored exactly.
  const float dl = hl + lambda, dr = hr + lambda;
  if (!(dl >= 0x1p-100f && dr >= 0x1p-100f && dl <= 0x1p100f && dr <= 0x1p100f)) return;
  const float gl = scaled_f32(lg, eg), gr = scaled_f32(rg, eg);  // signed: only their squares are used
  if ((gl != 0.0f && fabsf(gl) < 0x1p-50f) || (gr != 0.0f && fabsf(gr) < 0x1p-50f)) return;
  const float al = (gl * gl) * __builtin_amdgcn_rcpf(dl);
  const float ar = (gr * gr) * __builtin_amdgcn_rcpf(dr);
  const float m = (al + ar) + fabsf(n.parent_gain);
  if (!(m <= 0x1p100f)) return;  // huge, infinite or NaN
  const float a = (al + ar) - n.parent_gain;
  const float e = m * 0x1p-17f + 0x1p-120f;
  hi = a + e;
  if (certain) lo = a - e;
}

// Bounds of this lane's forward and backward candidates at bin b (same
// arguments as eval_bin); folds certain lower bounds into best_lo.
__device__ __forceinline__ void bound_bin(const NodeEval& n, uint64_t vg, uint64_t vh, uint64_t lg, uint64_t lh,
                                          uint32_t b, uint32_t count, int eg, int eh, float mcw, bool filter,
                                          float lambda, float& hi_f, float& hi_b, float& best_lo) {
  hi_f = hi_b = -INFINITY;
  if (b >= count) return;
  float lo;
  gain_bounds(n, lg, lh, eg, eh, mcw, filter, lambda, lo, hi_f);
  best_lo = fmaxf(best_lo, lo);
  if (n.has_missing) {
    const uint64_t rg = n.pg - (lg - vg), rh = n.ph - (lh - vh);
    gain_bounds(n, n.tg - rg, n.th - rh, eg, eh, mcw, filter, lambda, lo, hi_b);
    best_lo = fmaxf(best_lo, lo);
  }
}

// Wave maxima as DPP max-scans (the lane moves of wave_inclusive_u32: row_shr
// 1, 2, 4, 8 within each row of 16 lanes, then row_bcast 15 and 31 across
// rows), whose last lane holds the wave's maximum; a lane whose source lies
// outside its row, or a row the broadcast does not write, sees the identity.
// Six DPP moves instead of six LDS permutes.  Call with every lane active.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_move_or(uint32_t v, uint32_t identity) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)v, kCtrl, kRowMask, 0xf, false);
}

template <int kCtrl, int kRowMask>
__device__ __forceinline__ float max_step_f32(float v) {
  const float o = __uint_as_float(dpp_move_or<kCtrl, kRowMask>(__float_as_uint(v), 0xff800000u));  // -inf
  return fmaxf(v, o);
}

__device__ __forceinline__ float wave_max_f32(float v) {
  v = max_step_f32<kRowShr1, 0xf>(v);
  v = max_step_f32<kRowShr2, 0xf>(v);
  v = max_step_f32<kRowShr4, 0xf>(v);
  v = max_step_f32<kRowShr8, 0xf>(v);
  v = max_step_f32<kRowBcast15, 0xa>(v);
  v = max_step_f32<kRowBcast31, 0xc>(v);
  return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), kWave - 1));
}

__device__ __forceinline__ void load_pair(const int64_t* h, uint32_t bin, uint64_t& g, uint64_t& v) {
  const int4 x = *reinterpret_cast<const int4*>(h + 2 * (uint64_t)bin);
  g = (uint64_t)(uint32_t)x.x | ((uint64_t)(uint32_t)x.y << 32);
  v = (uint64_t)(uint32_t)x.z | ((uint64_t)(uint32_t)x.w << 32);
}

__device__ __forceinline__ void store_pair(int64_t* h, uint32_t bin, uint64_t g, uint64_t v) {
  *reinterpret_cast<int4*>(h + 2 * (uint64_t)bin) =
      make_int4((int)(uint32_t)g, (int)(uint32_t)(g >> 32), (int)(uint32_t)v, (int)(uint32_t)(v >> 32));
}

// A wave-uniform 64-bit value moved to scalar registers.
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (uint64_t)lo | ((uint64_t)hi << 32);
}

__device__ __forceinline__ uint64_t lane63_u64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, kWave - 1);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), kWave - 1);
  return (uint64_t)lo | ((uint64_t)hi << 32);
}

template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint64_t max_step_u64(uint64_t v) {
  const uint32_t lo = dpp_move_or<kCtrl, kRowMask>((uint32_t)v, 0u);
  const uint32_t hi = dpp_move_or<kCtrl, kRowMask>((uint32_t)(v >> 32), 0u);
  const uint64_t o = (uint64_t)lo | ((uint64_t)hi << 32);
  return o > v ? o : v;
}

// Unsigned 64-bit wave maximum (identity 0), uniform result.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = max_step_u64<kRowShr1, 0xf>(v);
  v = max_step_u64<kRowShr2, 0xf>(v);
  v = max_step_u64<kRowShr4, 0xf>(v);
  v = max_step_u64<kRowShr8, 0xf>(v);
  v = max_step_u64<kRowBcast15, 0xa>(v);
  v = max_step_u64<kRowBcast31, 0xc>(v);
  return lane63_u64(v);
}

// A lane's best candidate of one node as a key whose maximum is the largest
// gain and, among equal gains, the smallest order; 0 = no candidate.
__device__ __forceinline__ uint64_t candidate_key(const NodeEval& n) {
  if (n.best_order == 0xffffffffu) return 0;
  const uint32_t bits = n.best_gain == 0.0f ? 0u : __float_as_uint(n.best_gain);
  const uint32_t order = bits ^ ((bits & 0x80000000u) ? 0xffffffffu : 0x80000000u);
  return ((uint64_t)order << 32) | (uint64_t)(~n.best_order);
}

// A built node's histogram row for one feature: its bank row, or, for a node
// of several row tiles, the sum of the tiles' partial histograms (exact
// integers mod 2^64, any order), which is then written to the bank row that
// the next level reads as a parent.
struct BuiltHist {
  int64_t* bank;
  const int64_t* part;  // first tile's partial row (several tiles), else null
  uint64_t stride;      // int64 words between consecutive tiles' partials
  uint32_t ntiles;
};

__device__ __forceinline__ BuiltHist built_hist(const Tree& t, int64_t* bank_row, const Frontier& fb, uint32_t f) {
  BuiltHist h;
  h.bank = bank_row;
  h.part = nullptr;
  h.stride = 0;
  h.ntiles = fb.ntiles;
  if (fb.ntiles > 1 && !t.sparse) {
    h.stride = (uint64_t)t.groups * t.features_per_group * t.bins1 * 2;
    h.part = t.partials + (uint64_t)fb.first_task * h.stride + (uint64_t)f * t.bins1 * 2;
  }
  return h;
}

__device__ __forceinline__ void built_pair(const BuiltHist& hb, uint32_t bin, bool store, uint64_t& g, uint64_t& v) {
  if (!hb.part) {
    load_pair(hb.bank, bin, g, v);
    return;
  }
  g = v = 0;
  uint32_t k = 0;
  // Sixteen partial rows in flight per lane, then four: the sum is a chain of
  // dependent loads otherwise (a 32-tile root node).
  for (; k + 16 <= hb.ntiles; k += 16) {
    uint64_t a[16], c[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) load_pair(hb.part + (uint64_t)(k + u) * hb.stride, bin, a[u], c[u]);
#pragma unroll
    for (int u = 0; u < 16; ++u) { g += a[u]; v += c[u]; }
  }
  for (; k + 4 <= hb.ntiles; k += 4) {
    uint64_t a[4], c[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) load_pair(hb.part + (uint64_t)(k + u) * hb.stride, bin, a[u], c[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u) { g += a[u]; v += c[u]; }
  }
  for (; k < hb.ntiles; ++k) {
    uint64_t a, c;
    load_pair(hb.part + (uint64_t)k * hb.stride, bin, a, c);
    g += a;
    v += c;
  }
  if (store) store_pair(hb.bank, bin, g, v);
}

// Bins of one (node pair or root, feature) item held by a lane: inclusive
// in-lane prefix sums of CH consecutive bins.
template <int CH>
struct LaneBins {
  uint64_t g[CH], h[CH];
};

// Exclusive prefix of a lane's bin totals over the item's W waves: the wave
// scan plus (W > 1) the earlier waves' totals exchanged in LDS.  Returns the
// item total in `all`.  Every wave of the block calls it (barrier inside for
// W > 1).
template <int W>
__device__ __forceinline__ void item_prefix(const uint64_t (&tot_lane)[4], uint64_t (&pre)[4], uint64_t (&all)[4],
                                            uint64_t (*xchg)[4], uint32_t wave_in_item) {
  uint64_t inc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    inc[q] = wave_inclusive_u64(tot_lane[q]);
    pre[q] = inc[q] - tot_lane[q];
    all[q] = lane63_u64(inc[q]);
  }
  if constexpr (W > 1) {
    if (lane_id() == 0)
#pragma unroll
      for (int q = 0; q < 4; ++q) xchg[wave_in_item][q] = all[q];
    __syncthreads();
    uint64_t carry[4] = {0, 0, 0, 0}, sum[4] = {0, 0, 0, 0};
    for (uint32_t k = 0; k < (uint32_t)W; ++k) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint64_t v = uniform_u64(xchg[k][q]);
        if (k < wave_in_item) carry[q] += v;
        sum[q] += v;
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) { pre[q] += carry[q]; all[q] = sum[q]; }
  }
}

// Maximum over the item's waves of a per-wave value (W > 1: LDS + barrier).
template <int W>
__device__ __forceinline__ float item_max_f32(float v, float* xchg, uint32_t wave_in_item) {
  v = wave_max_f32(v);
  if constexpr (W > 1) {
    if (lane_id() == 0) xchg[wave_in_item] = v;
    __syncthreads();
    v = xchg[0];
    for (uint32_t k = 1; k < (uint32_t)W; ++k) v = fmaxf(v, xchg[k]);
  }
  return v;
}

// Both children's maxima with one barrier (W > 1).
template <int W>
__device__ __forceinline__ void item_max2_f32(float& a, float& b, float* xa, float* xb, uint32_t wave_in_item) {
  a = wave_max_f32(a);
  b = wave_max_f32(b);
  if constexpr (W > 1) {
    if (lane_id() == 0) { xa[wave_in_item] = a; xb[wave_in_item] = b; }
    __syncthreads();
    a = xa[0];
    b = xb[0];
    for (uint32_t k = 1; k < (uint32_t)W; ++k) { a = fmaxf(a, xa[k]); b = fmaxf(b, xb[k]); }
  }
}

template <int W>
__device__ __forceinline__ void item_max2_u64(uint64_t& a, uint64_t& b, uint64_t* xa, uint64_t* xb,
                                              uint32_t wave_in_item) {
  a = wave_max_u64(a);
  b = wave_max_u64(b);
  if constexpr (W > 1) {
    if (lane_id() == 0) { xa[wave_in_item] = a; xb[wave_in_item] = b; }
    __syncthreads();
    a = uniform_u64(xa[0]);
    b = uniform_u64(xb[0]);
    for (uint32_t k = 1; k < (uint32_t)W; ++k) {
      const uint64_t oa = uniform_u64(xa[k]), ob = uniform_u64(xb[k]);
      a = oa > a ? oa : a;
      b = ob > b ? ob : b;
    }
  }
}

template <int W>
__device__ __forceinline__ uint64_t item_max_u64(uint64_t v, uint64_t* xchg, uint32_t wave_in_item) {
  v = wave_max_u64(v);
  if constexpr (W > 1) {
    if (lane_id() == 0) xchg[wave_in_item] = v;
    __syncthreads();
    v = uniform_u64(xchg[0]);
    for (uint32_t k = 1; k < (uint32_t)W; ++k) {
      const uint64_t o = uniform_u64(xchg[k]);
      v = o > v ? o : v;
    }
  }
  return v;
}

// Division-free upper bounds of the lane's candidates (bin j forward and
// backward) and the lane's best certain lower bound.
template <int CH>
__device__ __forceinline__ void bound_lane(const NodeEval& n, const LaneBins<CH>& lb, uint64_t pre_g, uint64_t pre_h,
                                           uint32_t b0, uint32_t count, int eg, int eh, float mcw, bool filter,
                                           float lambda, float (&hi_f)[CH], float (&hi_b)[CH], float& lo) {
  lo = -INFINITY;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const uint64_t vg = lb.g[j] - (j ? lb.g[j - 1] : 0), vh = lb.h[j] - (j ? lb.h[j - 1] : 0);
    bound_bin(n, vg, vh, pre_g + lb.g[j], pre_h + lb.h[j], b0 + j, count, eg, eh, mcw, filter, lambda, hi_f[j],
              hi_b[j], lo);
  }
}

// The candidates whose upper bound reaches the node's best lower bound, as a
// mask (bit 2j: bin j forward, 2j+1: backward).
template <int CH>
__device__ __forceinline__ uint32_t survivors(const NodeEval& n, const float (&hi_f)[CH], const float (&hi_b)[CH],
                                              float node_lo, uint32_t b0, uint32_t count) {
  uint32_t mask = 0;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    if (b0 + j >= count) continue;
    if (hi_f[j] > -INFINITY && hi_f[j] >= node_lo) mask |= 1u << (2 * j);
    if (n.has_missing && hi_b[j] > -INFINITY && hi_b[j] >= node_lo) mask |= 2u << (2 * j);
  }
  return mask;
}

// Scores the surviving candidates exactly, one at a time.  One inlined copy
// of the binary64 scorer instead of one per bin and direction keeps the
// kernel's code within the instruction cache; the scorer keeps the best by
// (gain, lowest order), so the visiting order does not matter.
template <int CH>
__device__ __forceinline__ void score_survivors(NodeEval& n, const LaneBins<CH>& lb, uint64_t pre_g, uint64_t pre_h,
                                                uint32_t b0, uint32_t count, int eg, int eh, float mcw,
                                                const MgbSplitParams& p, uint32_t mask) {
  while (mask) {
    const uint32_t k = (uint32_t)__builtin_ctz(mask);
    mask &= mask - 1;
    const uint32_t j = k >> 1;
    uint64_t ig = lb.g[0], ih = lb.h[0], xg = 0, xh = 0;  // inclusive / exclusive in-lane prefixes
#pragma unroll
    for (int q = 1; q < CH; ++q) {
      if ((uint32_t)q == j) {
        ig = lb.g[q]; ih = lb.h[q];
        xg = lb.g[q - 1]; xh = lb.h[q - 1];
      }
    }
    const uint32_t b = b0 + j;
    const bool backward = (k & 1) != 0;
    // Backward (missing values go left): the left child is everything but the
    // present rows at or above bin b.
    const uint64_t lg = backward ? n.tg - (n.pg - (pre_g + xg)) : pre_g + ig;
    const uint64_t lh = backward ? n.th - (n.ph - (pre_h + xh)) : pre_h + ih;
    try_candidate(n, lg, lh, backward ? 2 * count - 1 - b : b, eg, eh, mcw, p);
  }
}

// The item's winner (the lane holding the largest key) records its SplitRec
// and offers its feature to the node's best key.
__device__ __forceinline__ void offer_best(const NodeEval& n, uint64_t mine, uint64_t top, SplitRec* rec,
                                           unsigned long long* node_best, uint32_t feature, uint32_t count,
                                           uint32_t cols) {
  if (top != 0 && mine == top) {
    *rec = SplitRec{n.best_gain, n.best_order, (int64_t)n.best_lg, (int64_t)n.best_lh};
    // With many features a node's items serialize on its one key (2,000
    // features: the split 1.59 -> 0.74 ms per round).  The key only grows, so
    // any value read is a lower bound: a key at or below it cannot win and
    // skips the atomic.  With few features the read's round trip costs more
    // than the contention (64 features: 0.125 -> 0.163 ms per round).
    const unsigned long long key = best_key(n.best_gain, feature, n.best_order, count, cols);
    // Few features spread their offers over the node's words; many offer
    // into its first word only, so the value read is the node's best so far
    // (eight words there: 1M x 2000 CSR split 0.74 -> 1.07 ms per round).
    const bool contended = cols >= kContendedFeatures;
    unsigned long long* word = node_best + (contended ? 0u : feature % kKeyWays);
    if (!contended || key > __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
      atomicMax(word, key);
  }
}

// Scores one node's candidates held by this lane (bins b0 .. b0+CH-1,
// in-lane inclusive sums in `lb`, item-exclusive prefix pre_g/pre_h):
// division-free bounds first, then the exact scorer for every candidate whose
// upper bound reaches the node's best certain lower bound.  The winner (if
// any) records its SplitRec and offers its feature to the node's best key.
template <int W, int CH>
__device__ __forceinline__ void score_node(NodeEval& n, const LaneBins<CH>& lb, uint64_t pre_g, uint64_t pre_h, uint32_t b0,
                                           uint32_t count, int eg, int eh, float mcw, bool filter, float lambda,
                                           const MgbSplitParams& p, float* xf, uint64_t* xk, uint32_t wave_in_item,
                                           SplitRec* rec, unsigned long long* node_best, uint32_t feature,
                                           uint32_t cols) {
  float hi_f[CH], hi_b[CH], lo;
  bound_lane<CH>(n, lb, pre_g, pre_h, b0, count, eg, eh, mcw, filter, lambda, hi_f, hi_b, lo);
  const float node_lo = item_max_f32<W>(lo, xf, wave_in_item);
  score_survivors<CH>(n, lb, pre_g, pre_h, b0, count, eg, eh, mcw, p, survivors<CH>(n, hi_f, hi_b, node_lo, b0, count));
  const uint64_t mine = candidate_key(n);
  offer_best(n, mine, item_max_u64<W>(mine, xk, wave_in_item), rec, node_best, feature, count, cols);
}

// Both children of a pair, with one barrier per exchange (W > 1) instead of
// one per child.
template <int W, int CH>
__device__ __forceinline__ void score_pair(NodeEval& na, const LaneBins<CH>& la, uint64_t pga, uint64_t pha,
                                           SplitRec* reca, unsigned long long* besta, NodeEval& nb,
                                           const LaneBins<CH>& lb, uint64_t pgb, uint64_t phb, SplitRec* recb,
                                           unsigned long long* bestb, uint32_t b0, uint32_t count, int eg, int eh,
                                           float mcw, bool filter, float lambda, const MgbSplitParams& p,
                                           float* xfa, float* xfb, uint64_t* xka, uint64_t* xkb,
                                           uint32_t wave_in_item, uint32_t feature, uint32_t cols) {
  float ha_f[CH], ha_b[CH], hb_f[CH], hb_b[CH], loa, lob;
  bound_lane<CH>(na, la, pga, pha, b0, count, eg, eh, mcw, filter, lambda, ha_f, ha_b, loa);
  bound_lane<CH>(nb, lb, pgb, phb, b0, count, eg, eh, mcw, filter, lambda, hb_f, hb_b, lob);
  item_max2_f32<W>(loa, lob, xfa, xfb, wave_in_item);
  score_survivors<CH>(na, la, pga, pha, b0, count, eg, eh, mcw, p, survivors<CH>(na, ha_f, ha_b, loa, b0, count));
  score_survivors<CH>(nb, lb, pgb, phb, b0, count, eg, eh, mcw, p, survivors<CH>(nb, hb_f, hb_b, lob, b0, count));
  const uint64_t minea = candidate_key(na), mineb = candidate_key(nb);
  uint64_t topa = minea, topb = mineb;
  item_max2_u64<W>(topa, topb, xka, xkb, wave_in_item);
  offer_best(na, minea, topa, reca, besta, feature, count, cols);
  offer_best(nb, mineb, topb, recb, bestb, feature, count, cols);
}

// ---------------------------------------------------------------------------
// One item = (node pair, feature) below the root, (feature) at the root, and
// W waves per item with CH consecutive bins per lane, so every bin of the
// feature is in registers at once (W * 64 * CH >= count).  W = 1 packs four
// independent items into a 256-thread block with no barrier; for W > 1 a
// block is one item, so early exits stay block-uniform.  Levels with few
// items spread each over more waves (CH = 1), wide levels use CH = 4.
// ---------------------------------------------------------------------------
template <int W, int CH>
__global__ __launch_bounds__(W == 1 ? kSplitPack * kWave : W * kWave) void k_split(Tree t, uint32_t depth) {
  constexpr uint32_t kItemsPerBlock = W == 1 ? kSplitPack : 1;  // barriers (W > 1) need whole-block items
  __shared__ uint64_t xtot[kItemsPerBlock][W][4];
  __shared__ float xlo[kItemsPerBlock][2][W];
  __shared__ uint64_t xkey[kItemsPerBlock][2][W];
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t slot_in_block = wave / W, wave_in_item = wave % W;
  const uint32_t item = blockIdx.x * kItemsPerBlock + slot_in_block;
  const uint32_t lane = lane_id();
  const LevelState* st = t.state;
  const uint32_t F = t.cols, B1 = t.bins1, MB = t.max_bin;
  const int eg = scale_exponent(t.scales[0]), eh = scale_exponent(t.scales[1]);
  const float mcw = fabsf(t.sp.min_child_weight);
  // The division-free bounds assume unclamped weights and no monotone
  // rejection: with constraints every valid candidate is scored exactly.
  const bool filter = t.sp.reg_alpha == 0.0f && t.sp.max_delta_step == 0.0f && !t.monotone;
  const float lambda = t.sp.reg_lambda;
  int64_t* cur = t.hist[depth & 1];
  const uint32_t b0 = (wave_in_item * kWave + lane) * CH;
  if (depth == 0) {
    if (item >= F) return;  // uniform per item (W > 1: one item per block)
    const uint32_t f = item, count = t.counts[f];
    // A feature outside the tree's column sample has no root histogram (the
    // histogram kernel skips it), except feature 0, whose row is always
    // completed: it gives the root's totals and the select kernel's dense
    // root sums.
    if (f != 0 && t.allowed && !t.allowed[f]) return;
    const BuiltHist hb = built_hist(t, cur + (uint64_t)f * B1 * 2, t.frontier[0][0], f);
    LaneBins<CH> x;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      uint64_t g = 0, v = 0;
      if (b0 + j < count) built_pair(hb, b0 + j, true, g, v);
      x.g[j] = (j ? x.g[j - 1] : 0) + g;
      x.h[j] = (j ? x.h[j - 1] : 0) + v;
    }
    uint64_t mg = 0, mh = 0;
    if (!t.sparse) built_pair(hb, MB, wave_in_item == 0 && lane == 0, mg, mh);
    const uint64_t lt[4] = {x.g[CH - 1], x.h[CH - 1], 0, 0};
    uint64_t pre[4], all[4];
    item_prefix<W>(lt, pre, all, xtot[slot_in_block], wave_in_item);
    uint64_t tg, th;
    if (t.sparse) {
      // CSR: the root totals come from every row (k_root_totals); a feature's
      // missing slot is what its present bins leave of them.
      tg = (uint64_t)t.frontier[0][0].sum_g;
      th = (uint64_t)t.frontier[0][0].sum_h;
      mg = tg - all[0];
      mh = th - all[1];
      if (wave_in_item == 0 && lane == 0) store_pair(hb.bank, MB, mg, mh);
    } else {
      // Root totals: every bin of the feature plus its missing slot.
      tg = all[0] + mg;
      th = all[1] + mh;
      if (f == 0 && wave_in_item == 0 && lane == 0) {
        t.frontier[0][0].sum_g = (int64_t)tg;
        t.frontier[0][0].sum_h = (int64_t)th;
      }
    }
    if (t.allowed && !t.allowed[f]) return;  // outside the tree's column sample
    NodeEval e;
    node_begin(e, tg, th, mg, mh, eg, eh, t.sp, t.frontier[0][0].lower, t.frontier[0][0].upper,
               t.monotone ? t.monotone[f] : 0);
    score_node<W, CH>(e, x, pre[0], pre[1], b0, count, eg, eh, mcw, filter, lambda, t.sp, xlo[slot_in_block][0],
                  xkey[slot_in_block][0], wave_in_item, t.recs + f, best_bank(t, depth), f, t.cols);
    return;
  }
  // The pair's frontier entries are requested before the level's node count,
  // so the two loads overlap instead of forming a chain.  The index is
  // clamped to the level's 2^(depth-1) possible pairs (the grid's last block
  // may run past them); every item kept below has pair < pairs anyway.
  const uint32_t pair = item / F, f = item % F;
  const Frontier* fr = t.frontier[depth & 1];
  const uint32_t pair_ld = min(pair, (1u << (depth - 1)) - 1);
  const Frontier a = fr[2 * pair_ld], b = fr[2 * pair_ld + 1];
  const uint32_t n = st->n_nodes;
  const uint32_t pairs = n / 2;
  if (item >= pairs * F) return;
  if (t.allowed && !t.allowed[f]) return;  // this tree never scores the feature: no sibling either
  const uint32_t built = a.built ? 2 * pair : 2 * pair + 1, other = built ^ 1u;
  const Frontier& fb = a.built ? a : b;
  const Frontier& fo = a.built ? b : a;
  const int64_t* parent = t.hist[(depth - 1) & 1] + ((uint64_t)a.parent_slot * F + f) * B1 * 2;
  int64_t* ob = cur + ((uint64_t)other * F + f) * B1 * 2;
  const bool store_other = depth + 1 < t.max_depth;  // both children are parents at the next level
  const BuiltHist hb = built_hist(t, cur + ((uint64_t)built * F + f) * B1 * 2, fb, f);
  const uint32_t count = t.counts[f];
  // Missing slots: they give each child's present-bin totals.
  uint64_t pmg, pmh, xmg = 0, xmh = 0;
  load_pair(parent, MB, pmg, pmh);
  if (!t.sparse) built_pair(hb, MB, store_other && wave_in_item == 0 && lane == 0, xmg, xmh);
  LaneBins<CH> x, o;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    uint64_t xg = 0, xh = 0, og = 0, oh = 0;
    if (b0 + j < count) {
      uint64_t pg, ph;
      load_pair(parent, b0 + j, pg, ph);
      built_pair(hb, b0 + j, store_other, xg, xh);
      og = pg - xg;
      oh = ph - xh;
      if (store_other) store_pair(ob, b0 + j, og, oh);
    }
    x.g[j] = (j ? x.g[j - 1] : 0) + xg;
    x.h[j] = (j ? x.h[j - 1] : 0) + xh;
    o.g[j] = (j ? o.g[j - 1] : 0) + og;
    o.h[j] = (j ? o.h[j - 1] : 0) + oh;
  }
  const uint64_t lt[4] = {x.g[CH - 1], x.h[CH - 1], o.g[CH - 1], o.h[CH - 1]};
  uint64_t pre[4], all[4];
  item_prefix<W>(lt, pre, all, xtot[slot_in_block], wave_in_item);
  if (t.sparse) {
    // CSR: the built child's missing slot is its total minus its present
    // bins (the sibling's present bins above already subtract to the right
    // values: its present parent bins minus the built child's).
    xmg = (uint64_t)fb.sum_g - all[0];
    xmh = (uint64_t)fb.sum_h - all[1];
    if (store_other && wave_in_item == 0 && lane == 0) store_pair(hb.bank, MB, xmg, xmh);
  }
  const uint64_t omg = pmg - xmg, omh = pmh - xmh;
  if (store_other && wave_in_item == 0 && lane == 0) store_pair(ob, MB, omg, omh);
  NodeEval ex, eo;
  const int32_t mono = t.monotone ? t.monotone[f] : 0;
  node_begin(ex, (uint64_t)fb.sum_g, (uint64_t)fb.sum_h, xmg, xmh, eg, eh, t.sp, fb.lower, fb.upper, mono);
  node_begin(eo, (uint64_t)fo.sum_g, (uint64_t)fo.sum_h, omg, omh, eg, eh, t.sp, fo.lower, fo.upper, mono);
  if constexpr (W > 1 && CH > 1) {
    // Several waves and bins per lane: both children share each exchange's
    // barrier (C4's wide levels: split 1.374 -> 1.352 ms per round).  With
    // one wave per item there is no barrier to share (scored together
    // anyway: C2 unchanged, 1M x 2000 CSR split 0.749 -> 0.784 ms per round),
    // and with one bin per lane the pair's longer live ranges cost more than
    // the barrier saves (C2: 39.2 -> 40.2 ms per fit).
    score_pair<W, CH>(ex, x, pre[0], pre[1], t.recs + (uint64_t)built * F + f,
                      best_bank(t, depth) + built * kKeyWays, eo, o, pre[2], pre[3],
                      t.recs + (uint64_t)other * F + f, best_bank(t, depth) + other * kKeyWays, b0, count, eg, eh,
                      mcw, filter, lambda, t.sp, xlo[slot_in_block][0], xlo[slot_in_block][1], xkey[slot_in_block][0],
                      xkey[slot_in_block][1], wave_in_item, f, t.cols);
  } else {
    score_node<W, CH>(ex, x, pre[0], pre[1], b0, count, eg, eh, mcw, filter, lambda, t.sp, xlo[slot_in_block][0],
                      xkey[slot_in_block][0], wave_in_item, t.recs + (uint64_t)built * F + f,
                      best_bank(t, depth) + built * kKeyWays, f, t.cols);
    score_node<W, CH>(eo, o, pre[2], pre[3], b0, count, eg, eh, mcw, filter, lambda, t.sp, xlo[slot_in_block][1],
                      xkey[slot_in_block][1], wave_in_item, t.recs + (uint64_t)other * F + f,
                      best_bank(t, depth) + other * kKeyWays, f, t.cols);
  }
}

// ---------------------------------------------------------------------------
// Select and apply (kernels/boost.metal:1245-1313 select_splits,
// kernels/scalar_root.metal.h:107-186 dense root, src/tree.cpp:1031-1104
// pop/apply, :1663-1717 replay).  One workgroup handles the whole level in
// node-id order, so child ids follow XGBoost's numbering.
// ---------------------------------------------------------------------------
// Full candidate of a node (totals in n) from its winning feature's record:
// the split kernel's scorer arithmetic for the chosen bin and direction.
__device__ Cand make_cand(const NodeEval& n, const SplitRec& r, uint32_t feature, uint32_t count, const float* cuts_f,
                          int eg, int eh, const MgbSplitParams& p) {
  Cand c;
  c.parent_w = n.w;
  c.total_h = (float)n.H;
  c.padding = 0;
  const uint32_t backward = r.order >= count ? 1u : 0u;
  const uint32_t bin = backward ? 2 * count - 1 - r.order : r.order;
  const uint64_t lg = (uint64_t)r.lg, lh = (uint64_t)r.lh, rg = n.tg - lg, rh = n.th - lh;
  const double GL = stat_value((int64_t)lg, eg), HL = stat_value((int64_t)lh, eh);
  const double GR = stat_value((int64_t)rg, eg), HR = stat_value((int64_t)rh, eh);
  c.gain = r.gain;
  c.feature = (int32_t)feature;
  c.bin = bin;
  c.default_left = backward;
  c.threshold = backward ? (bin == 0 ? -INFINITY : cuts_f[bin - 1]) : cuts_f[bin];
  c.left_w = clamp_weight(calc_weight(GL, HL, p), n.lower, n.upper);
  c.right_w = clamp_weight(calc_weight(GR, HR, p), n.lower, n.upper);
  c.left_h = (float)HL;
  c.right_h = (float)HR;
  c.lg = (int64_t)lg; c.lh = (int64_t)lh; c.rg = (int64_t)rg; c.rh = (int64_t)rh;
  return c;
}

// Serial binary64 sum of `steps` staged values (forward from index 0, or
// backward from count-1), in the reference's order.  Every lane of the
// calling wave runs the same chain (same LDS words: broadcast reads).
__device__ double serial_sum(const double* v, uint32_t steps, bool reverse, uint32_t count) {
  double a = 0;
  if (!reverse) {
#pragma unroll 16
    for (uint32_t s = 0; s < steps; ++s) a += v[s];
  } else {
#pragma unroll 16
    for (uint32_t s = 0; s < steps; ++s) a += v[count - 1 - s];
  }
  return a;
}

// Largest max_bin of the tree kernels: the dense root's select stages 4096 + 1
// bins of two features (147.5 KB of LDS), the split kernel holds 16 waves x
// 64 lanes x 4 bins in registers, and a 2-feature histogram group fits LDS.
constexpr uint32_t kMaxBin = 4096;

// Stage feature f's bins as binary64 statistics: g[b], h[b].
__device__ void stage_feature(const int64_t* fh, uint32_t count, int eg, int eh, double* g, double* h) {
  for (uint32_t b = threadIdx.x; b < count; b += blockDim.x) {
    g[b] = stat_value(fh[2 * b], eg);
    h[b] = stat_value(fh[2 * b + 1], eh);
  }
}

// LDS the select bookkeeping needs at the dense root: feature 0's and the
// chosen feature's bins as binary64 (g, h) and the chosen feature's cuts.
size_t root_stage_bytes(uint32_t bins1) { return 4ull * bins1 * sizeof(double) + (size_t)bins1 * sizeof(float); }

// Whether level `depth`'s bookkeeping plans the next level from the stable
// partition's counts (the host skips k_plan then; same rule on both sides).
__host__ __device__ inline bool counts_plan_level(const Tree& t, uint32_t depth) {
  return !t.select_plans && t.stable && depth < 31 && (1u << depth) <= kPlanNodes;
}

__device__ void select_level(const Tree& t, uint32_t depth, uint8_t* stage) {
  __shared__ uint32_t scan[kPartThreads / kWave + 1];
  __shared__ uint32_t s_off[kPartThreads], s_begin[kPartThreads], s_end[kPartThreads];
  __shared__ uint32_t scan_slot[kPartThreads], s_count[kPartThreads];
  LevelState* st = t.state;
  const uint32_t n = st->n_nodes;
  const uint32_t F = t.cols;
  const Frontier* fr = t.frontier[depth & 1];
  Frontier* next = t.frontier[(depth + 1) & 1];
  const bool final_level = depth + 1 >= t.max_depth;
  // With unit Hessians every row's quantized h is unit_q, so a child's row
  // count is its Hessian sum / unit_q -- exactly the rows the partition will
  // send it -- and the next level can be planned here (k_plan's work) instead
  // of after the partition.  With the stable partition the counting pass has
  // already counted every tile's left rows, whatever the Hessians.
  const bool count_plans = counts_plan_level(t, depth);
  const bool plan_next = (t.select_plans || count_plans) && !final_level;
  const uint64_t unit_q = plan_next ? (uint64_t)(int64_t)rintf(1.0f * t.scales[1]) : 1;
  const uint32_t node_base = st->node_count;
  const int eg = scale_exponent(t.scales[0]), eh = scale_exponent(t.scales[1]);
  const MgbSplitParams& p = t.sp;
  const unsigned long long* best_keys = best_bank(t, depth);
  // Dense root: feature 0 and the chosen feature staged in LDS by all threads
  // so the serial ordered sums below read LDS, not scattered global words.
  // The chosen feature's cuts are staged too: the threshold search below
  // would otherwise be a chain of dependent global loads.
  double* root0g = reinterpret_cast<double*>(stage);
  double* root0h = root0g + t.bins1;
  double* rootfg = root0h + t.bins1;
  double* rootfh = rootfg + t.bins1;
  float* rootcut = reinterpret_cast<float*>(rootfh + t.bins1);
  const bool dense_root = depth == 0 && t.dense && n > 0;
  // Capacities the level's writes must stay within: the node table, the next
  // frontier bank (2 * slots entries), the histogram and partition task lists.
  const uint32_t max_nodes = (2u << t.max_depth) - 1u;
  __shared__ uint32_t s_status;            // MGB_TREE_STATUS_* bits found by this level
  __shared__ uint32_t s_rows_split, s_rows_leaf;
  if (threadIdx.x == 0) s_status = s_rows_split = s_rows_leaf = 0;
  __syncthreads();
  __shared__ uint32_t s_left[kPlanNodes];  // count_plans: each node's left rows
  __shared__ double s_root[4];             // dense root: feature 0's ordered sums, the chosen child's
  __shared__ Frontier s_node;              // dense root: the root's frontier entry,
  __shared__ NodeEval s_ne;                // its totals
  __shared__ Cand s_best;                  // and its best candidate
  if (plan_next && count_plans) {
    // Sums over every task; only split nodes' sums are read (a leaf's tasks
    // keep older counts).
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) s_left[i] = 0;
    __syncthreads();
    const uint32_t ntasks = st->n_part[depth & 1];
    const PartTask* tasks = part_bank(t, depth);
    for (uint32_t w = threadIdx.x; w < ntasks; w += blockDim.x) atomicAdd(&s_left[tasks[w].slot], t.part_left[w]);
    __syncthreads();
  }
  if (dense_root) {
    const uint64_t key = node_key(best_keys);
    const uint32_t f = key ? key_feature(key, F) : 0u;
    const uint32_t cf = t.counts[f];
    stage_feature(t.hist[0], t.counts[0], eg, eh, root0g, root0h);
    stage_feature(t.hist[0] + (uint64_t)f * t.bins1 * 2, cf, eg, eh, rootfg, rootfh);
    for (uint32_t b = threadIdx.x; b < cf; b += blockDim.x) rootcut[b] = t.cuts[(uint64_t)f * t.cut_stride + b];
    __syncthreads();
    // The root's ordered sums (kernels/scalar_root.metal.h:1-105), four
    // serial chains on four waves at once: feature 0's g and h over all its
    // bins (waves 0, 1), and g and h over the chosen child's bin range of the
    // root's best candidate (waves 2, 3; rebuilt here exactly as the node loop
    // below builds it).
    static_assert(kPartThreads >= 4 * kWave, "the root's four sums take four waves");
    const uint32_t chain = threadIdx.x / kWave;
    if (chain < 4) {
      double sum = 0;
      if (chain < 2) {
        sum = serial_sum(chain == 0 ? root0g : root0h, t.counts[0], false, t.counts[0]);
      } else {
        const Frontier node = fr[0];
        NodeEval ne;
        node_begin(ne, (uint64_t)node.sum_g, (uint64_t)node.sum_h, 0, 0, eg, eh, p, node.lower, node.upper, 0);
        Cand best;
        best.feature = -1;
        best.gain = -INFINITY;
        if (key) best = make_cand(ne, t.recs[f], f, cf, t.cuts + (uint64_t)f * t.cut_stride, eg, eh, p);
        if (threadIdx.x == 2 * kWave) {
          s_node = node;
          s_ne = ne;
          s_best = best;
        }
        if (best.feature >= 0 && (uint32_t)best.feature < F) {
          uint32_t lo = 0, hi = cf;
          while (lo < hi) {
            uint32_t mid = lo + (hi - lo) / 2;
            if (rootcut[mid] < best.threshold) lo = mid + 1;
            else hi = mid;
          }
          uint32_t steps = lo + 1 < cf ? lo + 1 : cf;
          if (best.default_left) {
            uint32_t bin = best.threshold == -INFINITY ? 0 : lo + 1;
            steps = bin < cf ? cf - bin : 0;
          }
          sum = serial_sum(chain == 2 ? rootfg : rootfh, steps, best.default_left != 0, cf);
        }
      }
      if (lane_id() == 0) s_root[chain] = sum;
    }
    __syncthreads();
  }
  uint32_t carry_expanded = 0, carry_htasks = 0, carry_zero = 0, carry_rows = 0, carry_ptasks = 0;
  for (uint32_t base = 0; base < n; base += blockDim.x) {
    const uint32_t i = base + threadIdx.x;
    bool valid = i < n;
    Cand best;
    bool expand = false;
    float applied_w = 0, applied_h = 0, parent_w = 0, total_h = 0;
    Frontier node;
    if (valid) {
      if (!dense_root && (fr[i].id < 0 || (uint32_t)fr[i].id >= max_nodes)) {
        atomicOr(&s_status, (uint32_t)MGB_TREE_STATUS_NODE_ID);
        valid = false;  // nothing of this node is written
      }
    }
    if (valid) {
      NodeEval ne;
      if (dense_root) {
        // The root (i = 0): node, totals and candidate as the sums' pre-pass
        // built them.
        node = s_node;
        ne = s_ne;
        best = s_best;
      } else {
        node = fr[i];
        const uint64_t key = node_key(best_keys + (uint64_t)i * kKeyWays);
        node_begin(ne, (uint64_t)node.sum_g, (uint64_t)node.sum_h, 0, 0, eg, eh, p, node.lower, node.upper, 0);
        best.feature = -1;
        best.gain = -INFINITY;
        if (key) {
          const uint32_t f = key_feature(key, F);
          best = make_cand(ne, t.recs[(uint64_t)i * F + f], f, t.counts[f], t.cuts + (uint64_t)f * t.cut_stride, eg,
                           eh, p);
        }
      }
      parent_w = ne.w;
      total_h = (float)ne.H;
      expand = best.feature >= 0 && (uint32_t)best.feature < F && best.gain > 1.0e-6f &&
               best.gain >= p.min_split_loss && depth < t.max_depth;
      if (dense_root) {
        // Dense root: ordered binary64 sums of feature 0's bins, and of the
        // chosen child's bin range (wave 0 took them above).
        const double tg = s_root[0], th = s_root[1];
        parent_w = clamp_weight(calc_weight(tg, th, p), node.lower, node.upper);
        total_h = (float)th;
        if (best.feature >= 0 && (uint32_t)best.feature < F) {
          const double cg = s_root[2], ch = s_root[3];
          double og = tg - cg, oh = th - ch;
          double ag = cg + og, ah = ch + oh;
          applied_w = clamp_weight(calc_weight(ag, ah, p), node.lower, node.upper);
          applied_h = (float)ah;
        }
      } else if (best.feature >= 0) {
        double ag = stat_value(best.lg, eg) + stat_value(best.rg, eg);
        double ah = stat_value(best.lh, eh) + stat_value(best.rh, eh);
        applied_w = clamp_weight(calc_weight(ag, ah, p), node.lower, node.upper);
        applied_h = (float)ah;
      }
    }
    uint32_t total_expanded;
    const uint32_t rank = block_exclusive_u32(expand ? 1u : 0u, scan, &total_expanded) + carry_expanded;
    // Next level's plan (plan_next): the smaller child is built (ties left,
    // kernels/boost.metal:661-698) in row tiles, the other subtracted.
    uint32_t lcount = 0, htiles = 0, hzero = 0, hrows = 0;
    if (plan_next && valid && expand) {
      lcount = count_plans ? s_left[i] : (uint32_t)((uint64_t)best.lh / unit_q);
      if (lcount > node.count) {
        atomicOr(&s_status, (uint32_t)MGB_TREE_STATUS_PARTITION);
        lcount = node.count;
      }
      const uint32_t rcount = node.count - lcount;
      hrows = lcount <= rcount ? lcount : rcount;
      htiles = div_up(hrows, t.rows_per_tile);
      hzero = htiles != 1;
    }
    uint32_t total_htasks = 0, total_zero = 0, total_rows = 0, total_ptasks = 0;
    uint32_t hoff = 0, zoff = 0, poff = 0, pl = 0, pr = 0;
    if (plan_next) {
      hoff = block_exclusive_u32(htiles, scan, &total_htasks) + carry_htasks;
      zoff = block_exclusive_u32(hzero, scan, &total_zero) + carry_zero;
      block_exclusive_u32(hrows, scan, &total_rows);
      if (valid && expand) {
        pl = div_up(lcount, t.part_tile);
        pr = div_up(node.count - lcount, t.part_tile);
      }
      poff = block_exclusive_u32(pl + pr, scan, &total_ptasks);
    }
    if (valid) {
      MgbTreeNode* rec = t.nodes + node.id;
      rec->cover = total_h;
      if (node.id == 0) {
        rec->base_weight = parent_w;
        rec->leaf = parent_w * p.eta;
      }
      if (expand && ((uint64_t)node_base + 2 * rank + 2 > max_nodes || 2 * rank + 2 > 2 * t.slots)) {
        atomicOr(&s_status, (uint32_t)MGB_TREE_STATUS_CAPACITY);
        expand = false;  // the children would lie outside the node table or frontier
      }
      if (expand) {
        const int32_t left = (int32_t)(node_base + 2 * rank), right = left + 1;
        rec->left = left; rec->right = right;
        rec->feature = best.feature;
        rec->threshold = best.threshold;
        rec->default_left = best.default_left;
        rec->gain = best.gain;
        rec->base_weight = applied_w;
        rec->cover = applied_h;
        t.split_bins[node.id] = best.default_left ? (int32_t)best.bin - 1 : (int32_t)best.bin;
        MgbTreeNode l, r;
        l.left = l.right = -1; l.parent = node.id; l.feature = -1; l.threshold = 0;
        l.leaf = best.left_w * p.eta; l.cover = best.left_h; l.gain = 0; l.default_left = 0; l.base_weight = l.leaf;
        r = l;
        r.leaf = best.right_w * p.eta; r.cover = best.right_h; r.base_weight = r.leaf;
        t.nodes[left] = l;
        t.nodes[right] = r;
        if (!final_level) {
          // Both children carry the parent's segment until the next level's
          // plan splits it at the partition's final left cursor.
          Frontier lf, rf;
          lf.id = left; lf.begin = node.begin; lf.count = node.count; lf.parent_slot = i; lf.sum_g = best.lg;
          lf.sum_h = best.lh; lf.built = 0; lf.first_task = 0; lf.ntiles = 0; lf.leaf = l.leaf;
          lf.lower = node.lower; lf.upper = node.upper; lf.padding[0] = lf.padding[1] = 0;
          rf = lf;
          rf.id = right; rf.sum_g = best.rg; rf.sum_h = best.rh; rf.leaf = r.leaf;
          // Children's bounds (src/tree.cpp:1083-1086): the midpoint of the
          // child weights caps the left child from above and the right one
          // from below (increasing), or the reverse (decreasing).
          const int32_t mono = t.monotone ? t.monotone[best.feature] : 0;
          const float middle = (best.left_w + best.right_w) * 0.5f;
          if (mono > 0) {
            if (middle < lf.upper) lf.upper = middle;
            if (rf.lower < middle) rf.lower = middle;
          } else if (mono < 0) {
            if (lf.lower < middle) lf.lower = middle;
            if (middle < rf.upper) rf.upper = middle;
          }
          if (plan_next) {
            lf.count = lcount;
            rf.begin = node.begin + lcount;
            rf.count = node.count - lcount;
            Frontier& b = lcount <= rf.count ? lf : rf;
            b.built = 1;
            b.first_task = hoff;
            b.ntiles = htiles;
            if (hzero && zoff < 2 * t.slots) t.zero_list[zoff] = lcount <= rf.count ? 2 * rank : 2 * rank + 1;
            // The next level's partition cursors and best-feature keys.
            uint32_t* nc = cursor_bank(t, depth + 1);
            nc[4 * rank] = lf.begin;
            nc[4 * rank + 1] = lf.begin + lf.count;
            nc[4 * rank + 2] = rf.begin;
            nc[4 * rank + 3] = rf.begin + rf.count;
            unsigned long long* nb = best_bank(t, depth + 1);
            for (uint32_t k = 0; k < 2 * kKeyWays; ++k) nb[2 * rank * kKeyWays + k] = 0;
          }
          next[2 * rank] = lf;
          next[2 * rank + 1] = rf;
        }
      }
    }
    {
      // The level's rows of splitting and of stopping nodes: wave sums, one
      // LDS atomic per wave.
      const uint32_t split_rows = wave_inclusive_u32(valid && expand ? node.count : 0u);
      const uint32_t leaf_rows = wave_inclusive_u32(valid && !expand ? node.count : 0u);
      if (lane_id() == kWave - 1) {
        if (split_rows) atomicAdd(&s_rows_split, split_rows);
        if (leaf_rows) atomicAdd(&s_rows_leaf, leaf_rows);
      }
    }
    const uint32_t nitems = n - base < blockDim.x ? n - base : blockDim.x;
    if (plan_next) {
      // Row tiles of the next level's built children, in pair order.
      __syncthreads();
      const bool built_left = plan_next && valid && expand && lcount <= node.count - lcount;
      s_off[threadIdx.x] = hoff - carry_htasks;
      s_begin[threadIdx.x] = valid && expand ? (built_left ? node.begin : node.begin + lcount) : 0;
      s_end[threadIdx.x] = s_begin[threadIdx.x] + hrows;
      scan_slot[threadIdx.x] = expand ? 2 * rank + (built_left ? 0u : 1u) : 0u;
      __syncthreads();
      if (threadIdx.x == 0 && ((uint64_t)carry_htasks + total_htasks > t.max_hist_tasks ||
                               (uint64_t)carry_ptasks + total_ptasks > t.max_part_tasks))
        atomicOr(&s_status, (uint32_t)MGB_TREE_STATUS_TASKS);
      for (uint32_t j = threadIdx.x; j < total_htasks && carry_htasks + j < t.max_hist_tasks; j += blockDim.x) {
        const uint32_t k = owner_of(s_off, nitems, j);
        const uint32_t b = s_begin[k] + (j - s_off[k]) * t.rows_per_tile;
        const uint32_t e = b + t.rows_per_tile < s_end[k] ? b + t.rows_per_tile : s_end[k];
        const uint32_t ntiles = (k + 1 < nitems ? s_off[k + 1] : total_htasks) - s_off[k];
        t.hist_tasks[carry_htasks + j] = HistTask{scan_slot[k], b, e, ntiles == 1 ? 1u : 0u};
      }
      // Row tiles of the next level's nodes (both children of each split),
      // for the next level's partition.
      __syncthreads();
      s_off[threadIdx.x] = poff;  // non-decreasing; a node that does not split adds no tiles
      s_begin[threadIdx.x] = valid && expand ? node.begin : 0;
      s_end[threadIdx.x] = lcount;
      s_count[threadIdx.x] = valid && expand ? node.count : 0;
      scan_slot[threadIdx.x] = valid && expand ? 2 * rank : 0u;
      __syncthreads();
      PartTask* ntasks = part_bank(t, depth + 1);
      for (uint32_t j = threadIdx.x; j < total_ptasks && carry_ptasks + j < t.max_part_tasks; j += blockDim.x) {
        const uint32_t k = owner_of(s_off, nitems, j);
        const uint32_t q = j - s_off[k];
        const uint32_t lt = div_up(s_end[k], t.part_tile);
        const bool left = q < lt;
        // The node's rows: [begin, begin + lcount) go left, the rest right.
        const uint32_t nb = s_begin[k];
        const uint32_t cb = left ? nb : nb + s_end[k];
        const uint32_t ce = left ? nb + s_end[k] : nb + s_count[k];
        const uint32_t b = cb + (left ? q : q - lt) * t.part_tile;
        ntasks[carry_ptasks + j] = PartTask{scan_slot[k] + (left ? 0u : 1u), b, b + t.part_tile < ce ? b + t.part_tile : ce, 0u};
      }
      carry_htasks += total_htasks;
      carry_zero += total_zero;
      carry_rows += total_rows;
      carry_ptasks += total_ptasks;
    }
    carry_expanded += total_expanded;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (plan_next) {
      st->n_hist_tasks = carry_htasks;
      st->n_zero = carry_zero;
      st->n_part[(depth + 1) & 1] = carry_ptasks;
      if (depth + 1 < kMaxLevels) {
        st->rows_built[depth + 1] = carry_rows;
        st->nodes_built[depth + 1] = carry_expanded;
      }
    }
    st->node_count = node_base + 2 * carry_expanded;
    st->n_nodes = final_level ? 0 : 2 * carry_expanded;  // becomes the next level's frontier size
    if (t.node_count_out) *t.node_count_out = node_base + 2 * carry_expanded;
    if (depth < kMaxLevels) {
      st->rows_split[depth] = s_rows_split;
      st->rows_leaf[depth] = s_rows_leaf;
    }
    if (s_status) {
      // The tree is refused; the deeper levels get no work (the reference's
      // driver returns early once its error word is set).
      st->error |= s_status;
      if (t.status) atomicOr(t.status, s_status);
      st->n_nodes = 0;
      st->n_hist_tasks = 0;
      st->n_zero = 0;
      st->n_part[(depth + 1) & 1] = 0;
    }
  }
}

// ---------------------------------------------------------------------------
// Row partition (kernels/boost.metal:1316-1614): ballot + prefix scatter,
// stable within a tile of part_tile rows; tiles of one node claim their
// ranges in arrival order.  value < threshold <=> bin <= last_left_bin; missing follows
// default_left.  Rows of nodes that stop here get their leaf added to the
// training margin (prediction cache, kernels/boost.metal:1738-1763).
// ---------------------------------------------------------------------------
template <typename BinT>
__device__ __forceinline__ bool goes_left(const Tree& t, const NodeOp& op, uint32_t row) {
  uint32_t code;
  if (t.csr_indptr) {
    // CSR: binary search of the split feature among the row's sorted columns;
    // an absent entry is missing.
    uint64_t lo = t.csr_indptr[row], hi = t.csr_indptr[row + 1];
    const uint64_t end = hi;
    while (lo < hi) {
      const uint64_t mid = lo + (hi - lo) / 2;
      if (t.csr_indices[mid] < op.feature) lo = mid + 1;
      else hi = mid;
    }
    if (lo == end || t.csr_indices[lo] != op.feature) return op.default_left != 0;
    code = reinterpret_cast<const BinT*>(t.csr_codes)[lo];
  } else if (t.columns) {
    code = reinterpret_cast<const BinT*>(t.columns)[(uint64_t)op.feature * t.rows_n + row];
  } else {
    const uint32_t G = t.features_per_group;
    const BinT* codes = reinterpret_cast<const BinT*>(reinterpret_cast<const uint8_t*>(t.bins) +
                                                      (uint64_t)(op.feature / G) * t.group_stride +
                                                      (uint64_t)row * t.row_stride);
    code = codes[op.feature % G];
  }
  if (code == t.missing_code) return op.default_left != 0;
  return (int32_t)code <= op.last_left_bin;
}


// Row ids of a partition tile for this thread (positions begin + k*256 + tid).
template <bool IDENTITY, int PER>
__device__ __forceinline__ void load_tile_rows(const uint32_t* rows, const PartTask& task, uint32_t (&row)[PER],
                                               bool (&active)[PER]) {
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const uint32_t i = task.begin + k * kPartThreads + threadIdx.x;
    active[k] = i < task.end;
    row[k] = active[k] ? (IDENTITY ? i : rows[i]) : 0u;
  }
}

// The partition's view of one node of the level: whether it splits, on
// which bin and direction, and the leaf values -- the select arithmetic for
// this node alone (no other node's result is needed), so every workgroup of
// the node computes the same bits the bookkeeping workgroup writes into the
// tree.
__device__ NodeOp node_op(const Tree& t, uint32_t depth, uint32_t slot) {
  const Frontier node = t.frontier[depth & 1][slot];
  const uint64_t key = node_key(best_bank(t, depth) + (uint64_t)slot * kKeyWays);
  const MgbSplitParams& p = t.sp;
  if (key && depth + 1 < t.max_depth && t.cols <= kKeyFeatures) {
    // A split above the last level only moves rows, by the feature, bin and
    // direction the key carries: no record load, no candidate rebuilt.  The
    // expansion test is the one below on the same gain.
    const float gain = key_gain(key);
    const uint32_t f = key_feature(key, t.cols);
    if (f < t.cols && gain > 1.0e-6f && gain >= p.min_split_loss) {
      const uint32_t bin = (uint32_t)key & 0x7fffu, backward = ((uint32_t)key >> 15) & 1u;
      NodeOp op;
      op.op = kOpSplit;
      op.feature = f;
      op.last_left_bin = backward ? (int32_t)bin - 1 : (int32_t)bin;
      op.default_left = backward;
      op.leaf = node.leaf; op.left_leaf = 0; op.right_leaf = 0; op.child_slot = 0;
      return op;
    }
  }
  const int eg = scale_exponent(t.scales[0]), eh = scale_exponent(t.scales[1]);
  NodeEval ne;
  node_begin(ne, (uint64_t)node.sum_g, (uint64_t)node.sum_h, 0, 0, eg, eh, p, node.lower, node.upper, 0);
  Cand best;
  best.feature = -1;
  best.gain = -INFINITY;
  if (key) {
    const uint32_t f = key_feature(key, t.cols);
    best = make_cand(ne, t.recs[(uint64_t)slot * t.cols + f], f, t.counts[f], t.cuts + (uint64_t)f * t.cut_stride,
                     eg, eh, p);
  }
  const bool expand = best.feature >= 0 && (uint32_t)best.feature < t.cols && best.gain > 1.0e-6f &&
                      best.gain >= p.min_split_loss && depth < t.max_depth;
  NodeOp op;
  op.feature = 0; op.last_left_bin = -1; op.default_left = 0;
  op.leaf = node.leaf; op.left_leaf = 0; op.right_leaf = 0; op.child_slot = 0;
  if (!expand) {
    op.op = kOpLeaf;
    if (node.id == 0) {
      // A root that does not split: its weight, from the dense root's ordered
      // binary64 sums of feature 0's bins when the matrix has no missing
      // value (the same sums the bookkeeping workgroup stages in LDS).
      float parent_w = ne.w;
      if (t.dense) {
        const int64_t* h0 = t.hist[0];
        double tg = 0, th = 0;
        for (uint32_t b = 0; b < t.counts[0]; ++b) {
          tg += stat_value(h0[2 * b], eg);
          th += stat_value(h0[2 * b + 1], eh);
        }
        parent_w = clamp_weight(calc_weight(tg, th, p), node.lower, node.upper);
      }
      op.leaf = parent_w * p.eta;
    }
    return op;
  }
  op.op = depth + 1 >= t.max_depth ? kOpFinal : kOpSplit;
  op.feature = (uint32_t)best.feature;
  op.last_left_bin = best.default_left ? (int32_t)best.bin - 1 : (int32_t)best.bin;
  op.default_left = best.default_left;
  op.left_leaf = best.left_w * p.eta;
  op.right_leaf = best.right_w * p.eta;
  return op;
}

// Stable partition, first pass: every tile of a splitting node keeps its
// rows' directions (one wave64 ballot mask per (chunk, wave), in row-list
// order) and its left count.  k_apply then takes a tile's positions from the
// counts of its node's tiles -- left rows from begin + (left rows of earlier
// tiles), right rows from begin + L + (right rows of earlier tiles) -- so
// each child keeps the parent's row order (kernels/boost.metal:1550-1614).
// No workgroup waits for or signals another: the counts cross to k_apply
// at the kernel boundary.
template <typename BinT, bool IDENTITY, int PER>
__global__ __launch_bounds__(kPartThreads) void k_part_count(Tree t, uint32_t depth) {
  constexpr uint32_t kWaves = kPartThreads / kWave;
  constexpr int kPartPer = PER;                      // rows per thread, all loaded up front
  constexpr uint32_t kPartMasks = PER * kWaves;      // wave64 ballot masks per tile
  __shared__ uint32_t wave_left[kPartMasks];
  const LevelState* st = t.state;
  const uint32_t ntasks = st->n_part[depth & 1];
  const PartTask* tasks = part_bank(t, depth);
  const uint32_t* rows = t.rows[depth & 1];
  const uint32_t lane = lane_id(), wave = threadIdx.x / kWave;
  uint32_t op_slot = 0xffffffffu;
  NodeOp op;
  for (uint32_t w = blockIdx.x; w < ntasks; w += gridDim.x) {
    const PartTask task = tasks[w];
    uint32_t row[kPartPer];
    bool active[kPartPer];
    load_tile_rows<IDENTITY, kPartPer>(rows, task, row, active);
    if (task.slot != op_slot) {  // uniform: every thread read the same task
      op = node_op(t, depth, task.slot);
      op_slot = task.slot;
    }
    if (op.op != kOpSplit) continue;  // leaves and the last level move no rows
#pragma unroll
    for (int k = 0; k < kPartPer; ++k) {
      const uint64_t m = __ballot(active[k] && goes_left<BinT>(t, op, row[k]));
      if (lane == 0) {
        t.part_masks[(uint64_t)w * kPartMasks + k * kWaves + wave] = m;
        wave_left[k * kWaves + wave] = (uint32_t)__popcll(m);
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t left = 0;
      for (uint32_t q = 0; q < kPartMasks; ++q) left += wave_left[q];
      t.part_left[w] = left;
    }
    __syncthreads();  // wave_left is reused by the next task
  }
}

// The last level's margin updates, ordered by row range.  A node's rows are
// in row order (stable partition), so its tile q of T covers about the
// (q + 1/2)/T fraction of the row range; every node of the level spans all
// of it.  In node order, the workgroups resident at one time update margins
// of rows spread over the whole range, and each margin line (32 rows, from
// many nodes) is fetched and written back once per node that touches it.
// Here one workgroup sorts the level's tasks by that fraction (64 buckets,
// counting sort) and splits the order into 8 contiguous row ranges, one per
// XCD: the apply kernel's workgroups on an XCD take that XCD's list in
// order, so the margin lines in flight fit the XCD's L2.  The order only
// changes which workgroup updates which rows, and when.
constexpr uint32_t kOrderBuckets = 64;
constexpr uint32_t kOrderThreads = 1024;
__device__ __forceinline__ uint32_t order_bucket(const PartTask& task, const Frontier& node, uint32_t part_tile) {
  const uint32_t tiles = div_up(node.count, part_tile);
  const uint32_t q = (task.begin - node.begin) / part_tile;
  return (uint32_t)(((2ull * q + 1) * kOrderBuckets) / (2ull * tiles));
}
__global__ __launch_bounds__(kOrderThreads) void k_final_order(Tree t, uint32_t depth) {
  __shared__ uint32_t count[kOrderBuckets];
  const uint32_t ntasks = t.state->n_part[depth & 1];
  const PartTask* tasks = part_bank(t, depth);
  const Frontier* frontier = t.frontier[depth & 1];
  uint32_t* offsets = t.final_order + t.max_part_tasks;  // XCD x: [offsets[x], offsets[x + 1])
  if (threadIdx.x < kOrderBuckets) count[threadIdx.x] = 0;
  __syncthreads();
  for (uint32_t w = threadIdx.x; w < ntasks; w += blockDim.x) {
    const PartTask task = tasks[w];
    atomicAdd(&count[order_bucket(task, frontier[task.slot], t.part_tile)], 1u);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t pos = 0;
    for (uint32_t b = 0; b < kOrderBuckets; ++b) {
      if (b % (kOrderBuckets / 8) == 0) offsets[b / (kOrderBuckets / 8)] = pos;
      const uint32_t c = count[b];
      count[b] = pos;
      pos += c;
    }
    offsets[8] = pos;
  }
  __syncthreads();
  for (uint32_t w = threadIdx.x; w < ntasks; w += blockDim.x) {
    const PartTask task = tasks[w];
    t.final_order[atomicAdd(&count[order_bucket(task, frontier[task.slot], t.part_tile)], 1u)] = w;
  }
}

// Select and partition of one level in one launch.  The last workgroup does
// the level's bookkeeping (select_level: tree records, the next frontier, and
// with unit Hessians the next level's plan); every other workgroup takes
// partition tiles of up to part_tile rows of one node, works out that node's
// split itself (node_op), and moves its rows: a split node's left rows fill
// its segment upwards from the start and its right rows downwards from the
// end, each tile claiming both ranges with one 64-bit atomic on the node's
// two adjacent cursor words and writing ranks (chunk, wave, lane) into them.  The order of
// rows inside a child depends on which tile claims first; nothing downstream
// depends on it (histograms are exact integer sums and the margin update is
// per row).  STABLE: the tile's directions and positions come from
// k_part_count instead, and each child keeps the parent's row order.  Rows of
// nodes that stop here get their leaf added to the training margin.
template <typename BinT, bool IDENTITY, bool STABLE, int PER>
__global__ __launch_bounds__(kPartThreads) void k_apply(Tree t, uint32_t depth) {
  extern __shared__ __align__(16) uint8_t apply_stage[];  // dense-root staging (depth 0 only)
  if (blockIdx.x == gridDim.x - 1) {
    select_level(t, depth, apply_stage);
    return;
  }
  constexpr uint32_t kWaves = kPartThreads / kWave;
  constexpr uint32_t kPartTile = PER * kPartThreads;
  constexpr int kPartPer = PER;                      // rows per thread, all loaded up front
  constexpr uint32_t kPartMasks = PER * kWaves;      // wave64 ballot masks per tile
  __shared__ uint32_t wave_left[kPartPer][kWaves], wave_active[kPartPer][kWaves];
  __shared__ uint32_t wave_before[kWaves], wave_all[kWaves];  // STABLE: the node's tile counts
  __shared__ uint32_t base_left, base_right;
  const LevelState* st = t.state;
  const uint32_t ntasks = st->n_part[depth & 1];
  const PartTask* tasks = part_bank(t, depth);
  const Frontier* frontier = t.frontier[depth & 1];
  uint32_t* cursors = cursor_bank(t, depth);
  const uint32_t* rows = t.rows[depth & 1];
  uint32_t* out = t.rows[(depth + 1) & 1];
  const float2* gh_in = IDENTITY ? t.grad : t.gh[depth & 1];
  float2* gh_out = t.gh[(depth + 1) & 1];
  const uint32_t lane = lane_id(), wave = threadIdx.x / kWave;
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
  uint32_t op_slot = 0xffffffffu;
  NodeOp op;
  // The last level of a stable partition takes its tasks by row range, XCD
  // by XCD (k_final_order), when every XCD has a partition workgroup; other
  // levels, and grids of fewer than 8 partition workgroups, in task order.
  const bool ordered = STABLE && depth + 1 >= t.max_depth && gridDim.x - 1 >= 8;
  const uint32_t xcd = blockIdx.x % 8;
  const uint32_t first = ordered ? t.final_order[t.max_part_tasks + xcd] + blockIdx.x / 8 : blockIdx.x;
  const uint32_t last = ordered ? t.final_order[t.max_part_tasks + xcd + 1] : ntasks;
  const uint32_t stride = ordered ? (gridDim.x - 1 - xcd + 7) / 8 : gridDim.x - 1;
  for (uint32_t i = first; i < last; i += stride) {
    const uint32_t w = ordered ? t.final_order[i] : i;
    const PartTask task = tasks[w];
    // The tile's row ids are requested first; every thread then rebuilds the
    // node's split itself (uniform loads, no barrier), so the two chains of
    // loads overlap.
    uint32_t row[kPartPer];
    bool active[kPartPer];
    load_tile_rows<IDENTITY, kPartPer>(rows, task, row, active);
    if (task.slot != op_slot) {  // uniform: every thread read the same task
      op = node_op(t, depth, task.slot);
      op_slot = task.slot;
    }
    if (op.op == kOpLeaf) {
#pragma unroll
      for (int k = 0; k < kPartPer; ++k)
        if (active[k]) t.margin[row[k]] = t.margin[row[k]] + op.leaf;
      continue;
    }
    bool flag[kPartPer];
    if (STABLE && op.op == kOpSplit) {
      const uint64_t* masks = t.part_masks + (uint64_t)w * kPartMasks + wave;
#pragma unroll
      for (int k = 0; k < kPartPer; ++k) flag[k] = (masks[k * kWaves] >> lane) & 1u;
    } else {
#pragma unroll
      for (int k = 0; k < kPartPer; ++k) flag[k] = active[k] && goes_left<BinT>(t, op, row[k]);
    }
    if (op.op == kOpFinal) {
#pragma unroll
      for (int k = 0; k < kPartPer; ++k)
        if (active[k]) t.margin[row[k]] = t.margin[row[k]] + (flag[k] ? op.left_leaf : op.right_leaf);
      continue;
    }
    // Each moved row takes its gradient pair along (same positions as its id).
    float2 gh[kPartPer];
#pragma unroll
    for (int k = 0; k < kPartPer; ++k)
      gh[k] = gh_in[task.begin + k * kPartThreads + threadIdx.x < task.end ? task.begin + k * kPartThreads + threadIdx.x
                                                                           : task.begin];
    uint32_t node_begin = 0, tile = 0;
    if (STABLE) {
      // Left rows of the node's tiles before this one, and of all of them (L).
      node_begin = frontier[task.slot].begin;
      const uint32_t ntiles = div_up(frontier[task.slot].count, kPartTile);
      tile = (task.begin - node_begin) / kPartTile;
      const uint32_t* left = t.part_left + (w - tile);
      uint32_t before = 0, all = 0;
      for (uint32_t i = threadIdx.x; i < ntiles; i += kPartThreads) {
        const uint32_t c = left[i];
        all += c;
        if (i < tile) before += c;
      }
#pragma unroll
      for (int d = kWave / 2; d > 0; d >>= 1) {
        before += __shfl_xor(before, d, kWave);
        all += __shfl_xor(all, d, kWave);
      }
      if (lane == 0) { wave_before[wave] = before; wave_all[wave] = all; }
    }
    uint32_t lrank[kPartPer], arank[kPartPer];
#pragma unroll
    for (int k = 0; k < kPartPer; ++k) {
      const uint64_t lmask = __ballot(flag[k]);
      const uint64_t amask = __ballot(active[k]);
      lrank[k] = (uint32_t)__popcll(lmask & below);
      arank[k] = (uint32_t)__popcll(amask & below);
      if (lane == 0) {
        wave_left[k][wave] = (uint32_t)__popcll(lmask);
        wave_active[k][wave] = (uint32_t)__popcll(amask);
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      if (STABLE) {
        // The node's earlier tiles hold task.begin - node_begin rows, `before`
        // of them left; right rows start after all L left rows.
        uint32_t before = 0, all = 0;
        for (uint32_t q = 0; q < kWaves; ++q) { before += wave_before[q]; all += wave_all[q]; }
        base_left = node_begin + before;
        base_right = node_begin + all + (task.begin - node_begin - before);
        if (tile == 0) cursors[2 * task.slot] = node_begin + all;  // the final left cursor, for k_plan
      } else {
        uint32_t tl = 0, ta = 0;
        for (int k = 0; k < kPartPer; ++k)
          for (uint32_t q = 0; q < kWaves; ++q) { tl += wave_left[k][q]; ta += wave_active[k][q]; }
        // Both cursors (left: low word, rising from the node's start; right:
        // high word, falling from its end) in one 64-bit atomic: the low word
        // never carries (it stays below the node's end), and adding
        // (2^32 - right rows) << 32 subtracts them from the high word.
        const uint32_t tr = ta - tl;
        const unsigned long long old =
            atomicAdd(reinterpret_cast<unsigned long long*>(&cursors[2 * task.slot]),
                      (unsigned long long)tl | ((unsigned long long)(0u - tr) << 32));
        base_left = (uint32_t)old;
        base_right = (uint32_t)(old >> 32) - tr;
      }
    }
    __syncthreads();
    uint32_t done_left = 0, done_active = 0;  // rows of earlier chunks
#pragma unroll
    for (int k = 0; k < kPartPer; ++k) {
      uint32_t wl = 0, wa = 0, cl = 0, ca = 0;
      for (uint32_t q = 0; q < kWaves; ++q) {
        const uint32_t l = wave_left[k][q], a = wave_active[k][q];
        if (q < wave) { wl += l; wa += a; }
        cl += l; ca += a;
      }
      if (active[k]) {
        const uint32_t at = flag[k] ? base_left + done_left + wl + lrank[k]
                                    : base_right + (done_active - done_left) + (wa - wl) + (arank[k] - lrank[k]);
        out[at] = row[k];
        gh_out[at] = gh[k];
      }
      done_left += cl;
      done_active += ca;
    }
    __syncthreads();
  }
}

// Margin update of the rows a compaction dropped (stored at the end of the
// row list): each walks the finished tree from the root on its codes, the
// partition's test at every split (goes_left with the split's last left bin),
// and adds its leaf's value -- the value the partition adds to the rows it
// moves (kernels/boost.metal:1738-1763).  kWalkPer rows per thread walk
// side by side, so their dependent loads overlap.
constexpr int kWalkPer = 4;
template <typename BinT>
__global__ __launch_bounds__(kCompactThreads) void k_walk_dropped(Tree t) {
  const uint32_t dropped = t.state->dropped;
  const MgbTreeNode* nodes = t.nodes;
  constexpr uint32_t kStep = kCompactThreads * kWalkPer;
  for (uint32_t base = blockIdx.x * kStep; base < dropped; base += gridDim.x * kStep) {
    uint32_t row[kWalkPer];
    int32_t at[kWalkPer];
    bool active[kWalkPer];
#pragma unroll
    for (int k = 0; k < kWalkPer; ++k) {
      const uint32_t j = base + k * kCompactThreads + threadIdx.x;
      active[k] = j < dropped;
      row[k] = active[k] ? t.rows[0][t.rows_n - 1 - j] : 0u;
      at[k] = 0;
    }
    // A tree of depth max_depth reaches a leaf in at most max_depth steps.
    for (uint32_t d = 0; d < t.max_depth; ++d) {
#pragma unroll
      for (int k = 0; k < kWalkPer; ++k) {
        if (!active[k]) continue;
        const MgbTreeNode n = nodes[at[k]];
        if (n.left < 0) continue;
        NodeOp op;
        op.op = kOpSplit;
        op.feature = (uint32_t)n.feature;
        op.last_left_bin = t.split_bins[at[k]];
        op.default_left = n.default_left;
        op.leaf = op.left_leaf = op.right_leaf = 0.0f;
        op.child_slot = 0;
        at[k] = goes_left<BinT>(t, op, row[k]) ? n.left : n.right;
      }
    }
#pragma unroll
    for (int k = 0; k < kWalkPer; ++k)
      if (active[k]) t.margin[row[k]] = t.margin[row[k]] + nodes[at[k]].leaf;
  }
}

// ---------------------------------------------------------------------------
// Host side: workspace layout and the per-level launch sequence.
// ---------------------------------------------------------------------------
// Rows per partition task: 2048 for the stable partition of a dense matrix
// of at least 2^21 rows (10M x 128: partition 1.66 -> 1.55 ms per round
// against 1024), else 1024 -- smaller matrices need the narrower tasks to put
// a workgroup on every CU (262,144 rows: 128 tasks of 2048 rows a level).
uint32_t partition_tile(bool stable, bool sparse, uint32_t rows) {
  return stable && !sparse && rows >= (1u << 21) ? kPartTileWide : kPartTileNarrow;
}

struct Layout {
  size_t state, rows, gh, hist, frontier, recs, best, hist_tasks, zero, part_tasks, cursors, split_bins, partials;
  size_t part_masks, part_left, final_order, total;
  uint32_t slots, max_hist_tasks, max_part_tasks;
  uint64_t hist_entry;
};

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

Layout layout(const MgbTreeShape& s) {
  Layout L;
  uint32_t depth = s.max_depth ? s.max_depth : 1;
  L.slots = 1u << (depth - 1);
  L.hist_entry = (uint64_t)s.cols * (s.max_bin + 1) * 2;
  L.max_hist_tasks = div_up(s.rows ? s.rows : 1, s.rows_per_tile) + L.slots + 1;
  const uint32_t part_tile = partition_tile(s.stable_partition != 0, s.sparse != 0, s.rows);
  L.max_part_tasks = div_up(s.rows ? s.rows : 1, part_tile) + 2 * L.slots + 1;
  size_t off = 0;
  L.state = off; off = align_up(off + sizeof(LevelState));
  L.rows = off; off = align_up(off + 2 * (size_t)s.rows * sizeof(uint32_t));
  L.gh = off; off = align_up(off + 2 * (size_t)s.rows * sizeof(float2));
  L.hist = off; off = align_up(off + 2 * (size_t)L.slots * L.hist_entry * sizeof(int64_t));
  L.frontier = off; off = align_up(off + 2 * (size_t)(2 * L.slots) * sizeof(Frontier));
  L.recs = off; off = align_up(off + (size_t)(2 * L.slots) * s.cols * sizeof(SplitRec));
  L.best = off; off = align_up(off + (size_t)(2 * L.slots) * kKeyWays * sizeof(uint64_t));
  L.hist_tasks = off; off = align_up(off + (size_t)L.max_hist_tasks * sizeof(HistTask));
  L.zero = off; off = align_up(off + (size_t)(2 * L.slots) * sizeof(uint32_t));
  L.part_tasks = off; off = align_up(off + 2 * (size_t)L.max_part_tasks * sizeof(PartTask));
  L.cursors = off; off = align_up(off + (size_t)(2 * 2 * L.slots) * sizeof(uint32_t));
  L.split_bins = off; off = align_up(off + ((size_t)2 << depth) * sizeof(int32_t));
  {
    // Per-tile partial histograms of multi-tile nodes (dense path only: the
    // CSR histogram adds every tile into the node's own row).
    const uint64_t groups = div_up(s.cols, s.features_per_group ? s.features_per_group : 1);
    L.partials = off;
    if (!s.sparse)
      off = align_up(off + (size_t)L.max_hist_tasks * groups * s.features_per_group * (s.max_bin + 1) * 16);
  }
  if (s.stable_partition) {
    L.part_masks = off; off = align_up(off + (size_t)L.max_part_tasks * (part_tile / 64) * sizeof(uint64_t));
    L.part_left = off; off = align_up(off + (size_t)L.max_part_tasks * sizeof(uint32_t));
    L.final_order = off; off = align_up(off + ((size_t)L.max_part_tasks + 9) * sizeof(uint32_t));
  } else {
    L.part_masks = L.part_left = L.final_order = 0;
  }
  L.total = off;
  return L;
}

template <typename BinT, int G>
int launch_hist(const Tree& t, uint32_t depth, bool unit, uint32_t grid) {
  size_t lds = (size_t)G * t.bins1 * (8 + (unit ? 4 : 8));
  bool identity = depth == 0;  // the root histogram reads rows [0, N) in order
  const bool cols = t.columns != nullptr && depth < t.column_levels;
#define MGB_HIST_CASE(U, I)                                                                           \
  {                                                                                                   \
    auto fn = cols ? k_histogram<BinT, G, U, I, true> : k_histogram<BinT, G, U, I, false>;            \
    if (hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != \
        hipSuccess) {                                                                                 \
      set_error("hipFuncSetAttribute(histogram LDS) failed");                                         \
      return -1;                                                                                      \
    }                                                                                                 \
    launch(MGB_PROF_HISTOGRAM, fn, dim3(grid), dim3(kHistThreads), (uint32_t)lds, t, depth);          \
  }
  if (unit && identity) MGB_HIST_CASE(true, true)
  else if (unit) MGB_HIST_CASE(true, false)
  else if (identity) MGB_HIST_CASE(false, true)
  else MGB_HIST_CASE(false, false)
#undef MGB_HIST_CASE
  MGB_LAUNCH_CHECK("k_histogram");
  return 0;
}

template <typename BinT>
int dispatch_hist(const Tree& t, uint32_t depth, uint32_t grid) {
  bool unit = t.unit_hessian != 0;
  switch (t.features_per_group) {
    case 1: return launch_hist<BinT, 1>(t, depth, unit, grid);
    case 2: return launch_hist<BinT, 2>(t, depth, unit, grid);
    case 4: return launch_hist<BinT, 4>(t, depth, unit, grid);
    case 8: return launch_hist<BinT, 8>(t, depth, unit, grid);
    case 16: return launch_hist<BinT, 16>(t, depth, unit, grid);
  }
  set_error("features_per_group must be 1, 2, 4, 8 or 16");
  return -1;
}

// Waves per split item with four bins per lane (every bin in registers).
uint32_t split_waves(uint32_t max_bin) {
  uint32_t w = 1;
  while (w < 16 && w * kWave * 4 < max_bin) w *= 2;
  return w;
}

// Items of a level (upper bound known on the host) below about eight waves
// per CU take one bin per lane on four times the waves: shallow levels are
// latency bound, deep ones throughput bound.
int launch_split(const Tree& t, uint32_t depth, uint32_t items) {
  const uint32_t w4 = split_waves(t.max_bin);
  if (w4 * kWave * 4 < t.max_bin) { set_error("max_bin too large for the split kernel"); return -1; }
  items = items ? items : 1;
  // Spread shape (one bin per lane on 4·w4 waves per item) while a level has
  // few items: under 2048 waves of the four-bin shape up to 512 bins, under
  // 2048 items at 1024 bins, whose mid levels also sum many tiles' partials
  // per item (10M x 128: split 1.35 -> 1.31 ms per round; under 4096 items
  // 1.33; 262,144 x 64 slower with any wider spread).
  const bool spread = (w4 >= 4 ? (uint64_t)items < 2048 : (uint64_t)items * w4 < 2048) && w4 * 4 <= 16;
  const uint32_t w = spread ? 4 * w4 : w4;
  const dim3 grid(w == 1 ? div_up(items, kSplitPack) : items), block(w == 1 ? kSplitPack * kWave : w * kWave);
  if (!spread) {
    switch (w) {
      case 1: launch(MGB_PROF_SPLIT, k_split<1, 4>, grid, block, 0, t, depth); break;
      case 2: launch(MGB_PROF_SPLIT, k_split<2, 4>, grid, block, 0, t, depth); break;
      case 4: launch(MGB_PROF_SPLIT, k_split<4, 4>, grid, block, 0, t, depth); break;
      case 8: launch(MGB_PROF_SPLIT, k_split<8, 4>, grid, block, 0, t, depth); break;
      default: launch(MGB_PROF_SPLIT, k_split<16, 4>, grid, block, 0, t, depth); break;
    }
  } else {
    switch (w) {
      case 4: launch(MGB_PROF_SPLIT, k_split<4, 1>, grid, block, 0, t, depth); break;
      case 8: launch(MGB_PROF_SPLIT, k_split<8, 1>, grid, block, 0, t, depth); break;
      default: launch(MGB_PROF_SPLIT, k_split<16, 1>, grid, block, 0, t, depth); break;
    }
  }
  MGB_LAUNCH_CHECK("k_split");
  return 0;
}

// Select + partition of a level: `grid` partition workgroups plus the
// bookkeeping workgroup; the dense root stages two features in LDS.
template <typename BinT>
int launch_apply(const Tree& t, uint32_t depth, uint32_t grid) {
  const uint32_t lds = depth == 0 && t.dense ? (uint32_t)root_stage_bytes(t.bins1) : 0u;
  const bool identity = depth == 0 && !t.compact;
  if (t.stable && depth + 1 >= t.max_depth) {
    // The last level moves no rows: its tasks are ordered for the margin
    // updates instead of counted.
    launch(MGB_PROF_PARTITION, k_final_order, dim3(1), dim3(kOrderThreads), 0, t, depth);
    MGB_LAUNCH_CHECK("k_final_order");
  } else if (t.stable) {
    const bool wide = t.part_tile == kPartTileWide;
    auto count = identity ? (wide ? k_part_count<BinT, true, 8> : k_part_count<BinT, true, 4>)
                          : (wide ? k_part_count<BinT, false, 8> : k_part_count<BinT, false, 4>);
    launch(MGB_PROF_PARTITION, count, dim3(grid), dim3(kPartThreads), 0, t, depth);
    MGB_LAUNCH_CHECK("k_part_count");
  }
  static_assert(kPartTileWide == 8 * kPartThreads && kPartTileNarrow == 4 * kPartThreads, "partition tiles");
  const bool wide = t.part_tile == kPartTileWide;
  auto fn = identity ? (t.stable ? (wide ? k_apply<BinT, true, true, 8> : k_apply<BinT, true, true, 4>)
                                 : k_apply<BinT, true, false, 4>)
                     : (t.stable ? (wide ? k_apply<BinT, false, true, 8> : k_apply<BinT, false, true, 4>)
                                 : k_apply<BinT, false, false, 4>);
  if (lds && hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
    set_error("hipFuncSetAttribute(select LDS) failed");
    return -1;
  }
  launch(MGB_PROF_PARTITION, fn, dim3(grid + 1), dim3(kPartThreads), lds, t, depth);
  MGB_LAUNCH_CHECK("k_apply");
  return 0;
}

// Row positions inside the kernels are 32-bit and run up to two batches past
// a task's end (the histogram's prefetch), so row counts stay below 2^31, the
// sketch's own limit.
constexpr uint32_t kMaxTreeRows = 0x7fffffffu;

int validate(const MgbTreeShape* s, const MgbMatrix* m) {
  if (!s || !m) { set_error("null shape or matrix"); return -1; }
  if (s->max_depth < 1 || s->max_depth > 16) { set_error("max_depth must be in [1, 16]"); return -1; }
  if (s->rows > kMaxTreeRows) { set_error("rows must be below 2^31"); return -1; }
  if (s->rows != m->rows || s->cols != m->cols || s->max_bin != m->max_bin) {
    set_error("tree shape does not match the bin matrix");
    return -1;
  }
  if (m->bin_bytes != 1 && m->bin_bytes != 2) { set_error("bin_bytes must be 1 or 2"); return -1; }
  uint32_t G = s->features_per_group;
  if (G != 1 && G != 2 && G != 4 && G != 8 && G != 16) { set_error("features_per_group must be a power of two <= 16"); return -1; }
  uint32_t groups = div_up(m->cols, G);
  if (m->group_features != G) { set_error("features_per_group does not match the bin matrix's groups"); return -1; }
  const uint64_t gbytes = (uint64_t)G * m->bin_bytes;
  const bool row_major = m->group_stride == gbytes && m->row_stride == groups * gbytes;
  const bool group_major = m->row_stride == gbytes && m->group_stride == (uint64_t)m->rows * gbytes;
  if (!row_major && !group_major) { set_error("bin matrix strides describe neither layout"); return -1; }
  if (s->rows_per_tile < 64) { set_error("rows_per_tile must be >= 64"); return -1; }
  if (s->root_rows_per_tile && s->root_rows_per_tile < s->rows_per_tile) {
    set_error("root_rows_per_tile must be 0 or >= rows_per_tile");
    return -1;
  }
  if (m->max_bin < 1 || m->max_bin > kMaxBin) { set_error("max_bin must be in [1, " + std::to_string(kMaxBin) + "]"); return -1; }
  if ((size_t)G * (m->max_bin + 1) * 16 > 160 * 1024) { set_error("feature group does not fit in LDS"); return -1; }
  return 0;
}

Tree make_tree(const MgbTreeShape* s, const MgbMatrix* m, const Layout& L, uint8_t* ws) {
  Tree t;
  std::memset(&t, 0, sizeof(t));
  t.state = reinterpret_cast<LevelState*>(ws + L.state);
  uint32_t* rows = reinterpret_cast<uint32_t*>(ws + L.rows);
  t.rows[0] = rows;
  t.rows[1] = rows + s->rows;
  float2* gh = reinterpret_cast<float2*>(ws + L.gh);
  t.gh[0] = gh;
  t.gh[1] = gh + s->rows;
  int64_t* hist = reinterpret_cast<int64_t*>(ws + L.hist);
  t.hist[0] = hist;
  t.hist[1] = hist + (size_t)L.slots * L.hist_entry;
  Frontier* fr = reinterpret_cast<Frontier*>(ws + L.frontier);
  t.frontier[0] = fr;
  t.frontier[1] = fr + 2 * L.slots;
  t.recs = reinterpret_cast<SplitRec*>(ws + L.recs);
  t.best = reinterpret_cast<unsigned long long*>(ws + L.best);
  t.hist_tasks = reinterpret_cast<HistTask*>(ws + L.hist_tasks);
  t.zero_list = reinterpret_cast<uint32_t*>(ws + L.zero);
  t.part_tasks = reinterpret_cast<PartTask*>(ws + L.part_tasks);
  t.cursors = reinterpret_cast<uint32_t*>(ws + L.cursors);
  t.split_bins = reinterpret_cast<int32_t*>(ws + L.split_bins);
  t.partials = reinterpret_cast<int64_t*>(ws + L.partials);
  t.rows_n = s->rows; t.cols = s->cols; t.max_bin = m->max_bin; t.bins1 = m->max_bin + 1;
  t.row_stride = m->row_stride; t.bin_bytes = m->bin_bytes; t.missing_code = m->missing_code;
  t.group_stride = m->group_stride;
  t.cut_stride = m->cut_stride;
  t.max_depth = s->max_depth; t.slots = L.slots; t.rows_per_tile = s->rows_per_tile;
  t.root_tile = s->root_rows_per_tile ? s->root_rows_per_tile : s->rows_per_tile;
  t.features_per_group = s->features_per_group;
  t.groups = div_up(s->cols, s->features_per_group);
  t.unit_hessian = s->unit_hessian; t.dense = s->dense; t.max_hist_tasks = L.max_hist_tasks;
  t.max_part_tasks = L.max_part_tasks;
  t.column_levels = s->column_levels;
  t.sparse = s->sparse;
  t.compact = s->compact_sampled && !s->sparse ? 1u : 0u;
  t.stable = s->stable_partition ? 1u : 0u;
  t.part_tile = partition_tile(t.stable != 0, t.sparse != 0, s->rows);
  if (t.stable) {
    t.part_masks = reinterpret_cast<uint64_t*>(ws + L.part_masks);
    t.part_left = reinterpret_cast<uint32_t*>(ws + L.part_left);
    t.final_order = reinterpret_cast<uint32_t*>(ws + L.final_order);
  }
  t.hist_entry = L.hist_entry;
  return t;
}

uint32_t reduce_grid(const Tree& t) {
  // Blocks stride over (multi-tile node, 64-entry block) pairs; enough blocks
  // to fill the device when one node's entries are all there is.
  const uint64_t eblocks = div_up((uint64_t)t.cols * t.bins1, kWave);
  const uint64_t g = eblocks * 4 < 2048 ? eblocks * 4 : 2048;
  return (uint32_t)(g ? g : 1);
}

// Workgroups for `tasks` histogram tasks: one per (task, feature group), at
// most 2048 (the kernel loops), a multiple of 8 for the XCD-aware schedule.
uint32_t hist_grid_for(const Tree& t, uint64_t tasks) {
  uint64_t items = tasks * t.groups;
  uint64_t g = items < 2048 ? items : 2048;
  g = (g + 7) / 8 * 8;
  return (uint32_t)(g ? g : 8);
}

uint32_t hist_grid(const Tree& t) { return hist_grid_for(t, t.max_hist_tasks); }

// A level's histogram tasks are bounded on the host without reading the
// device: the root has ceil(N / tile) row tiles; below it the built (smaller)
// children of at most 2^(depth-1) sibling pairs hold at most N/2 rows, so
// their tiles number at most floor(N/2 / tile) + 2^(depth-1) (each node adds
// at most one partial tile).  Idle 1024-thread workgroups are not free: each
// costs a dispatch, so the grid follows the level's bound.
uint64_t level_hist_tasks(const Tree& t, uint32_t depth) {
  uint64_t tasks;
  if (depth == 0) {
    tasks = t.rows_n ? div_up(t.rows_n, t.root_tile) : 0;
  } else {
    const uint64_t nodes = depth - 1 < 32 ? (1ull << (depth - 1)) : ~0ull >> 1;
    tasks = (uint64_t)(t.rows_n / 2) / t.rows_per_tile + nodes;
  }
  return tasks < t.max_hist_tasks ? tasks : t.max_hist_tasks;
}

// Partition workgroups at a level: nodes at depth d (at most 2^d) hold at
// most N rows, in at most floor(N / tile) + 2^d tiles; the kernel loops over
// tasks, so 2048 workgroups cover any level (10M x 128: partition 1.70 /
// 1.67 / 1.71 ms per round with at most 1024 / 2048 / 4096).
uint32_t level_part_grid(const Tree& t, uint32_t depth) {
  const uint64_t nodes = depth < 32 ? (1ull << depth) : ~0ull >> 1;
  const uint64_t tasks = (uint64_t)t.rows_n / t.part_tile + nodes;
  return (uint32_t)(tasks < 2048 ? tasks : 2048);
}

}  // namespace
}  // namespace mgb

using namespace mgb;

extern "C" {

size_t mgb_tree_workspace_bytes(const MgbTreeShape* shape) { return layout(*shape).total; }

int mgb_grow_tree(const MgbTreeShape* shape, const MgbMatrix* m, const void* bins, const void* columns,
                  const float* cuts, const uint32_t* counts, const float* grad, const float* scales,
                  const MgbSplitParams* sp, const uint32_t* features, const int32_t* monotone, void* workspace,
                  size_t workspace_bytes, float* margin, MgbTreeNode* nodes, uint32_t* node_count) {
  if (validate(shape, m)) return -1;
  Layout L = layout(*shape);
  if (!workspace || workspace_bytes < L.total) { set_error("mgb_grow_tree: workspace too small"); return -1; }
  Tree t = make_tree(shape, m, L, reinterpret_cast<uint8_t*>(workspace));
  t.bins = bins; t.columns = columns; t.cuts = cuts; t.counts = counts; t.grad = reinterpret_cast<const float2*>(grad);
  t.scales = scales; t.margin = margin; t.nodes = nodes; t.node_count_out = node_count; t.sp = *sp;
  t.status = node_count ? node_count + 1 : nullptr;
  t.allowed = features;
  t.monotone = monotone;
  if (t.compact) {
    launch(MGB_PROF_CONTROL, k_compact_reset, dim3(1), dim3(64), 0, t);
    MGB_LAUNCH_CHECK("k_compact_reset");
    if (t.rows_n) {
      launch(MGB_PROF_CONTROL, k_compact_rows, dim3(div_up(t.rows_n, kCompactRows)), dim3(kCompactThreads), 0, t);
      MGB_LAUNCH_CHECK("k_compact_rows");
    }
  }
  // The root histogram's workgroup 0 does the level-0 set-up (one launch
  // fewer per tree).
  t.fused_level0 = 1;
  // Unit Hessians: the select bookkeeping plans each next level (child counts are known
  // from the count histograms), so k_plan is not launched.
  t.select_plans = t.unit_hessian ? 1u : 0u;
  for (uint32_t depth = 0; depth < shape->max_depth; ++depth) {
    if (depth > 0 && !t.select_plans && !counts_plan_level(t, depth - 1)) {
      launch(MGB_PROF_CONTROL, k_plan, dim3(1), dim3(kSelectThreads), 0, t, depth);
      MGB_LAUNCH_CHECK("k_plan");
    }
    const uint32_t hgrid = hist_grid_for(t, level_hist_tasks(t, depth));
    const uint32_t pgrid = level_part_grid(t, depth);
    if ((m->bin_bytes == 1 ? dispatch_hist<uint8_t>(t, depth, hgrid) : dispatch_hist<uint16_t>(t, depth, hgrid)))
      return -1;
    uint32_t max_nodes = 1u << depth;
    uint32_t items = depth == 0 ? shape->cols : (max_nodes / 2) * shape->cols;
    if (launch_split(t, depth, items)) return -1;
    if ((m->bin_bytes == 1 ? launch_apply<uint8_t>(t, depth, pgrid) : launch_apply<uint16_t>(t, depth, pgrid)))
      return -1;
  }
  if (t.compact) {
    // Dropped rows: at most N, kWalkPer per thread; the kernel strides over
    // the device's count, so a bounded grid covers any number.
    const uint32_t per_block = kCompactThreads * kWalkPer;
    const uint32_t wgrid = t.rows_n ? std::min<uint32_t>(div_up(t.rows_n, per_block), 4096) : 1;
    if (m->bin_bytes == 1) launch(MGB_PROF_PARTITION, k_walk_dropped<uint8_t>, dim3(wgrid), dim3(kCompactThreads), 0, t);
    else launch(MGB_PROF_PARTITION, k_walk_dropped<uint16_t>, dim3(wgrid), dim3(kCompactThreads), 0, t);
    MGB_LAUNCH_CHECK("k_walk_dropped");
  }
  return 0;
}

}  // extern "C"

namespace mgb {
namespace {

std::mutex g_scratch_mutex;
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the library's device, looked up once per
// device with that device current (each device holds its own copy).
int scratch_address(void** out) {
  const int dev = bound_device();
  if (dev < 0) return -1;
  if (dev >= kMaxDevices) { set_error("mgb_grow_tree_noalloc: device index above 63"); return -1; }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    int current = -1;
    MGB_CHECK(hipGetDevice(&current));
    if (current != dev) MGB_CHECK(hipSetDevice(dev));
    void* ptr = nullptr;
    const hipError_t status = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (current != dev) MGB_CHECK(hipSetDevice(current));
    MGB_CHECK(status);
    if (!ptr) { set_error("hipGetSymbolAddress(scratch) returned a null address"); return -1; }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace
}  // namespace mgb

extern "C" {

int mgb_grow_tree_noalloc(const MgbTreeShape* shape, const MgbMatrix* m, const void* bins, const void* columns,
                          const float* cuts, const uint32_t* counts, const float* grad, const float* scales,
                          const MgbSplitParams* sp, const uint32_t* features, const int32_t* monotone, float* margin,
                          MgbTreeNode* nodes, uint32_t* node_count) {
  if (!shape || !m || !sp) { set_error("mgb_grow_tree_noalloc: null shape, matrix or parameters"); return -1; }
  if (validate(shape, m)) return -1;
  const size_t need = layout(*shape).total;
  if (need > kNoAllocScratchBytes) {
    set_error("mgb_grow_tree_noalloc: this tree shape needs " + std::to_string(need) +
              " bytes of workspace, above the " + std::to_string(kNoAllocScratchBytes) +
              "-byte allocation-free scratch; use mgb_grow_tree with a workspace");
    return -1;
  }
  if (profiling_enabled()) {
    set_error("mgb_grow_tree_noalloc: per-kernel timing creates HIP events; disable mgb_profile_enable first");
    return -1;
  }
  void* ws = nullptr;
  if (scratch_address(&ws)) return -1;
  return mgb_grow_tree(shape, m, bins, columns, cuts, counts, grad, scales, sp, features, monotone, ws,
                       kNoAllocScratchBytes, margin, nodes, node_count);
}

}  // extern "C"

namespace mgb {
namespace {

// One level's CSR histograms: the root from the column-major codes when
// given, else clear the built nodes' rows and add their rows' nonzeros.
int csr_histogram(const Tree& t, uint32_t bin_bytes, uint32_t depth, bool root_columns, uint32_t hgrid, uint32_t zx) {
  if (depth == 0 && root_columns) {
    uint32_t per_group = kRootFeatures;
    while (per_group > 1 && per_group * t.bins1 * 16 > 160 * 1024) per_group >>= 1;
    const uint32_t lds = per_group * t.bins1 * 16;
    const dim3 grid(div_up(t.cols, per_group));
    auto fn = bin_bytes == 1 ? k_histogram_csc_root<uint8_t> : k_histogram_csc_root<uint16_t>;
    if (hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
      set_error("hipFuncSetAttribute(root histogram LDS) failed");
      return -1;
    }
    launch(MGB_PROF_HISTOGRAM, fn, grid, dim3(kRootThreads), lds, t, per_group);
    MGB_LAUNCH_CHECK("k_histogram_csc_root");
    return 0;
  }
  const uint32_t zy = depth == 0 ? 1 : (1u << depth) < 1024 ? (1u << depth) : 1024;
  launch(MGB_PROF_HISTOGRAM, k_zero_built, dim3(zx, zy), dim3(256), 0, t, depth);
  MGB_LAUNCH_CHECK("k_zero_built");
  auto fn = bin_bytes == 1 ? (depth == 0 ? k_histogram_csr<uint8_t, true> : k_histogram_csr<uint8_t, false>)
                           : (depth == 0 ? k_histogram_csr<uint16_t, true> : k_histogram_csr<uint16_t, false>);
  launch(MGB_PROF_HISTOGRAM, fn, dim3(hgrid), dim3(kCsrThreads), 0, t, depth);
  MGB_LAUNCH_CHECK("k_histogram_csr");
  return 0;
}

}  // namespace
}  // namespace mgb

extern "C" {

int mgb_grow_tree_csr(const MgbTreeShape* shape, const MgbCsrMatrix* m, const uint64_t* indptr,
                      const uint32_t* indices, const void* codes, const uint64_t* colptr, const uint32_t* csc_rows,
                      const void* csc_codes, const float* cuts, const uint32_t* counts,
                      const float* grad, const float* scales, const MgbSplitParams* sp, const uint32_t* features,
                      const int32_t* monotone, void* workspace, size_t workspace_bytes, float* margin, MgbTreeNode* nodes,
                      uint32_t* node_count) {
  if (!shape || !m) { set_error("null shape or matrix"); return -1; }
  if (!shape->sparse) { set_error("mgb_grow_tree_csr: the tree shape must have sparse = 1"); return -1; }
  if (shape->max_depth < 1 || shape->max_depth > 16) { set_error("max_depth must be in [1, 16]"); return -1; }
  if (shape->rows > kMaxTreeRows) { set_error("rows must be below 2^31"); return -1; }
  if (shape->rows != m->rows || shape->cols != m->cols || shape->max_bin != m->max_bin) {
    set_error("tree shape does not match the CSR matrix");
    return -1;
  }
  if (m->bin_bytes != 1 && m->bin_bytes != 2) { set_error("bin_bytes must be 1 or 2"); return -1; }
  if (m->max_bin < 1 || m->max_bin > kMaxBin) { set_error("max_bin must be in [1, " + std::to_string(kMaxBin) + "]"); return -1; }
  if (shape->rows_per_tile < 64) { set_error("rows_per_tile must be >= 64"); return -1; }
  if (!shape->features_per_group) { set_error("features_per_group must be at least 1"); return -1; }
  Layout L = layout(*shape);
  if (!workspace || workspace_bytes < L.total) { set_error("mgb_grow_tree_csr: workspace too small"); return -1; }
  MgbMatrix dm;
  std::memset(&dm, 0, sizeof(dm));
  dm.rows = m->rows; dm.cols = m->cols; dm.bin_bytes = m->bin_bytes; dm.max_bin = m->max_bin;
  dm.cut_stride = m->cut_stride; dm.missing_code = m->missing_code; dm.group_features = shape->features_per_group;
  Tree t = make_tree(shape, &dm, L, reinterpret_cast<uint8_t*>(workspace));
  t.csr_indptr = indptr; t.csr_indices = indices; t.csr_codes = codes;
  const bool root_columns = colptr && csc_rows && csc_codes;
  t.csc_colptr = colptr; t.csc_rows = csc_rows; t.csc_codes = csc_codes;
  t.cuts = cuts; t.counts = counts; t.grad = reinterpret_cast<const float2*>(grad);
  t.scales = scales; t.margin = margin; t.nodes = nodes; t.node_count_out = node_count; t.sp = *sp;
  t.status = node_count ? node_count + 1 : nullptr;
  t.allowed = features;
  t.monotone = monotone;
  t.column_levels = 0;
  launch(MGB_PROF_CONTROL, k_level0, dim3(1), dim3(256), 0, t);
  MGB_LAUNCH_CHECK("k_level0");
  launch(MGB_PROF_HISTOGRAM, k_root_totals, dim3(m->rows ? div_up(m->rows, kCsrThreads * 8) : 1),
         dim3(kCsrThreads), 0, t);
  MGB_LAUNCH_CHECK("k_root_totals");
  const uint64_t row_int4 = (uint64_t)t.cols * t.bins1;
  const uint32_t zx = (uint32_t)(row_int4 / (256 * 8) + 1 < 64 ? row_int4 / (256 * 8) + 1 : 64);
  for (uint32_t depth = 0; depth < shape->max_depth; ++depth) {
    if (depth > 0 && !counts_plan_level(t, depth - 1)) {
      launch(MGB_PROF_CONTROL, k_plan, dim3(1), dim3(kSelectThreads), 0, t, depth);
      MGB_LAUNCH_CHECK("k_plan");
    }
    const uint64_t tasks = level_hist_tasks(t, depth);
    const uint32_t hgrid = (uint32_t)(tasks < 4096 ? (tasks ? tasks : 1) : 4096);
    if (csr_histogram(t, m->bin_bytes, depth, root_columns, hgrid, zx)) return -1;
    uint32_t max_nodes = 1u << depth;
    uint32_t items = depth == 0 ? shape->cols : (max_nodes / 2) * shape->cols;
    if (launch_split(t, depth, items)) return -1;
    const uint32_t pgrid = level_part_grid(t, depth);
    if ((m->bin_bytes == 1 ? launch_apply<uint8_t>(t, depth, pgrid) : launch_apply<uint16_t>(t, depth, pgrid)))
      return -1;
  }
  return 0;
}

int mgb_tree_level_stats(const MgbTreeShape* shape, const void* workspace, uint64_t* rows_built,
                         uint32_t* nodes_built, uint32_t levels) {
  Layout L = layout(*shape);
  LevelState st;
  MGB_CHECK(hipMemcpyAsync(&st, reinterpret_cast<const uint8_t*>(workspace) + L.state, sizeof(st),
                           hipMemcpyDeviceToHost, stream()));
  MGB_CHECK(hipStreamSynchronize(stream()));
  for (uint32_t d = 0; d < levels && d < kMaxLevels; ++d) {
    bool valid = d < shape->max_depth;
    if (rows_built) rows_built[d] = valid ? st.rows_built[d] : 0;
    if (nodes_built) nodes_built[d] = valid ? st.nodes_built[d] : 0;
  }
  return 0;
}

int mgb_tree_partition_stats(const MgbTreeShape* shape, const void* workspace, uint32_t* rows_split,
                             uint32_t* rows_leaf, uint32_t levels) {
  if (!shape || !workspace) { set_error("mgb_tree_partition_stats: null argument"); return -1; }
  Layout L = layout(*shape);
  LevelState st;
  MGB_CHECK(hipMemcpyAsync(&st, reinterpret_cast<const uint8_t*>(workspace) + L.state, sizeof(st),
                           hipMemcpyDeviceToHost, stream()));
  MGB_CHECK(hipStreamSynchronize(stream()));
  for (uint32_t d = 0; d < levels && d < kMaxLevels; ++d) {
    const bool valid = d < shape->max_depth;
    if (rows_split) rows_split[d] = valid ? st.rows_split[d] : 0;
    if (rows_leaf) rows_leaf[d] = valid ? st.rows_leaf[d] : 0;
  }
  return 0;
}

int mgb_tree_row_list(const MgbTreeShape* shape, const void* workspace, uint32_t depth, uint32_t* rows) {
  if (!shape || !workspace || !rows) { set_error("mgb_tree_row_list: null argument"); return -1; }
  Layout L = layout(*shape);
  const uint8_t* list = reinterpret_cast<const uint8_t*>(workspace) + L.rows +
                        (size_t)(depth & 1) * shape->rows * sizeof(uint32_t);
  MGB_CHECK(hipMemcpyAsync(rows, list, (size_t)shape->rows * sizeof(uint32_t), hipMemcpyDeviceToHost, stream()));
  MGB_CHECK(hipStreamSynchronize(stream()));
  return 0;
}

int mgb_histogram(const MgbTreeShape* shape, const MgbMatrix* m, const void* bins, const uint32_t* rows,
                  uint32_t count, const float* grad, const float* scales, int64_t* hist, void* workspace,
                  size_t workspace_bytes) {
  if (validate(shape, m)) return -1;
  Layout L = layout(*shape);
  if (!workspace || workspace_bytes < L.total) { set_error("mgb_histogram: workspace too small"); return -1; }
  if (count > shape->rows) { set_error("mgb_histogram: count exceeds rows"); return -1; }
  Tree t = make_tree(shape, m, L, reinterpret_cast<uint8_t*>(workspace));
  t.bins = bins; t.grad = reinterpret_cast<const float2*>(grad); t.scales = scales;
  t.nodes = nullptr;  // no tree records: k_level0 skips the root record
  // Level-0 layout with the caller's row list copied into the row buffer.
  t.rows_n = count;
  hipStream_t s = stream();
  hipLaunchKernelGGL(k_level0, dim3(1), dim3(256), 0, s, t);
  MGB_LAUNCH_CHECK("k_level0");
  uint32_t depth = 0;
  if (rows) {
    MGB_CHECK(hipMemcpyAsync(t.rows[0], rows, (size_t)count * sizeof(uint32_t), hipMemcpyDeviceToDevice, s));
    depth = 2;  // even depth selects bank 0 and row buffer 0 without the identity shortcut
    if (count) {
      hipLaunchKernelGGL(k_gather_pairs, dim3(std::min<uint32_t>(div_up(count, 256), 4096)), dim3(256), 0, s, t, count);
      MGB_LAUNCH_CHECK("k_gather_pairs");
    }
  }
  const uint32_t grid = hist_grid(t);
  if ((m->bin_bytes == 1 ? dispatch_hist<uint8_t>(t, depth, grid) : dispatch_hist<uint16_t>(t, depth, grid))) return -1;
  hipLaunchKernelGGL(k_reduce_hist, dim3(reduce_grid(t)), dim3(kReduceWaves * kWave), 0, s, t, depth);
  MGB_LAUNCH_CHECK("k_reduce_hist");
  MGB_CHECK(hipMemcpyAsync(hist, t.hist[0], (size_t)L.hist_entry * sizeof(int64_t), hipMemcpyDeviceToDevice, s));
  return 0;
}

}  // extern "C"
