// Prediction beyond values and margins (reference src/learner.cpp:455-560
// Learner::predict types 2 to 6): each row's leaf index in every tree, its
// per-feature contributions to its margin and their pairwise interactions --
// exact path-dependent TreeSHAP (Lundberg, Erion and Lee 2018, "Consistent
// individualized feature attribution for tree ensembles", Algorithm 2), or
// the approximation that credits each split's feature with the change of the
// cover-weighted node mean along the row's path.  Rows are dense (X with
// `cols` values a row) or CSR (indptr/indices/values; absent entries are
// missing), walked with the predictor's rule: value < threshold goes left,
// NaN follows default_left.  One thread per row walks every tree, so a row's
// sums need no atomics.
#include <hip/hip_runtime.h>

#include <cmath>

#include "device_common.hpp"

namespace mgb {
namespace {

// One row's feature values.
struct RowView {
  const float* dense;
  const uint32_t* indices;
  const float* values;
  uint64_t begin, end;
  uint32_t cols;
  __device__ float operator()(uint32_t f) const {
    if (f >= cols) return __uint_as_float(0x7fc00000u);  // a model feature the matrix lacks reads as missing
    if (dense) return dense[f];
    uint64_t lo = begin, hi = end;
    while (lo < hi) {
      const uint64_t mid = lo + (hi - lo) / 2;
      if (indices[mid] < f) lo = mid + 1;
      else hi = mid;
    }
    return lo < end && indices[lo] == f ? values[lo] : __uint_as_float(0x7fc00000u);
  }
};

__device__ __forceinline__ RowView row_view(const float* X, const uint64_t* indptr, const uint32_t* indices,
                                            uint64_t r, uint32_t cols) {
  if (!indptr) return RowView{X + r * cols, nullptr, nullptr, 0, 0, cols};
  return RowView{nullptr, indices, X, indptr[r], indptr[r + 1], cols};
}

__device__ __forceinline__ int32_t child_of(const MgbTreeNode& n, float v) {
  const bool left = isnan(v) ? n.default_left != 0 : v < n.threshold;
  return left ? n.left : n.right;
}

__global__ void k_predict_leaf(const float* __restrict__ X, const uint64_t* __restrict__ indptr,
                               const uint32_t* __restrict__ indices, uint32_t rows, uint32_t cols,
                               const MgbTreeNode* __restrict__ nodes, const uint32_t* __restrict__ offsets,
                               uint32_t trees, float* __restrict__ out) {
  for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (uint64_t)gridDim.x * blockDim.x) {
    const RowView x = row_view(X, indptr, indices, r, cols);
    for (uint32_t t = 0; t < trees; ++t) {
      const MgbTreeNode* tree = nodes + offsets[t];
      int32_t id = 0;
      while (tree[id].left >= 0) id = child_of(tree[id], x((uint32_t)tree[id].feature));
      out[r * trees + t] = (float)id;
    }
  }
}

// Row r's contributions: out[r * (cols + 1) + f] for feature f, and the bias
// (the base margin plus every tree's root mean) at f = cols.
// With `interactions` the row is a (cols + 1) x (cols + 1) matrix holding
// these values on its diagonal (the reference's approximate interactions,
// kernels/boost.metal:2183).
__global__ void k_contribs_approx(const float* __restrict__ X, const uint64_t* __restrict__ indptr,
                                  const uint32_t* __restrict__ indices, uint32_t rows, uint32_t cols,
                                  const MgbTreeNode* __restrict__ nodes, const float* __restrict__ means,
                                  const uint32_t* __restrict__ offsets, uint32_t trees,
                                  const float* __restrict__ base, float base_value, uint32_t interactions,
                                  float* __restrict__ out) {
  const uint64_t width = (uint64_t)cols + 1, elements = interactions ? width * width : width;
  const uint64_t stride = interactions ? width + 1 : 1;
  for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (uint64_t)gridDim.x * blockDim.x) {
    const RowView x = row_view(X, indptr, indices, r, cols);
    float* phi = out + r * elements;
    for (uint64_t e = 0; e < elements; ++e) phi[e] = 0.0f;
    float bias = base ? base[r] : base_value;
    for (uint32_t t = 0; t < trees; ++t) {
      const MgbTreeNode* tree = nodes + offsets[t];
      const float* mean = means + offsets[t];
      int32_t id = 0;
      float here = mean[0];
      bias += here;
      while (tree[id].left >= 0) {
        const uint32_t f = (uint32_t)tree[id].feature;
        id = child_of(tree[id], x(f));
        if (f < cols) phi[f * stride] += mean[id] - here;
        here = mean[id];
      }
    }
    phi[elements - 1] = bias;
  }
}

// ---- exact TreeSHAP ---------------------------------------------------------
// A path element: the feature split on, the fraction of the node's cover that
// follows the path ("zero": the feature left out), whether the row follows it
// ("one": the feature present), and the element's permutation weight.
struct PathElem {
  int32_t feature;
  float zero, one, weight;
};

// Appends (feature, zero, one) to a path of `len` elements and updates the
// permutation weights of subsets of every size (Algorithm 2, EXTEND).
__device__ void path_extend(PathElem* p, uint32_t len, float zero, float one, int32_t feature) {
  p[len] = PathElem{feature, zero, one, len == 0 ? 1.0f : 0.0f};
  for (int i = (int)len - 1; i >= 0; --i) {
    p[i + 1].weight += one * p[i].weight * (float)(i + 1) / (float)(len + 1);
    p[i].weight = zero * p[i].weight * (float)(len - i) / (float)(len + 1);
  }
}

// Removes element idx from a path whose last element is `last` (UNWIND): the
// inverse of the extension that added it.
__device__ void path_unwind(PathElem* p, uint32_t last, uint32_t idx) {
  const float one = p[idx].one, zero = p[idx].zero;
  float next = p[last].weight;
  for (int i = (int)last - 1; i >= 0; --i) {
    if (one != 0.0f) {
      const float kept = p[i].weight;
      p[i].weight = next * (float)(last + 1) / ((float)(i + 1) * one);
      next = kept - p[i].weight * zero * (float)(last - i) / (float)(last + 1);
    } else {
      p[i].weight = p[i].weight * (float)(last + 1) / (zero * (float)(last - i));
    }
  }
  for (uint32_t i = idx; i < last; ++i) {
    p[i].feature = p[i + 1].feature;
    p[i].zero = p[i + 1].zero;
    p[i].one = p[i + 1].one;
  }
}

// Total weight of the path with element idx unwound, without changing it.
__device__ float path_unwound_sum(const PathElem* p, uint32_t last, uint32_t idx) {
  const float one = p[idx].one, zero = p[idx].zero;
  float next = p[last].weight, total = 0.0f;
  for (int i = (int)last - 1; i >= 0; --i) {
    if (one != 0.0f) {
      const float w = next * (float)(last + 1) / ((float)(i + 1) * one);
      total += w;
      next = p[i].weight - w * zero * ((float)(last - i) / (float)(last + 1));
    } else if (zero != 0.0f) {
      total += (p[i].weight / zero) / ((float)(last - i) / (float)(last + 1));
    }
  }
  return total;
}

// Trees up to this depth (the training limit): a node at depth d extends a
// path segment of at most d + 1 elements placed after its parent's, so the
// segments of one root-to-leaf walk fit kShapPath elements, and at most one
// pending sibling per level waits on the stack.
constexpr uint32_t kShapDepth = 16;
constexpr uint32_t kShapPath = (kShapDepth + 2) * (kShapDepth + 3) / 2;

// A node still to visit: its path is its parent's segment (at `parent`,
// `len` elements), extended by (feature, zero, one) unless `extend` is 0 (the
// split was on the conditioned feature, which never enters the path);
// `share` is the part of the conditioned walk that reaches the node.
struct ShapFrame {
  int32_t node;
  uint32_t len, parent;
  float zero, one, share;
  int32_t feature;
  uint32_t extend;
};

// Adds scale x tree's exact contributions of row x to phi[f * stride]
// (feature f).  condition 0: plain TreeSHAP; +1 / -1: Shapley values of the
// other features with feature `fixed` always present / always absent (the
// conditioned walk of SHAP interaction values).  Returns false, having added
// a part only, for a tree deeper than kShapDepth.
__device__ bool shap_tree(const MgbTreeNode* __restrict__ tree, const RowView& x, uint32_t cols, float* phi,
                          uint32_t stride, float scale, int condition, int32_t fixed, PathElem* path,
                          ShapFrame* stack) {
  uint32_t top = 0;
  stack[top++] = ShapFrame{0, 0, 0, 1.0f, 1.0f, 1.0f, -1, 1u};
  while (top) {
    const ShapFrame fr = stack[--top];
    if (fr.share == 0.0f) continue;
    const uint32_t seg = fr.parent + fr.len + 1;
    // The host admits trees of depth <= kShapDepth only, which never reach
    // these limits.
    if (seg + fr.len >= kShapPath || top + 2 > kShapDepth + 2) return false;
    for (uint32_t i = 0; i < fr.len; ++i) path[seg + i] = path[fr.parent + i];
    PathElem* p = path + seg;
    if (fr.extend) path_extend(p, fr.len, fr.zero, fr.one, fr.feature);
    uint32_t last = fr.extend ? fr.len : fr.len - 1;
    const MgbTreeNode n = tree[fr.node];
    if (n.left < 0) {
      for (uint32_t i = 1; i <= last; ++i) {
        const float w = path_unwound_sum(p, last, i);
        if ((uint32_t)p[i].feature < cols)
          phi[(uint64_t)p[i].feature * stride] += scale * (w * (p[i].one - p[i].zero) * n.leaf * fr.share);
      }
      continue;
    }
    const int32_t hot = child_of(n, x((uint32_t)n.feature));
    const int32_t cold = hot == n.left ? n.right : n.left;
    const float hot_zero = tree[hot].cover / n.cover, cold_zero = tree[cold].cover / n.cover;
    // A feature already on the path is unwound, and its fractions carry
    // into both children.
    float in_zero = 1.0f, in_one = 1.0f;
    uint32_t k = 0;
    while (k <= last && p[k].feature != n.feature) ++k;
    if (k <= last) {
      in_zero = p[k].zero;
      in_one = p[k].one;
      path_unwind(p, last, k);
      --last;
    }
    // The conditioned feature: present, the walk follows the row; absent,
    // it splits by cover; neither child extends the path with it.
    float hot_share = fr.share, cold_share = fr.share;
    const bool on_fixed = condition != 0 && n.feature == fixed;
    if (on_fixed && condition > 0) cold_share = 0.0f;
    if (on_fixed && condition < 0) {
      hot_share *= hot_zero;
      cold_share *= cold_zero;
    }
    const uint32_t extend = on_fixed ? 0u : 1u;
    stack[top++] = ShapFrame{cold, last + 1, seg, cold_zero * in_zero, 0.0f, cold_share, n.feature, extend};
    stack[top++] = ShapFrame{hot, last + 1, seg, hot_zero * in_zero, in_one, hot_share, n.feature, extend};
  }
  return true;
}

__global__ __launch_bounds__(64) void k_contribs_shap(const float* __restrict__ X, const uint64_t* __restrict__ indptr,
                                                      const uint32_t* __restrict__ indices, uint32_t rows,
                                                      uint32_t cols, const MgbTreeNode* __restrict__ nodes,
                                                      const float* __restrict__ means,
                                                      const uint32_t* __restrict__ offsets, uint32_t trees,
                                                      const float* __restrict__ base, float base_value,
                                                      float* __restrict__ out) {
  PathElem path[kShapPath];
  ShapFrame stack[kShapDepth + 2];
  for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (uint64_t)gridDim.x * blockDim.x) {
    const RowView x = row_view(X, indptr, indices, r, cols);
    float* phi = out + r * (cols + 1);
    for (uint32_t f = 0; f < cols; ++f) phi[f] = 0.0f;
    float bias = base ? base[r] : base_value;
    for (uint32_t t = 0; t < trees; ++t) {
      bias += means[offsets[t]];
      if (!shap_tree(nodes + offsets[t], x, cols, phi, 1, 1.0f, 0, -1, path, stack))
        bias = __uint_as_float(0x7fc00000u);  // a NaN bias marks the row
    }
    phi[cols] = bias;
  }
}

// SHAP interaction values of row r, a (cols + 1) x (cols + 1) matrix at
// out + r * (cols + 1)^2: off the diagonal, half the change of feature j's
// value between feature i always present and always absent; on it, feature
// i's value less its interactions; the bias in the last corner.
__global__ __launch_bounds__(64) void k_interactions_shap(const float* __restrict__ X,
                                                          const uint64_t* __restrict__ indptr,
                                                          const uint32_t* __restrict__ indices, uint32_t rows,
                                                          uint32_t cols, const MgbTreeNode* __restrict__ nodes,
                                                          const float* __restrict__ means,
                                                          const uint32_t* __restrict__ offsets, uint32_t trees,
                                                          const float* __restrict__ base, float base_value,
                                                          float* __restrict__ out) {
  PathElem path[kShapPath];
  ShapFrame stack[kShapDepth + 2];
  const uint64_t width = (uint64_t)cols + 1;
  for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (uint64_t)gridDim.x * blockDim.x) {
    const RowView x = row_view(X, indptr, indices, r, cols);
    float* m = out + r * width * width;
    for (uint64_t e = 0; e < width * width; ++e) m[e] = 0.0f;
    float bias = base ? base[r] : base_value;
    bool ok = true;
    for (uint32_t t = 0; t < trees; ++t) {
      bias += means[offsets[t]];
      ok &= shap_tree(nodes + offsets[t], x, cols, m, (uint32_t)width + 1, 1.0f, 0, -1, path, stack);
    }
    for (uint32_t i = 0; i < cols; ++i) {
      float* row_i = m + (uint64_t)i * width;
      for (uint32_t t = 0; t < trees; ++t) {
        ok &= shap_tree(nodes + offsets[t], x, cols, row_i, 1, 0.5f, 1, (int32_t)i, path, stack);
        ok &= shap_tree(nodes + offsets[t], x, cols, row_i, 1, -0.5f, -1, (int32_t)i, path, stack);
      }
      // Feature i never enters its own conditioned walks, so row_i[i] still
      // holds its value.
      float sum = 0.0f;
      for (uint32_t j = 0; j < cols; ++j)
        if (j != i) sum += row_i[j];
      row_i[i] -= sum;
    }
    m[width * width - 1] = ok ? bias : __uint_as_float(0x7fc00000u);
  }
}

uint32_t explain_grid(uint64_t rows, uint32_t block) {
  uint64_t g = (rows + block - 1) / block;
  if (g < 1) g = 1;
  if (g > 8192) g = 8192;
  return (uint32_t)g;
}

}  // namespace
}  // namespace mgb

using namespace mgb;

extern "C" {

int mgb_predict_leaf(const float* X, const uint64_t* indptr, const uint32_t* indices, uint32_t rows, uint32_t cols,
                     const MgbTreeNode* nodes, const uint32_t* tree_offsets, uint32_t trees, float* out) {
  if (!rows || !trees) return 0;
  if (!X || !nodes || !tree_offsets || !out || (indptr && !indices)) {
    set_error("mgb_predict_leaf: null argument");
    return -1;
  }
  launch(MGB_PROF_PREDICT, k_predict_leaf, dim3(explain_grid(rows, 256)), dim3(256), 0, X, indptr, indices, rows,
         cols, nodes, tree_offsets, trees, out);
  MGB_LAUNCH_CHECK("k_predict_leaf");
  return 0;
}

int mgb_predict_contribs(const float* X, const uint64_t* indptr, const uint32_t* indices, uint32_t rows,
                         uint32_t cols, const MgbTreeNode* nodes, const float* node_means,
                         const uint32_t* tree_offsets, uint32_t trees, uint32_t max_depth, uint32_t approximate,
                         uint32_t interactions, const float* base, float base_value, float* out) {
  if (!rows) return 0;
  if (!X || !nodes || !node_means || !tree_offsets || !out || (indptr && !indices)) {
    set_error("mgb_predict_contribs: null argument");
    return -1;
  }
  if (!approximate && max_depth > kShapDepth) {
    set_error("mgb_predict_contribs: exact contributions need trees of depth at most " + std::to_string(kShapDepth));
    return -1;
  }
  if (approximate) {
    launch(MGB_PROF_PREDICT, k_contribs_approx, dim3(explain_grid(rows, 256)), dim3(256), 0, X, indptr, indices,
           rows, cols, nodes, node_means, tree_offsets, trees, base, base_value, interactions ? 1u : 0u, out);
    MGB_LAUNCH_CHECK("k_contribs_approx");
  } else if (interactions) {
    launch(MGB_PROF_PREDICT, k_interactions_shap, dim3(explain_grid(rows, 64)), dim3(64), 0, X, indptr, indices,
           rows, cols, nodes, node_means, tree_offsets, trees, base, base_value, out);
    MGB_LAUNCH_CHECK("k_interactions_shap");
  } else {
    launch(MGB_PROF_PREDICT, k_contribs_shap, dim3(explain_grid(rows, 64)), dim3(64), 0, X, indptr, indices, rows,
           cols, nodes, node_means, tree_offsets, trees, base, base_value, out);
    MGB_LAUNCH_CHECK("k_contribs_shap");
  }
  return 0;
}

}  // extern "C"
