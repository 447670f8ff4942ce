// Compressed sparse row (CSR) input: the column-major copy the quantile
// sketch reads, per-nonzero bin codes, and prediction (reference
// src/data.cpp:721-870 Matrix::sparse, kernels/sparse_data.metal.h:460-498
// sparse_quantize_csr, kernels/boost.metal:1738-1763 prediction).  Entries
// absent from a row are missing values, like NaN entries of a dense matrix;
// every kernel here requires strictly increasing column indices within a row.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <cmath>

#include "device_common.hpp"

namespace mgb {
namespace {

// row_of[k] = the row that owns nonzero k.
__global__ void k_row_of(const uint64_t* __restrict__ indptr, uint32_t rows, uint32_t* __restrict__ row_of) {
  for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (uint64_t)gridDim.x * blockDim.x)
    for (uint64_t k = indptr[r]; k < indptr[r + 1]; ++k) row_of[k] = r;
}

__global__ void k_iota(uint32_t* __restrict__ p, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = (uint32_t)i;
}

__global__ void k_gather_csc(const uint32_t* __restrict__ perm, const uint32_t* __restrict__ row_of,
                             const float* __restrict__ values, uint64_t nnz, uint32_t* __restrict__ csc_rows,
                             float* __restrict__ csc_values) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nnz; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t k = perm[i];
    csc_rows[i] = row_of[k];
    csc_values[i] = values[k];
  }
}

// colptr[f] = first position of column f in the column-sorted indices.
__global__ void k_colptr(const uint32_t* __restrict__ sorted_cols, uint64_t nnz, uint32_t cols,
                         uint64_t* __restrict__ colptr) {
  for (uint64_t f = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; f <= cols; f += (uint64_t)gridDim.x * blockDim.x) {
    uint64_t lo = 0, hi = nnz;
    while (lo < hi) {
      const uint64_t mid = lo + (hi - lo) / 2;
      if (sorted_cols[mid] < f) lo = mid + 1;
      else hi = mid;
    }
    colptr[f] = lo;
  }
}

// Bin rule of the dense bin matrix: min(#{cuts <= v}, count-1); NaN or a
// feature without cuts -> missing code.
template <typename BinT>
__global__ void k_quantize_csr(const uint32_t* __restrict__ indices, const float* __restrict__ values, uint64_t nnz,
                               const float* __restrict__ cuts, const uint32_t* __restrict__ counts,
                               uint32_t cut_stride, uint32_t missing_code, BinT* __restrict__ codes) {
  for (uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; k < nnz; k += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t f = indices[k];
    const float v = values[k];
    const uint32_t count = counts[f];
    BinT code = (BinT)missing_code;
    if (!isnan(v) && count) {
      const float* column = cuts + (uint64_t)f * cut_stride;
      uint32_t lo = 0, hi = count;
      while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (v >= column[mid]) lo = mid + 1;
        else hi = mid;
      }
      code = (BinT)(lo < count - 1 ? lo : count - 1);
    }
    codes[k] = code;
  }
}

// Position of feature f among a row's sorted column indices, or -1.
__device__ __forceinline__ int64_t find_in_row(const uint32_t* __restrict__ indices, uint64_t begin, uint64_t end,
                                               uint32_t f) {
  uint64_t lo = begin, hi = end;
  while (lo < hi) {
    const uint64_t mid = lo + (hi - lo) / 2;
    if (indices[mid] < f) lo = mid + 1;
    else hi = mid;
  }
  return lo < end && indices[lo] == f ? (int64_t)lo : -1;
}

// The dense predictor's walk (value < threshold, NaN and absent entries
// follow default_left) with each feature looked up in the row.
__global__ void k_predict_csr(const uint64_t* __restrict__ indptr, const uint32_t* __restrict__ indices,
                              const float* __restrict__ values, uint32_t rows, const MgbTreeNode* __restrict__ nodes,
                              const uint32_t* __restrict__ offsets, uint32_t trees, float* __restrict__ margin) {
  for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t b = indptr[r], e = indptr[r + 1];
    float sum = margin[r];
    for (uint32_t t = 0; t < trees; ++t) {
      const MgbTreeNode* tree = nodes + offsets[t];
      int32_t id = 0;
      while (tree[id].left >= 0) {
        const int64_t k = find_in_row(indices, b, e, (uint32_t)tree[id].feature);
        const float v = k < 0 ? __uint_as_float(0x7fc00000u) : values[k];
        const bool left = isnan(v) ? tree[id].default_left != 0 : v < tree[id].threshold;
        id = left ? tree[id].left : tree[id].right;
      }
      sum = sum + tree[id].leaf;
    }
    margin[r] = sum;
  }
}

uint32_t grid_of(uint64_t work, uint32_t block, uint32_t cap) {
  const uint64_t g = (work + block - 1) / block;
  return (uint32_t)(g < 1 ? 1 : (g > cap ? cap : g));
}

struct Scratch {
  void* p = nullptr;
  ~Scratch() { if (p) (void)mgb_free(p); }
  int alloc(size_t bytes) { return mgb_malloc(&p, bytes ? bytes : 16); }
};

}  // namespace
}  // namespace mgb

using namespace mgb;

extern "C" {

int mgb_csr_to_csc(const uint64_t* indptr, const uint32_t* indices, const float* values, uint32_t rows, uint32_t cols,
                   uint64_t nnz, uint64_t* colptr, uint32_t* csc_rows, float* csc_values, uint32_t* csc_cols) {
  if (nnz >= (1ull << 31)) { set_error("mgb_csr_to_csc: more than 2^31 - 1 nonzeros"); return -1; }
  hipStream_t s = stream();
  if (!nnz) {
    hipLaunchKernelGGL(k_colptr, dim3(grid_of(cols + 1, 256, 1024)), dim3(256), 0, s, indices, (uint64_t)0, cols,
                       colptr);
    MGB_LAUNCH_CHECK("k_colptr");
    return 0;
  }
  Scratch row_of, keys_out, perm_in, perm_out, temp;
  if (row_of.alloc(nnz * 4) || keys_out.alloc(nnz * 4) || perm_in.alloc(nnz * 4) || perm_out.alloc(nnz * 4)) return -1;
  hipLaunchKernelGGL(k_row_of, dim3(grid_of(rows, 256, 8192)), dim3(256), 0, s, indptr, rows, (uint32_t*)row_of.p);
  MGB_LAUNCH_CHECK("k_row_of");
  hipLaunchKernelGGL(k_iota, dim3(grid_of(nnz, 256, 8192)), dim3(256), 0, s, (uint32_t*)perm_in.p, nnz);
  MGB_LAUNCH_CHECK("k_iota");
  // Stable LSD radix sort by column: positions of one column keep CSR order,
  // which is row order.
  int end_bit = 1;
  while (end_bit < 32 && (cols - 1) >> end_bit) ++end_bit;
  size_t temp_bytes = 0;
  MGB_CHECK(hipcub::DeviceRadixSort::SortPairs(nullptr, temp_bytes, indices, (uint32_t*)keys_out.p,
                                               (const uint32_t*)perm_in.p, (uint32_t*)perm_out.p, (int)nnz, 0,
                                               end_bit, s));
  if (temp.alloc(temp_bytes)) return -1;
  MGB_CHECK(hipcub::DeviceRadixSort::SortPairs(temp.p, temp_bytes, indices, (uint32_t*)keys_out.p,
                                               (const uint32_t*)perm_in.p, (uint32_t*)perm_out.p, (int)nnz, 0,
                                               end_bit, s));
  hipLaunchKernelGGL(k_gather_csc, dim3(grid_of(nnz, 256, 8192)), dim3(256), 0, s, (const uint32_t*)perm_out.p,
                     (const uint32_t*)row_of.p, values, nnz, csc_rows, csc_values);
  MGB_LAUNCH_CHECK("k_gather_csc");
  hipLaunchKernelGGL(k_colptr, dim3(grid_of(cols + 1, 256, 1024)), dim3(256), 0, s, (const uint32_t*)keys_out.p, nnz,
                     cols, colptr);
  MGB_LAUNCH_CHECK("k_colptr");
  if (csc_cols) MGB_CHECK(hipMemcpyAsync(csc_cols, keys_out.p, nnz * 4, hipMemcpyDeviceToDevice, s));
  MGB_CHECK(hipStreamSynchronize(s));  // the copy is complete when the call returns
  return 0;
}

int mgb_quantize_csr(const uint32_t* indices, const float* values, uint64_t nnz, const float* cuts,
                     const uint32_t* counts, uint32_t cut_stride, uint32_t bin_bytes, uint32_t missing_code,
                     void* codes) {
  if (bin_bytes != 1 && bin_bytes != 2) { set_error("mgb_quantize_csr: bin_bytes must be 1 or 2"); return -1; }
  if (!nnz) return 0;
  const uint32_t grid = grid_of(nnz, 256, 65535);
  if (bin_bytes == 1)
    hipLaunchKernelGGL(k_quantize_csr<uint8_t>, dim3(grid), dim3(256), 0, stream(), indices, values, nnz, cuts,
                       counts, cut_stride, missing_code, (uint8_t*)codes);
  else
    hipLaunchKernelGGL(k_quantize_csr<uint16_t>, dim3(grid), dim3(256), 0, stream(), indices, values, nnz, cuts,
                       counts, cut_stride, missing_code, (uint16_t*)codes);
  MGB_LAUNCH_CHECK("k_quantize_csr");
  return 0;
}

int mgb_predict_csr(const uint64_t* indptr, const uint32_t* indices, const float* values, uint32_t rows,
                    const MgbTreeNode* nodes, const uint32_t* offsets, uint32_t trees, float* margin) {
  if (!rows || !trees) return 0;
  launch(MGB_PROF_PREDICT, k_predict_csr, dim3(grid_of(rows, 256, 8192)), dim3(256), 0, indptr, indices, values,
         rows, nodes, offsets, trees, margin);
  MGB_LAUNCH_CHECK("k_predict_csr");
  return 0;
}

}  // extern "C"
