// Evaluation metrics on the device (reference src/metrics.cpp:8-159).
//
// Elementwise metrics keep the reference's fp32 summation order exactly
// (kernels/boost.metal:2225-2295): each block of 256 rows is summed by the
// pairwise tree v[t] += v[t + d], d = 128 .. 1; one workgroup then sums the
// block results with a compensated (Kahan) sum per thread over blocks
// t, t + 256, ... and the same tree.  With exactly rounded fp32 operations
// (no contraction, IEEE division and square root) the result is bitwise the
// reference's for rmse, mae, error and mape.
//
// AUC and PR-AUC use binary64, which gfx950 has in hardware: sort rows by
// descending prediction (tied predictions, +0 and -0 included, form one
// step), sum (positive weight, negative weight) per step, take the exclusive
// prefix over steps, and add up each step's area (kernels/radix_sort.metal.h:
// 427-790).  With 0/1 labels and unit weights every sum is an integer or a
// half-integer below 2^53, so the area is exact whatever the order of
// additions.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <cmath>

#include "device_common.hpp"

namespace mgb {
namespace {

constexpr uint32_t kMetricBlock = 256;

// log(1 + x) with the rounding of 1 + x compensated (kernels/boost.metal:51).
__device__ __forceinline__ float log1p_compensated(float x) {
  const float y = 1.0f + x;
  return y == 1.0f ? x : logf(y) * x / (y - 1.0f);
}

// Per-row loss of each metric kind (kernels/boost.metal:2245-2264).
__device__ float metric_loss(uint32_t kind, float pred, float label, float parameter) {
  switch (kind) {
    case MGB_METRIC_RMSE: {
      const float d = pred - label;
      return d * d;
    }
    case MGB_METRIC_MAE:
      return fabsf(pred - label);
    case MGB_METRIC_RMSLE: {
      const float d = log1p_compensated(pred) - log1p_compensated(label);
      return d * d;
    }
    case MGB_METRIC_LOGLOSS:
      return -label * logf(fmaxf(pred, 1.0e-16f)) - (1.0f - label) * logf(fmaxf(1.0f - pred, 1.0e-16f));
    case MGB_METRIC_ERROR:  // a fractional label counts partially
      return pred > parameter ? 1.0f - label : label;
    case MGB_METRIC_MAPE:
      return fabsf((pred - label) / label);
    case MGB_METRIC_MPHE: {
      const float z = (pred - label) / parameter;
      return parameter * parameter * (sqrtf(1.0f + z * z) - 1.0f);
    }
    case MGB_METRIC_POISSON:
      return lgammaf(label + 1.0f) + pred - label * logf(fmaxf(pred, 1.0e-16f));
    case MGB_METRIC_GAMMA_DEVIANCE: {
      const float r = label / pred;
      return 2.0f * (-logf(r) + r - 1.0f);
    }
    case MGB_METRIC_TWEEDIE:
      return -label * powf(pred, 1.0f - parameter) / (1.0f - parameter) +
             powf(pred, 2.0f - parameter) / (2.0f - parameter);
    case MGB_METRIC_GAMMA_NLOGLIK:
      return label / pred + logf(pred);
  }
  return 0.0f;
}

// Pairwise tree over the workgroup's 256 pairs; the result is in thread 0.
// Steps d = 128 and 64 cross waves through LDS; d = 32 .. 1 run inside wave 0
// with lane shuffles (lane t adds lane t + d, as the LDS form does).
__device__ __forceinline__ float2 block_tree(float2 v, float2* lds) {
  const uint32_t t = threadIdx.x;
  lds[t] = v;
  __syncthreads();
  for (uint32_t d = 128; d >= 64; d >>= 1) {
    if (t < d) {
      const float2 o = lds[t + d];
      lds[t] = make_float2(lds[t].x + o.x, lds[t].y + o.y);
    }
    __syncthreads();
  }
  if (t < kWave) {
    v = lds[t];
    for (int d = 32; d > 0; d >>= 1) {
      const float ox = __shfl_down(v.x, d, kWave), oy = __shfl_down(v.y, d, kWave);
      v = make_float2(v.x + ox, v.y + oy);
    }
  }
  return v;
}

__global__ __launch_bounds__(kMetricBlock) void k_metric_partial(const float* __restrict__ pred,
                                                                 const float* __restrict__ labels,
                                                                 const float* __restrict__ weights, uint32_t rows,
                                                                 uint32_t kind, float parameter,
                                                                 float2* __restrict__ partial) {
  __shared__ float2 lds[kMetricBlock];
  const uint64_t i = (uint64_t)blockIdx.x * kMetricBlock + threadIdx.x;
  float2 v = make_float2(0.0f, 0.0f);
  if (i < rows) {
    const float w = weights ? weights[i] : 1.0f;
    v = make_float2(w * metric_loss(kind, pred[i], labels[i], parameter), w);
  }
  v = block_tree(v, lds);
  if (threadIdx.x == 0) partial[blockIdx.x] = v;
}

__global__ __launch_bounds__(kMetricBlock) void k_metric_reduce(const float2* __restrict__ partial, uint32_t blocks,
                                                                float2* __restrict__ out) {
  __shared__ float2 lds[kMetricBlock];
  float2 sum = make_float2(0.0f, 0.0f), c = make_float2(0.0f, 0.0f);
  for (uint32_t i = threadIdx.x; i < blocks; i += kMetricBlock) {
    const float2 p = partial[i];
    const float2 y = make_float2(p.x - c.x, p.y - c.y);
    const float2 next = make_float2(sum.x + y.x, sum.y + y.y);
    c = make_float2((next.x - sum.x) - y.x, (next.y - sum.y) - y.y);
    sum = next;
  }
  sum = block_tree(sum, lds);
  if (threadIdx.x == 0) out[0] = sum;
}

// ---- AUC ------------------------------------------------------------------
struct Mass {
  double tp, fp;  // positive and negative weight
};
struct MassSum {
  __host__ __device__ Mass operator()(const Mass& a, const Mass& b) const { return Mass{a.tp + b.tp, a.fp + b.fp}; }
};

// Ascending uint32 keys for descending prediction order; +0 and -0 share one.
__global__ void k_auc_keys(const float* __restrict__ pred, uint32_t rows, uint32_t* __restrict__ keys,
                           uint32_t* __restrict__ index) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < rows; i += (uint64_t)gridDim.x * blockDim.x) {
    uint32_t b = __float_as_uint(pred[i]);
    if ((b & 0x7fffffffu) == 0) b = 0;
    const uint32_t ascending = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    keys[i] = ~ascending;
    index[i] = i;
  }
}

// (label * weight, (1 - label) * weight), each an fp32 product widened to
// binary64 (kernels/radix_sort.metal.h:316-323).
__global__ void k_auc_mass(const uint32_t* __restrict__ order, const float* __restrict__ labels,
                           const float* __restrict__ weights, uint32_t rows, Mass* __restrict__ mass) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < rows; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t r = order[i];
    const float y = labels[r], w = weights ? weights[r] : 1.0f;
    mass[i] = Mass{(double)fabsf(y * w), (double)fabsf((1.0f - y) * w)};
  }
}

// 1 - log(1 + u) / u for 0 < u <= 1/4 by its alternating series
// u/2 - u^2/3 + u^3/4 - ..., free of the cancellation of the direct form.
__device__ double one_minus_log1p_ratio(double u) {
  double term = u, sum = 0.0;
  for (int k = 1; k <= 40; ++k) {
    const double add = term / (double)(k + 1);
    sum = (k & 1) ? sum + add : sum - add;
    term *= u;
  }
  return sum;
}

// Area under the precision-recall curve over one step of `step` weight that
// follows `previous` cumulative weight: recall rises by step.tp / positives
// while precision moves along the straight line between the two (TP, FP)
// points; the integral of precision over that rise is
// rise * (r * L + q * (1 - L)) with r = TP / (TP + FP) before the step,
// q = step.tp / step mass, L = log(1 + u) / u and u = step mass / (TP + FP).
__device__ double pr_step_area(Mass previous, Mass step, double positives) {
  if (step.tp == 0.0 || positives == 0.0) return 0.0;
  const double mass = step.tp + step.fp;
  if (mass == 0.0) return 0.0;
  const double rise = step.tp / positives, q = step.tp / mass;
  const double cumulative = previous.tp + previous.fp;
  if (cumulative == 0.0) return rise * q;
  const double r = previous.tp / cumulative;
  double retained, added;
  if (mass <= cumulative) {
    const double u = mass / cumulative;
    if (u <= 0.25) {
      added = one_minus_log1p_ratio(u);
      retained = 1.0 - added;
    } else {
      retained = log1p(u) / u;
      added = 1.0 - retained;
    }
  } else {
    const double v = cumulative / mass;  // L = v * (log(1 + v) - log(v))
    retained = v == 0.0 ? 0.0 : v * (log1p(v) - log(v));
    added = 1.0 - retained;
  }
  return rise * (r * retained + q * added);
}

// Area of each step (ROC: trapezoid fp * (2 TP + tp) / 2); step `runs` holds
// nothing and the last slot receives the class totals.
__global__ void k_auc_area(const Mass* __restrict__ steps, const Mass* __restrict__ before,
                           const uint32_t* __restrict__ runs_ptr, int pr, double* __restrict__ area,
                           Mass* __restrict__ totals) {
  const uint32_t runs = *runs_ptr;
  const Mass last_before = before[runs - 1], last = steps[runs - 1];
  const double positives = last_before.tp + last.tp;
  for (uint64_t s = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; s < runs; s += (uint64_t)gridDim.x * blockDim.x) {
    const Mass step = steps[s], prev = before[s];
    area[s] = pr ? pr_step_area(prev, step, positives) : step.fp * (2.0 * prev.tp + step.tp) * 0.5;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) *totals = Mass{positives, last_before.fp + last.fp};
}

uint32_t grid_of(uint64_t work, uint32_t block, uint32_t cap) {
  const uint64_t g = (work + block - 1) / block;
  return (uint32_t)(g < 1 ? 1 : (g > cap ? cap : g));
}

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

// Workspace carve-up for AUC over n rows; temp = the largest hipcub scratch.
struct AucLayout {
  size_t keys_in, keys_out, index_in, index_out, mass, unique, steps, before, area, runs, totals, sum, temp, temp_bytes,
      total;
};

int auc_layout(uint32_t n, AucLayout& L) {
  size_t sort_bytes = 0, rbk_bytes = 0, scan_bytes = 0, sum_bytes = 0;
  MGB_CHECK(hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                                               (const uint32_t*)nullptr, (uint32_t*)nullptr, (int)n, 0, 32,
                                               stream()));
  MGB_CHECK(hipcub::DeviceReduce::ReduceByKey(nullptr, rbk_bytes, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                                              (const Mass*)nullptr, (Mass*)nullptr, (uint32_t*)nullptr, MassSum(),
                                              (int)n, stream()));
  MGB_CHECK(hipcub::DeviceScan::ExclusiveScan(nullptr, scan_bytes, (const Mass*)nullptr, (Mass*)nullptr, MassSum(),
                                              Mass{0.0, 0.0}, (int)n, stream()));
  MGB_CHECK(hipcub::DeviceReduce::Sum(nullptr, sum_bytes, (const double*)nullptr, (double*)nullptr, (int)n,
                                      stream()));
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align_up(bytes);
    return at;
  };
  L.keys_in = take((size_t)n * 4);
  L.keys_out = take((size_t)n * 4);
  L.index_in = take((size_t)n * 4);
  L.index_out = take((size_t)n * 4);
  L.mass = take((size_t)n * sizeof(Mass));
  L.unique = take((size_t)n * 4);
  L.steps = take((size_t)n * sizeof(Mass));
  L.before = take((size_t)n * sizeof(Mass));
  L.area = take((size_t)n * 8);
  L.runs = take(4);
  L.totals = take(sizeof(Mass));
  L.sum = take(8);
  size_t temp = sort_bytes;
  for (size_t b : {rbk_bytes, scan_bytes, sum_bytes}) temp = b > temp ? b : temp;
  L.temp_bytes = temp ? temp : 16;
  L.temp = take(L.temp_bytes);
  L.total = off;
  return 0;
}

}  // namespace
}  // namespace mgb

using namespace mgb;

extern "C" {

size_t mgb_metric_workspace_bytes(uint32_t rows) {
  const size_t n = rows ? rows : 1;
  const size_t partial = ((n + kMetricBlock - 1) / kMetricBlock + 1) * sizeof(float2) + 256;
  AucLayout L{};
  if (auc_layout((uint32_t)n, L) != 0) return 0;
  return L.total > partial ? L.total : partial;
}

int mgb_metric_sum(const float* pred, const float* labels, const float* weights, uint32_t rows, uint32_t kind,
                   float parameter, float* out, void* workspace, size_t workspace_bytes) {
  if (kind > MGB_METRIC_GAMMA_NLOGLIK || kind == 4 || kind == 5) {
    set_error("mgb_metric_sum: unknown metric kind");
    return -1;
  }
  const uint32_t blocks = (uint32_t)(((uint64_t)rows + kMetricBlock - 1) / kMetricBlock);
  const size_t need = ((size_t)blocks + 1) * sizeof(float2);
  if (!workspace || workspace_bytes < need) {
    set_error("mgb_metric_sum: workspace too small");
    return -1;
  }
  float2* partial = (float2*)workspace;
  float2* result = partial + blocks;
  hipStream_t s = stream();
  if (blocks)
    hipLaunchKernelGGL(k_metric_partial, dim3(blocks), dim3(kMetricBlock), 0, s, pred, labels, weights, rows, kind,
                       parameter, partial);
  MGB_LAUNCH_CHECK("k_metric_partial");
  hipLaunchKernelGGL(k_metric_reduce, dim3(1), dim3(kMetricBlock), 0, s, (const float2*)partial, blocks, result);
  MGB_LAUNCH_CHECK("k_metric_reduce");
  MGB_CHECK(hipMemcpyAsync(out, result, sizeof(float2), hipMemcpyDeviceToHost, s));
  MGB_CHECK(hipStreamSynchronize(s));
  return 0;
}

int mgb_metric_auc(const float* pred, const float* labels, const float* weights, uint32_t rows, int pr, double* out,
                   void* workspace, size_t workspace_bytes) {
  if (!rows) {
    out[0] = out[1] = out[2] = 0.0;
    return 0;
  }
  if (rows > 0x7fffffffu) {
    set_error("mgb_metric_auc: more than 2^31 - 1 rows");
    return -1;
  }
  AucLayout L{};
  if (auc_layout(rows, L) != 0) return -1;
  if (!workspace || workspace_bytes < L.total) {
    set_error("mgb_metric_auc: workspace too small");
    return -1;
  }
  char* w = (char*)workspace;
  auto at = [&](size_t off) { return (void*)(w + off); };
  uint32_t *keys_in = (uint32_t*)at(L.keys_in), *keys_out = (uint32_t*)at(L.keys_out);
  uint32_t *index_in = (uint32_t*)at(L.index_in), *index_out = (uint32_t*)at(L.index_out);
  Mass *mass = (Mass*)at(L.mass), *steps = (Mass*)at(L.steps), *before = (Mass*)at(L.before);
  uint32_t *unique = (uint32_t*)at(L.unique), *runs = (uint32_t*)at(L.runs);
  double *area = (double*)at(L.area), *sum = (double*)at(L.sum);
  Mass* totals = (Mass*)at(L.totals);
  void* temp = at(L.temp);
  size_t temp_bytes = L.temp_bytes;
  hipStream_t s = stream();
  const uint32_t grid = grid_of(rows, 256, 8192);
  hipLaunchKernelGGL(k_auc_keys, dim3(grid), dim3(256), 0, s, pred, rows, keys_in, index_in);
  MGB_LAUNCH_CHECK("k_auc_keys");
  MGB_CHECK(hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, (const uint32_t*)keys_in, keys_out,
                                               (const uint32_t*)index_in, index_out, (int)rows, 0, 32, s));
  hipLaunchKernelGGL(k_auc_mass, dim3(grid), dim3(256), 0, s, (const uint32_t*)index_out, labels, weights, rows,
                     mass);
  MGB_LAUNCH_CHECK("k_auc_mass");
  temp_bytes = L.temp_bytes;
  MGB_CHECK(hipcub::DeviceReduce::ReduceByKey(temp, temp_bytes, (const uint32_t*)keys_out, unique,
                                              (const Mass*)mass, steps, runs, MassSum(), (int)rows, s));
  uint32_t host_runs = 0;
  MGB_CHECK(hipMemcpyAsync(&host_runs, runs, 4, hipMemcpyDeviceToHost, s));
  MGB_CHECK(hipStreamSynchronize(s));
  if (host_runs == 0 || host_runs > rows) {
    set_error("mgb_metric_auc: invalid step count");
    return -1;
  }
  temp_bytes = L.temp_bytes;
  MGB_CHECK(hipcub::DeviceScan::ExclusiveScan(temp, temp_bytes, (const Mass*)steps, before, MassSum(),
                                              Mass{0.0, 0.0}, (int)host_runs, s));
  hipLaunchKernelGGL(k_auc_area, dim3(grid_of(host_runs, 256, 8192)), dim3(256), 0, s, (const Mass*)steps,
                     (const Mass*)before, (const uint32_t*)runs, pr, area, totals);
  MGB_LAUNCH_CHECK("k_auc_area");
  temp_bytes = L.temp_bytes;
  MGB_CHECK(hipcub::DeviceReduce::Sum(temp, temp_bytes, (const double*)area, sum, (int)host_runs, s));
  Mass t{};
  MGB_CHECK(hipMemcpyAsync(out, sum, 8, hipMemcpyDeviceToHost, s));
  MGB_CHECK(hipMemcpyAsync(&t, totals, sizeof(Mass), hipMemcpyDeviceToHost, s));
  MGB_CHECK(hipStreamSynchronize(s));
  out[1] = t.tp;
  out[2] = t.fp;
  return 0;
}

}  // extern "C"
