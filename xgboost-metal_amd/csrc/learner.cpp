#include "learner.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <iomanip>
#include <limits>
#include <sstream>

namespace mgb {

void require(bool ok, const std::string& message) {
  if (!ok) throw Error(message);
}

void kcheck(int status, const char* what) {
  if (status != 0) throw Error(std::string(what) + ": " + mgb_last_error());
}

// ---------------------------------------------------------------------------
// DeviceBuffer
// ---------------------------------------------------------------------------
void DeviceBuffer::resize(size_t bytes) {
  release();
  kcheck(mgb_malloc(&ptr_, bytes ? bytes : 16), "device allocation");
  bytes_ = bytes;
}
void DeviceBuffer::upload(const void* host, size_t bytes) {
  ensure(bytes);
  kcheck(mgb_memcpy_h2d(ptr_, host, bytes), "host-to-device copy");
}
void DeviceBuffer::download(void* host, size_t bytes) const {
  kcheck(mgb_memcpy_d2h(host, ptr_, bytes), "device-to-host copy");
}
void DeviceBuffer::release() {
  if (ptr_) mgb_free(ptr_);
  ptr_ = nullptr;
  bytes_ = 0;
}

// ---------------------------------------------------------------------------
// DMatrix (src/data.cpp:414-491 dense ingest, :1210-1306 quantize)
// ---------------------------------------------------------------------------
static uint64_t next_matrix_id() {
  static std::mutex m;
  static uint64_t id = 0;
  std::lock_guard<std::mutex> lock(m);
  return ++id;
}

DMatrix::DMatrix() : id(next_matrix_id()) {}

void DMatrix::upload() {
  if (data_uploaded) return;
  if (sparse) {
    d_indptr.upload(indptr.data(), indptr.size() * sizeof(uint64_t));
    d_indices.upload(indices.data(), indices.size() * sizeof(uint32_t));
    d_values.upload(values.data(), values.size() * sizeof(float));
  } else {
    d_data.upload(data.data(), data.size() * sizeof(float));
  }
  data_uploaded = true;
}

uint64_t DMatrix::nonmissing() const {
  uint64_t n = 0;
  for (float x : sparse ? values : data) n += !std::isnan(x);
  return n;
}

void DMatrix::upload_info() {
  if (!labels_uploaded && !labels.empty()) {
    d_labels.upload(labels.data(), labels.size() * sizeof(float));
    labels_uploaded = true;
  }
  if (!weights_uploaded && !weights.empty()) {
    d_weights.upload(weights.data(), weights.size() * sizeof(float));
    weights_uploaded = true;
  }
}

void DMatrix::set_info(const std::string& field, const float* values, size_t count) {
  std::vector<float> v(values, values + count);
  if (field == "label") { labels = std::move(v); labels_uploaded = false; labels_in_unit = -1; }
  else if (field == "weight") {
    weights = std::move(v);
    weights_uploaded = false;
    quantized_max_bin = 0;  // the sketch is weighted
  } else if (field == "base_margin") base_margin = std::move(v);
  else if (field == "label_lower_bound" || field == "label_upper_bound" || field == "feature_weights" ||
           field == "group_ptr" || field == "qid")
    throw Error("Field '" + field + "' is not supported by this engine (single-output hist regression and "
                "binary classification).");
  else throw Error("Unknown float field: " + field);
}

const std::vector<float>& DMatrix::get_info(const std::string& field) const {
  if (field == "label") return labels;
  if (field == "weight") return weights;
  if (field == "base_margin") return base_margin;
  throw Error("Unknown float field: " + field);
}

static uint32_t next_pow2(uint32_t v) {
  uint32_t p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Features per histogram workgroup: the largest power of two (at most 16, at
// most the feature count rounded up) whose LDS histogram (16 bytes per bin)
// fits in the 160 KB of a CU.  Wider groups cut the bytes each row-major row
// costs the L2->L1 path per workgroup; on 10M x 128 rows with 1024 bins, 8
// features (one workgroup per CU) build the histograms 1.7x faster than 4
// (two per CU).  A request (hip_histogram_features) overrides the rule.
uint32_t DMatrix::choose_group(uint32_t request) const {
  if (request) {
    require(request <= 16 && (request & (request - 1)) == 0, "hip_histogram_features must be 1, 2, 4, 8 or 16.");
    require((size_t)request * (hist_bins + 1) * 16 <= 160 * 1024,
            "hip_histogram_features: the feature group's histogram does not fit in 160 KB of LDS.");
    return request;
  }
  // About eight feature groups per matrix: a tile's LDS atomics all run on
  // the one CU that holds the tile, and below the root a level has few row
  // tiles, so more groups put more CUs to work; fewer features per group than
  // that repeat each row's id, gradient and code-line reads for little gain.
  // Measured: 262,144 x 64 histograms 18% faster at 8 than at 16 features and
  // slower at 4; 100,000 x 32 fastest at 4; 10M x 128 (1024 bins) 1.7x faster
  // at 8 than at 4.
  uint32_t G = 16;
  while (G > 1 && (G > cols / 8 || (size_t)G * (hist_bins + 1) * 16 > 160 * 1024)) G >>= 1;
  return std::min(G, next_pow2(cols));
}

void DMatrix::quantize(uint32_t max_bin, int layout, uint32_t group_request) {
  require(max_bin >= 2, "max_bin must be at least 2.");
  require(layout >= 0 && layout <= 2, "hip_bin_layout must be auto, row or group.");
  if (sparse) {
    // One layout: codes per nonzero (the CSR structure is the layout).
    if (quantized_max_bin != max_bin) quantize_sparse(max_bin);
    quantized_layout = layout;
    quantized_group_request = group_request;
    return;
  }
  if (quantized_max_bin == max_bin) {
    if (quantized_layout == layout && quantized_group_request == group_request) return;
    const uint32_t G = choose_group(group_request);
    features_per_group = G;
    matrix.group_features = G;
    quantized_group_request = group_request;
    relayout(layout);
    return;
  }
  require(!is_quantile || quantile_max_bin == max_bin, "Inconsistent max_bin between QuantileDMatrix and Booster.");
  require(cols > 0, "Data must contain at least one feature.");
  if (rows == 0) return quantize_empty(max_bin, layout, group_request);
  upload();
  upload_info();
  auto t0 = std::chrono::steady_clock::now();
  hist_bins = std::max(1u, std::min(max_bin, rows));
  d_cuts.ensure((size_t)cols * max_bin * sizeof(float));
  d_counts.ensure((size_t)cols * sizeof(uint32_t));
  if (cut_source) {
    take_cuts(max_bin);
  } else {
    const float* w = weights.empty() ? nullptr : d_weights.as<float>();
    kcheck(mgb_sketch_cuts(d_data.as<float>(), rows, cols, w, max_bin, d_cuts.as<float>(), d_counts.as<uint32_t>()),
           "quantile sketch");
    counts_host.resize(cols);
    cuts_host.resize((size_t)cols * max_bin);
    d_counts.download(counts_host.data(), cols * sizeof(uint32_t));
    d_cuts.download(cuts_host.data(), cuts_host.size() * sizeof(float));
  }
  auto t1 = std::chrono::steady_clock::now();
  uint32_t max_count = 0;
  for (auto c : counts_host) max_count = std::max(max_count, c);
  hist_bins = std::max(hist_bins, max_count);  // a reference matrix's cuts may outnumber these rows
  require(max_count <= hist_bins, "internal error: more cuts than histogram bins");
  d_missing.ensure(sizeof(uint32_t));
  kcheck(mgb_memset(d_missing.get(), 0, sizeof(uint32_t)), "memset");
  kcheck(mgb_any_missing(d_data.as<float>(), (uint64_t)rows * cols, d_missing.as<uint32_t>()), "missing scan");
  uint32_t missing = 0;
  d_missing.download(&missing, sizeof(missing));
  has_missing = missing != 0;
  // u8 codes when every bin fits in a byte: with missing values 0xFF is the
  // missing code (so at most 255 bins); a matrix without missing values uses
  // all 256 codes and a missing code no byte can equal.
  uint32_t bin_bytes = (has_missing ? max_count <= 255 : max_count <= 256) ? 1 : 2;
  const uint32_t G = choose_group(group_request);
  features_per_group = G;
  quantized_group_request = group_request;
  matrix.rows = rows;
  matrix.cols = cols;
  matrix.bin_bytes = bin_bytes;
  matrix.max_bin = hist_bins;
  matrix.cut_stride = max_bin;
  matrix.missing_code = !has_missing ? 0xFFFFFFFFu : (bin_bytes == 1 ? 0xFFu : 0xFFFFu);
  matrix.group_features = G;
  quantized_max_bin = max_bin;
  sketch_seconds += std::chrono::duration<double>(t1 - t0).count();
  relayout(layout);
}

// A matrix without rows (the reference trains on one, tests/test_gpu_tree.py:
// 51-52): every feature's summary is empty, whose cuts are the tail sentinel
// of a zero maximum, 0 + (|0| + 1e-5) (kernels/quantile.metal.h:367, the
// sketch's empty case); a reference matrix's cuts are taken as they are.
// There is nothing to bin and no device work.
void DMatrix::quantize_empty(uint32_t max_bin, int layout, uint32_t group_request) {
  if (cut_source) {
    take_cuts(max_bin);
  } else {
    counts_host.assign(cols, 1u);
    cuts_host.assign((size_t)cols * max_bin, 0.0f);
    for (uint32_t f = 0; f < cols; ++f) cuts_host[(size_t)f * max_bin] = 1e-5f;
  }
  uint32_t max_count = 1;
  for (auto c : counts_host) max_count = std::max(max_count, c);
  hist_bins = max_count;
  has_missing = false;
  matrix = MgbMatrix{};
  matrix.cols = cols;
  matrix.max_bin = hist_bins;
  matrix.cut_stride = max_bin;
  quantized_max_bin = max_bin;
  quantized_layout = layout;
  quantized_group_request = group_request;
}

// Cuts of the reference matrix (QuantileDMatrix ref=, src/c_api.cpp:225-239):
// evaluation data binned exactly like the training data.
void DMatrix::take_cuts(uint32_t max_bin) {
  DMatrix& src = *cut_source;
  require(src.cols == cols, "The reference DMatrix has " + std::to_string(src.cols) + " features, this one " +
                                std::to_string(cols) + ".");
  src.quantize(max_bin, src.quantized_layout, src.quantized_group_request);
  counts_host = src.counts_host;
  cuts_host = src.cuts_host;
  d_cuts.upload(cuts_host.data(), cuts_host.size() * sizeof(float));
  d_counts.upload(counts_host.data(), counts_host.size() * sizeof(uint32_t));
}

// CSR matrices (src/data.cpp:721-870): the sketch reads a column-major copy
// of the nonzeros (each column in row order, so the cuts equal the dense
// matrix's with NaN at the absent entries); the bins are one code per nonzero.
void DMatrix::quantize_sparse(uint32_t max_bin) {
  require(!is_quantile || quantile_max_bin == max_bin, "Inconsistent max_bin between QuantileDMatrix and Booster.");
  require(cols > 0, "Data must contain at least one feature.");
  if (rows == 0) return quantize_empty(max_bin, quantized_layout, quantized_group_request);
  const uint64_t nnz = values.size();
  require(nnz < (1ull << 31), "CSR matrices are limited to 2^31 - 1 stored entries.");
  upload();
  upload_info();
  auto t0 = std::chrono::steady_clock::now();
  hist_bins = std::max(1u, std::min(max_bin, rows));
  d_cuts.ensure((size_t)cols * max_bin * sizeof(float));
  d_counts.ensure((size_t)cols * sizeof(uint32_t));
  // Column-major copy: the sketch's input, and (with its codes) the root
  // histogram's.
  DeviceBuffer csc_values, csc_cols;
  d_colptr.ensure(((size_t)cols + 1) * sizeof(uint64_t));
  d_csc_rows.ensure(std::max<size_t>(nnz, 1) * sizeof(uint32_t));
  csc_values.ensure(std::max<size_t>(nnz, 1) * sizeof(float));
  csc_cols.ensure(std::max<size_t>(nnz, 1) * sizeof(uint32_t));
  kcheck(mgb_csr_to_csc(d_indptr.as<uint64_t>(), d_indices.as<uint32_t>(), d_values.as<float>(), rows, cols, nnz,
                        d_colptr.as<uint64_t>(), d_csc_rows.as<uint32_t>(), csc_values.as<float>(),
                        csc_cols.as<uint32_t>()),
         "CSR column copy");
  if (cut_source) {
    take_cuts(max_bin);
  } else {
    const float* w = weights.empty() ? nullptr : d_weights.as<float>();
    kcheck(mgb_sketch_cuts_csc(csc_values.as<float>(), d_csc_rows.as<uint32_t>(), d_colptr.as<uint64_t>(), rows,
                               cols, w, max_bin, d_cuts.as<float>(), d_counts.as<uint32_t>()),
           "quantile sketch");
    counts_host.resize(cols);
    cuts_host.resize((size_t)cols * max_bin);
    d_counts.download(counts_host.data(), cols * sizeof(uint32_t));
    d_cuts.download(cuts_host.data(), cuts_host.size() * sizeof(float));
  }
  auto t1 = std::chrono::steady_clock::now();
  uint32_t max_count = 0;
  for (auto c : counts_host) max_count = std::max(max_count, c);
  hist_bins = std::max(hist_bins, max_count);
  require(max_count <= hist_bins, "internal error: more cuts than histogram bins");
  // Absent entries carry no code, so a missing code is needed only for
  // stored NaN entries: without them 256 cuts still fit u8 codes.
  const bool stored_nan = nonmissing() < nnz;
  has_missing = nnz < (uint64_t)rows * cols || stored_nan;
  const uint32_t bin_bytes = (stored_nan ? max_count <= 255 : max_count <= 256) ? 1 : 2;
  matrix = MgbMatrix{};
  matrix.rows = rows;
  matrix.cols = cols;
  matrix.bin_bytes = bin_bytes;
  matrix.max_bin = hist_bins;
  matrix.cut_stride = max_bin;
  matrix.missing_code = !stored_nan ? 0xFFFFFFFFu : (bin_bytes == 1 ? 0xFFu : 0xFFFFu);
  matrix.group_features = 1;
  features_per_group = 1;
  csr = MgbCsrMatrix{rows, cols, hist_bins, max_bin, bin_bytes, matrix.missing_code, nnz};
  d_codes.ensure(std::max<size_t>(nnz, 1) * bin_bytes);
  kcheck(mgb_quantize_csr(d_indices.as<uint32_t>(), d_values.as<float>(), nnz, d_cuts.as<float>(),
                          d_counts.as<uint32_t>(), max_bin, bin_bytes, matrix.missing_code, d_codes.get()),
         "CSR codes");
  d_csc_codes.ensure(std::max<size_t>(nnz, 1) * bin_bytes);
  kcheck(mgb_quantize_csr(csc_cols.as<uint32_t>(), csc_values.as<float>(), nnz, d_cuts.as<float>(),
                          d_counts.as<uint32_t>(), max_bin, bin_bytes, matrix.missing_code, d_csc_codes.get()),
         "CSR column codes");
  kcheck(mgb_synchronize(), "synchronize");
  quantized_max_bin = max_bin;
  sketch_seconds += std::chrono::duration<double>(t1 - t0).count();
  quantize_seconds += std::chrono::duration<double>(std::chrono::steady_clock::now() - t1).count();
}

// Bin matrix in the requested layout (the cuts stay).  Row-major is the
// default (auto): below the root the histogram gathers rows by index, and a
// row's codes then share one cache line that every feature group's workgroup
// reuses from L2.  Group-major (each group's codes contiguous over rows) is
// faster only for the dense root level; measured on 10M x 128 u16 bins, it
// halves the root pass but doubles the deeper gathered levels.
void DMatrix::relayout(int layout) {
  auto t0 = std::chrono::steady_clock::now();
  const uint32_t G = features_per_group, groups = (cols + G - 1) / G;
  const uint32_t gbytes = G * matrix.bin_bytes;
  const bool group_major = layout == 2;
  matrix.row_stride = group_major ? gbytes : groups * gbytes;
  matrix.group_stride = group_major ? (uint64_t)rows * gbytes : gbytes;
  d_bins.ensure((size_t)rows * groups * gbytes);
  kcheck(mgb_memset(d_missing.get(), 0, sizeof(uint32_t)), "memset");
  // With the column-major copy (one feature's codes contiguous over rows):
  // the row partition reads a single feature per node, 1-2 bytes a row
  // instead of a cache line of the row-major matrix.
  d_columns.ensure((size_t)rows * cols * matrix.bin_bytes);
  kcheck(mgb_quantize_bins_columns(d_data.as<float>(), d_cuts.as<float>(), d_counts.as<uint32_t>(), &matrix,
                                   d_bins.get(), d_columns.get(), d_missing.as<uint32_t>()),
         "bin matrix");
  kcheck(mgb_synchronize(), "synchronize");
  quantize_seconds += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  quantized_layout = layout;
}

// ---------------------------------------------------------------------------
// Learner
// ---------------------------------------------------------------------------
Learner::Learner() = default;
Learner::~Learner() = default;

static const std::map<std::string, std::string>& aliases() {
  static const std::map<std::string, std::string> a = {
      {"eta", "learning_rate"}, {"lambda", "reg_lambda"}, {"alpha", "reg_alpha"}, {"gamma", "min_split_loss"},
      {"random_state", "seed"}, {"n_jobs", "nthread"}};
  return a;
}

void Learner::set_param(const std::string& name, const std::string& value) {
  std::string key = name;
  auto it = aliases().find(name);
  if (it != aliases().end()) key = it->second;
  if (key == "eval_metric") {  // a list: each value once, in order (src/learner.cpp:119-126)
    if (std::find(metrics.begin(), metrics.end(), value) == metrics.end()) metrics.push_back(value);
    return;
  }
  params_[key] = value;
}

std::string Learner::param(const std::string& name, const std::string& fallback) const {
  auto it = params_.find(name);
  return it == params_.end() ? fallback : it->second;
}

double Learner::number(const std::string& name, double fallback) const {
  auto it = params_.find(name);
  if (it == params_.end()) return fallback;
  try {
    return std::stod(it->second);
  } catch (...) {
    throw Error("Invalid numeric value for " + name + ": " + it->second);
  }
}

// Float parameters parse straight to binary32, as XGBoost's parameter parser does.
float Learner::fnumber(const std::string& name, float fallback) const {
  auto it = params_.find(name);
  if (it == params_.end()) return fallback;
  try {
    return std::stof(it->second);
  } catch (...) {
    throw Error("Invalid numeric value for " + name + ": " + it->second);
  }
}

int64_t Learner::integer(const std::string& name, int64_t fallback) const {
  auto it = params_.find(name);
  if (it == params_.end()) return fallback;
  try {
    return (int64_t)std::stod(it->second);
  } catch (...) {
    throw Error("Invalid integer value for " + name + ": " + it->second);
  }
}

std::string Learner::objective_name() const { return param("objective", "reg:squarederror"); }

// Objective codes as in the reference (src/learner.cpp objective map).
int Learner::objective() const {
  auto name = objective_name();
  if (name == "reg:squarederror") return 0;
  if (name == "binary:logistic" || name == "reg:logistic") return 1;
  if (name == "binary:logitraw") return 2;
  throw Error("Objective is not implemented by the HIP hist engine: " + name);
}

void Learner::configure_check() const {
  (void)objective();
  auto method = param("tree_method", "hist");
  require(method == "hist" || method == "auto" || method == "approx",
          "This engine implements tree_method='hist' only, got '" + method + "'.");
  require(param("booster", "gbtree") == "gbtree", "Only booster='gbtree' is supported.");
  require(param("grow_policy", "depthwise") == "depthwise", "Only grow_policy='depthwise' is supported.");
  require(param("multi_strategy", "one_output_per_tree") == "one_output_per_tree",
          "Only multi_strategy='one_output_per_tree' is supported.");
  require(integer("num_parallel_tree", 1) == 1, "num_parallel_tree must be 1.");
  require(integer("max_leaves", 0) == 0, "max_leaves is not supported (depthwise growth only).");
  auto depth = integer("max_depth", 6);
  require(depth >= 1 && depth <= 16, "max_depth must be in [1, 16].");
  for (auto key : {"subsample", "colsample_bytree"}) {
    const double v = number(key, 1);
    require(v > 0 && v <= 1, std::string(key) + " must be in (0, 1].");
  }
  for (auto key : {"colsample_bylevel", "colsample_bynode"})
    require(number(key, 1) == 1.0, std::string(key) + " < 1 is not supported yet.");
  require(param("sampling_method", "uniform") == "uniform", "Only sampling_method='uniform' is supported.");
  require(param("interaction_constraints", "").empty() || param("interaction_constraints", "") == "[]",
          "interaction_constraints are not supported yet.");
  for (auto key : {"reg_lambda", "reg_alpha", "min_child_weight", "min_split_loss", "max_delta_step", "learning_rate",
                   "scale_pos_weight"})
    require(number(key, 0) >= 0, std::string("Parameter must be nonnegative: ") + key);
  auto bins = integer("max_bin", 256);
  require(bins >= 2 && bins <= 4096, "max_bin must be in [2, 4096].");
}

float Learner::base_margin_value() const {
  int obj = objective();
  float value = base_score;
  if (obj == 1) {
    // src/objectives.cpp:17-31 (score_margins).
    value = std::min(std::max(value, 1.0e-6f), 1.0f - 1.0e-6f);
    value = -std::log(1.0f / value - 1.0f);
  }
  return value;
}

void Learner::initialize(DMatrix& data, bool custom) {
  if (initialized) {
    require(num_feature == data.cols, "Number of columns does not match the trained model.");
    return;
  }
  num_feature = data.cols;
  // Feature metadata is not taken from a matrix without rows
  // (src/learner.cpp:297-298).
  if (data.rows) {
    feature_names = data.feature_names;
    feature_types = data.feature_types;
  }
  int obj = objective();
  auto given = params_.find("base_score");
  if (given != params_.end()) {
    base_score = std::stof(given->second);
  } else if (custom) {
    base_score = 0.5f;
  } else if (data.rows == 0) {
    // The weighted mean of no labels: 0 for squared error, else 0.5 (the
    // rule mgb_base_score applies when the weight sum is not positive).
    base_score = obj == 0 ? 0.0f : 0.5f;
    if (obj == 2) base_score = 0.0f;  // logit(0.5)
  } else {
    // src/learner.cpp:316-333: weighted label mean on the device.
    d_base_.ensure(sizeof(float));
    const float* w = data.weights.empty() ? nullptr : data.d_weights.as<float>();
    kcheck(mgb_base_score(data.d_labels.as<float>(), w, data.rows, (uint32_t)obj, fnumber("scale_pos_weight", 1.0f),
                          d_base_.as<float>()),
           "base score");
    d_base_.download(&base_score, sizeof(float));
    if (obj == 2) {
      float v = std::min(std::max(base_score, 1.0e-6f), 1.0f - 1.0e-6f);
      base_score = std::log(v / (1 - v));
    }
  }
  if (obj == 1) require(base_score >= 0 && base_score <= 1, "base_score must be in [0,1] for logistic loss.");
  initialized = true;
}

void Learner::upload_model() {
  if (uploaded_trees_ == trees.size() && model_version_ == trees.size()) return;
  std::vector<MgbTreeNode> nodes;
  std::vector<uint32_t> offsets;
  for (auto const& t : trees) {
    offsets.push_back((uint32_t)nodes.size());
    nodes.insert(nodes.end(), t.nodes.begin(), t.nodes.end());
  }
  if (nodes.empty()) nodes.resize(1);
  if (offsets.empty()) offsets.resize(1);
  d_model_nodes_.upload(nodes.data(), nodes.size() * sizeof(MgbTreeNode));
  d_model_offsets_.upload(offsets.data(), offsets.size() * sizeof(uint32_t));
  uploaded_trees_ = trees.size();
  model_version_ = trees.size();
}

// Adds trees [offsets, offsets + count) of the uploaded model to margin.
void Learner::predict_into(DMatrix& data, const uint32_t* offsets, uint32_t count, float* margin) {
  data.upload();
  if (data.sparse)
    kcheck(mgb_predict_csr(data.d_indptr.as<uint64_t>(), data.d_indices.as<uint32_t>(), data.d_values.as<float>(),
                           data.rows, d_model_nodes_.as<MgbTreeNode>(), offsets, count, margin),
           "prediction");
  else
    kcheck(mgb_predict(data.d_data.as<float>(), data.rows, data.cols, d_model_nodes_.as<MgbTreeNode>(), offsets,
                       count, margin),
           "prediction");
}

DeviceBuffer* Learner::margin_cache(DMatrix& data) {
  if (cache_id_ == data.id && cache_trees_ == boosted_rounds() && d_margin_.get()) return &d_margin_;
  drain();  // the margin is rebuilt from every tree
  data.upload();
  d_margin_.ensure((size_t)data.rows * sizeof(float));
  if (!data.base_margin.empty()) {
    require(data.base_margin.size() == data.rows, "base_margin must have one value per row.");
    d_margin_.upload(data.base_margin.data(), data.rows * sizeof(float));
  } else {
    kcheck(mgb_fill_f32(d_margin_.as<float>(), data.rows, base_margin_value()), "margin fill");
  }
  if (!trees.empty()) {
    upload_model();
    predict_into(data, d_model_offsets_.as<uint32_t>(), (uint32_t)trees.size(), d_margin_.as<float>());
  }
  cache_id_ = data.id;
  cache_trees_ = trees.size();
  return &d_margin_;
}

int Learner::bin_layout() const {
  const std::string v = param("hip_bin_layout", "auto");
  if (v == "auto") return 0;
  if (v == "row") return 1;
  if (v == "group") return 2;
  throw Error("hip_bin_layout must be auto, row or group, got '" + v + "'.");
}

void Learner::configure_rng() {
  const std::string seed = param("seed", "0");
  if (seed != rng_seed_) {
    size_t read = 0;
    long long value = 0;
    try {
      value = std::stoll(seed, &read);
    } catch (...) {
      read = 0;
    }
    require(read == seed.size(), "Invalid random seed.");
    rng_.seed(static_cast<std::mt19937::result_type>(value));
    rng_seed_ = seed;
  }
}

void Learner::sample_rows(DMatrix& data, MgbGradParams& gp) {
  configure_rng();
  // src/learner.cpp:668: reseed with the number of rounds already boosted,
  // counting the rounds still queued on the device.
  if (integer("seed_per_iteration", 0))
    rng_.seed(static_cast<std::mt19937::result_type>((uint32_t)std::stoll(param("seed", "0")) * 127u +
                                                     (uint32_t)boosted_rounds()));
  const double subsample = number("subsample", 1);
  const auto budget = static_cast<uint64_t>(static_cast<float>(data.rows) * subsample);
  gp.subsample = 1.0f;
  gp.sample_seed = 0;
  if (budget < data.rows) {
    gp.sample_seed = static_cast<uint32_t>(rng_());
    gp.subsample = static_cast<float>(subsample);
  }
}

// Uniform integer in [0, range), range <= 2^32, the way libstdc++'s
// std::uniform_int_distribution draws it from a 32-bit engine (GCC 11 and
// later): Lemire's multiply-shift, "Fast Random Integer Generation in an
// Interval" (ACM TOMACS 29(1), 2019): the high half of engine() * range,
// redrawn while the low half falls below 2^32 mod range.
static uint32_t libstdcxx_uniform(std::mt19937& engine, uint64_t range) {
  const uint32_t r32 = (uint32_t)range;
  uint64_t product = (uint64_t)(uint32_t)engine() * r32;
  uint32_t low = (uint32_t)product;
  if (low < r32) {
    const uint32_t threshold = (uint32_t)(0u - r32) % r32;
    while (low < threshold) {
      product = (uint64_t)(uint32_t)engine() * r32;
      low = (uint32_t)product;
    }
  }
  return (uint32_t)(product >> 32);
}

// std::shuffle as x86-64 Linux builds compile it (libstdc++): position i
// (from 1 upwards) swaps with a uniform position in [0, i].  While
// n^2 < 2^32 the draws come in pairs: for an even n position 1 first takes
// one draw over {0, 1}; then positions i, i + 1 take one draw x over
// [0, (i + 1)(i + 2)) and swap with x / (i + 2) and x % (i + 2).  Larger n
// take one draw per position.
static void shuffle_libstdcxx(std::vector<uint32_t>& v, std::mt19937& engine) {
  const uint64_t n = v.size();
  if (n < 2) return;
  if (0xffffffffull / n >= n) {
    uint64_t i = 1;
    if (n % 2 == 0) {
      std::swap(v[1], v[libstdcxx_uniform(engine, 2)]);
      i = 2;
    }
    for (; i < n; i += 2) {
      const uint64_t b0 = i + 1, b1 = i + 2;
      const uint32_t x = libstdcxx_uniform(engine, b0 * b1);
      std::swap(v[i], v[x / b1]);
      std::swap(v[i + 1], v[x % b1]);
    }
    return;
  }
  for (uint64_t i = 1; i < n; ++i) std::swap(v[i], v[libstdcxx_uniform(engine, i + 1)]);
}

// std::shuffle as the reference's macOS builds compile it (libc++):
// Fisher-Yates from the front, position pos swapping with pos + u, u uniform
// in [0, n - pos) drawn by masking one engine output to the bit width of
// n - pos - 1 and rejecting values >= n - pos.
static void shuffle_libcxx(std::vector<uint32_t>& v, std::mt19937& engine) {
  const size_t n = v.size();
  for (size_t pos = 0; pos + 1 < n; ++pos) {
    const uint64_t range = n - pos;
    uint32_t width = 0;
    while (width < 32 && ((range - 1) >> width)) ++width;
    const uint32_t mask = width >= 32 ? 0xffffffffu : (1u << width) - 1u;
    uint32_t u;
    do u = static_cast<uint32_t>(engine()) & mask; while (u >= range);
    std::swap(v[pos], v[pos + u]);
  }
}

void std_shuffle(std::vector<uint32_t>& order, std::mt19937& engine, ShuffleModel model) {
  if (model == ShuffleModel::libcxx) shuffle_libcxx(order, engine);
  else shuffle_libstdcxx(order, engine);
}

void set_error(std::string message);  // the library's last-error slot (runtime.hip)

// The first inconsistency of one tree's node records as the device emitted
// them, or "" (checked before the tree is published, as the reference checks
// its emitted table against the host replay: src/learner.cpp:36-61,
// src/tree.cpp:1663-1717).  Split nodes take their children in node-id
// order: the k-th split node (by id) has children 2k + 1 and 2k + 2.
static std::string tree_violation(const MgbTreeNode* nodes, uint32_t count, uint32_t status, uint32_t max_nodes,
                                  uint32_t cols) {
  if (status) {
    static const char* const names[] = {"a node id outside the node table", "node or frontier capacity exceeded",
                                        "task lists exceed the workspace", "a child holds more rows than its parent"};
    std::string what;
    for (uint32_t b = 0; b < 4; ++b)
      if (status & (1u << b)) what += (what.empty() ? "" : ", ") + std::string(names[b]);
    if (status >> 4) what += (what.empty() ? "" : ", ") + std::string("unknown bits");
    std::ostringstream hex;
    hex << std::hex << status;
    return "the device reported tree status 0x" + hex.str() + " (" + what + ")";
  }
  if (count < 1 || count > max_nodes)
    return "node count " + std::to_string(count) + " is outside [1, " + std::to_string(max_nodes) + "]";
  if (nodes[0].parent != -1) return "node 0 is not a root (parent " + std::to_string(nodes[0].parent) + ")";
  uint32_t next = 1;  // the next unused node id
  for (uint32_t i = 0; i < count; ++i) {
    const MgbTreeNode& x = nodes[i];
    // The message is built only for a node that fails (every round's trees
    // pass through here when the model is read).
    auto node = [i] { return "node " + std::to_string(i); };
    if (x.default_left > 1) return node() + " has default_left " + std::to_string(x.default_left);
    if (x.left == -1 && x.right == -1) {
      if (x.feature != -1) return node() + " is a leaf with split feature " + std::to_string(x.feature);
      continue;
    }
    if (x.left < 0 || x.right < 0) return node() + " has one child";
    if ((uint32_t)x.left != next || x.right != x.left + 1)
      return node() + " has children (" + std::to_string(x.left) + ", " + std::to_string(x.right) +
             "), not the next unused ids (" + std::to_string(next) + ", " + std::to_string(next + 1) + ")";
    if ((uint32_t)x.right >= count)
      return node() + "'s children lie beyond the node count " + std::to_string(count);
    if (x.feature < 0 || (uint32_t)x.feature >= cols)
      return node() + " splits on feature " + std::to_string(x.feature) + " of " + std::to_string(cols);
    if (nodes[x.left].parent != (int32_t)i || nodes[x.right].parent != (int32_t)i)
      return node() + "'s children do not name it as their parent";
    next += 2;
  }
  if (next != count)
    return "the split nodes' children end at id " + std::to_string(next) + ", not at the node count " +
           std::to_string(count);
  return "";
}

extern "C" int mgb_validate_tree(const MgbTreeNode* nodes, uint32_t count, uint32_t status, uint32_t max_nodes,
                                 uint32_t cols) {
  if (!nodes && count) {
    set_error("mgb_validate_tree: null node records");
    return -1;
  }
  const std::string why = tree_violation(nodes, count, status, max_nodes, cols);
  if (why.empty()) return 0;
  set_error(why);
  return -1;
}

extern "C" int mgb_std_shuffle(uint32_t seed, uint32_t n, uint32_t model, uint32_t* order, uint32_t* next_draw) {
  if (model > 1 || (n && !order)) return -1;
  std::vector<uint32_t> v(n);
  for (uint32_t i = 0; i < n; ++i) v[i] = i;
  std::mt19937 engine(seed);
  std_shuffle(v, engine, model == 1 ? ShuffleModel::libcxx : ShuffleModel::libstdcxx);
  for (uint32_t i = 0; i < n; ++i) order[i] = v[i];
  if (next_draw) *next_draw = (uint32_t)engine();
  return 0;
}

ShuffleModel shuffle_model(const std::string& name) {
  if (name == "libstdc++") return ShuffleModel::libstdcxx;
  if (name == "libc++") return ShuffleModel::libcxx;
  throw std::runtime_error("std_shuffle must be \"libstdc++\" or \"libc++\", got \"" + name + "\"");
}

// src/tree.cpp:15-26: "(1,0,-1)" or "[1,0,-1]", one entry per leading
// feature (the rest unconstrained), each -1, 0 or 1.
const int32_t* Learner::monotone_constraints(uint32_t cols) {
  const std::string text = param("monotone_constraints", "()");
  if (text != monotone_text_ || monotone_.size() != cols) {
    std::vector<int32_t> values(cols, 0);
    std::string json = text;
    std::replace(json.begin(), json.end(), '(', '[');
    std::replace(json.begin(), json.end(), ')', ']');
    if (!json.empty() && json != "[]") {
      Json list;
      try {
        list = Json::parse(json);
      } catch (const std::exception&) {
        throw std::runtime_error("monotone_constraints must be a list of -1, 0 or 1: " + text);
      }
      require(list.is_array(), "monotone_constraints must be a list of -1, 0 or 1.");
      require(list.size() <= cols, "monotone_constraints has more entries than features.");
      for (size_t i = 0; i < list.size(); ++i) {
        require(list[i].is_number() && list[i].number() == (double)list[i].integer(),
                "monotone_constraints must be a list of -1, 0 or 1.");
        const int64_t v = list[i].integer();
        require(v >= -1 && v <= 1, "Monotone constraints must be -1, 0 or 1.");
        values[i] = (int32_t)v;
      }
    }
    monotone_ = std::move(values);
    monotone_text_ = text;
    monotone_active_ = std::any_of(monotone_.begin(), monotone_.end(), [](int32_t v) { return v != 0; });
    if (monotone_active_) {
      d_monotone_.ensure((size_t)cols * sizeof(int32_t));
      kcheck(mgb_memcpy_h2d(d_monotone_.get(), monotone_.data(), (size_t)cols * sizeof(int32_t)),
             "monotone constraints upload");
    }
  }
  return monotone_active_ ? d_monotone_.as<int32_t>() : nullptr;
}

// src/tree.cpp:28-45 (kernels/tree_sample_columns.metal.h): a fresh engine
// seeded by one draw shuffles the features; the first
// max(1, floor(n * fraction)) of them are kept.  The shuffle follows the
// standard library named by `std_shuffle` (default libstdc++, as stock
// XGBoost's x86-64 build; "libc++" gives the reference's macOS draws).
const uint32_t* Learner::sample_columns(uint32_t cols) {
  const float fraction = fnumber("colsample_bytree", 1.0f);
  if (!(fraction < 1.0f) || cols == 0) return nullptr;
  std::mt19937 engine(rng_());
  std::vector<uint32_t> order(cols);
  for (uint32_t i = 0; i < cols; ++i) order[i] = i;
  const float scaled = std::floor(static_cast<float>(cols) * fraction);
  const uint32_t keep = std::min<uint32_t>(cols, scaled < 1.0f ? 1u : static_cast<uint32_t>(scaled));
  std_shuffle(order, engine, shuffle_model(param("std_shuffle", "libstdc++")));
  feature_flags_.assign(cols, 0u);
  for (uint32_t i = 0; i < keep; ++i) feature_flags_[order[i]] = 1u;
  d_features_.ensure((size_t)cols * sizeof(uint32_t));
  kcheck(mgb_memcpy_h2d_async(d_features_.get(), feature_flags_.data(), (size_t)cols * sizeof(uint32_t)),
         "feature sample upload");
  return d_features_.as<uint32_t>();
}

void Learner::grow(DMatrix& data, bool unit_hessian, bool sampled) {
  const uint32_t depth = (uint32_t)integer("max_depth", 6);
  MgbTreeShape shape{};
  shape.rows = data.rows;
  shape.cols = data.cols;
  shape.max_bin = data.hist_bins;
  shape.max_depth = depth;
  // Rows per histogram tile: small enough for a few hundred workgroups at the
  // root, large enough that the per-tile partial histograms (F x (bins+1) x
  // 16 bytes each) stay well below the bin matrix they summarise.
  uint32_t tile = data.rows >= 262144 ? 4096 : 2048;
  while (tile < 65536 && (uint64_t)tile * 160 < data.rows) tile *= 2;
  shape.rows_per_tile = (uint32_t)integer("hip_histogram_rows", tile);
  shape.features_per_group = data.features_per_group;
  shape.unit_hessian = unit_hessian ? 1 : 0;
  // A subsample's dropped rows (zero gradients) leave the row list before the
  // root; a walk of the finished tree adds their leaves to the margin.
  shape.compact_sampled = sampled && integer("hip_compact_sampled", 1) != 0 ? 1 : 0;
  // 1: children keep their parent's row order (one counting pass more per
  // level); 0: tiles claim their ranges by atomics in arrival order.  The
  // trees are the same either way.  Default: stable from 2^19 rows.  Measured
  // per round: 10M x 128 partition 1.65 ms stable against 2.11 ms by claims
  // (the claims serialize on a large node's two cursors), 1M x 2000 CSR
  // 0.36 against 0.45 ms; 262,144 x 64: 39.1 against 35.2 ms per 100 rounds
  // (the counting pass's extra launch per level costs more than the few
  // claims there).
  const int64_t stable = integer("hip_stable_partition", -1);
  shape.stable_partition = (stable < 0 ? data.rows >= (1u << 19) : stable != 0) ? 1 : 0;
  {
    // Root tiles: the root streams every row in order, so a workgroup can take
    // a long tile (its batches software-pipelined) at no cost in locality.
    // Size them so the root's (tile, feature group) workgroups give each of
    // the 256 CUs one; each leaves one partial histogram for the split kernel
    // to sum, so fewer tiles also mean fewer partials.  Measured: 262,144 x 64
    // 3.4% faster per round with 32 tiles of 8192 rows than 64 of 4096 (two
    // workgroups per CU) or 16 of 16384; 10M x 128 1.7% faster with 16 tiles
    // than with 153 of 65536 rows.
    const uint64_t G = data.features_per_group, groups = (data.cols + G - 1) / G;
    const uint64_t root_tiles = std::max<uint64_t>(1, 256 / std::max<uint64_t>(groups, 1));
    uint64_t root = (data.rows + root_tiles - 1) / root_tiles;
    root = std::max<uint64_t>((root + 1023) / 1024 * 1024, shape.rows_per_tile);
    shape.root_rows_per_tile = (uint32_t)integer("hip_histogram_root_rows", (int64_t)std::min<uint64_t>(root, UINT32_MAX));
    require(shape.root_rows_per_tile >= shape.rows_per_tile, "hip_histogram_root_rows must be >= hip_histogram_rows.");
  }
  shape.dense = data.has_missing ? 0 : 1;
  // The root's histogram reads every row: it takes the column-major codes
  // (whole cache lines of one feature) rather than a few bytes of each
  // row-major row.  Deeper levels gather rows, where a row-major row's lines
  // serve every feature group from L2 (10M x 128, 1024 bins: the root level
  // 20% faster, deeper levels slower from columns).
  const bool columns_on = integer("hip_partition_columns", 1) != 0;
  shape.column_levels = columns_on ? (uint32_t)integer("hip_histogram_column_levels", 1) : 0;
  if (data.sparse) {
    // CSR: row tiles are only work units (every tile adds into the node's
    // histogram), so small tiles spread a level over many workgroups.
    shape.sparse = 1;
    shape.compact_sampled = 0;
    shape.column_levels = 0;
    shape.rows_per_tile = (uint32_t)integer("hip_histogram_rows", 512);
    shape.root_rows_per_tile = 0;
  }
  size_t ws = mgb_tree_workspace_bytes(&shape);
  d_tree_ws_.ensure(ws);
  const uint32_t max_nodes = (2u << depth) - 1u;
  const size_t node_bytes = (size_t)max_nodes * sizeof(MgbTreeNode);
  // This round's slot in the queue of rounds not yet copied to the host
  // (up to 1,024 rounds or 64 MB; a full queue is drained first).  A drain
  // waits for every queued round and the device then idles until the host
  // launches again, so the queue holds a whole fit of the usual round counts
  // (depth 8: 1,024 rounds in 20 MB; depth 10: 819 rounds).
  const size_t slot_bytes = (node_bytes + 16 + 255) / 256 * 256;
  if (pending_bytes_ + slot_bytes > d_pending_.bytes()) {
    drain();
    const size_t rounds = std::max<size_t>(1, std::min<size_t>(1024, (64u << 20) / slot_bytes));
    if (d_pending_.bytes() < rounds * slot_bytes) d_pending_.resize(rounds * slot_bytes);
  }
  const size_t slot_offset = pending_bytes_;
  MgbSplitParams sp{};
  sp.reg_lambda = fnumber("reg_lambda", 1.0f);
  sp.reg_alpha = fnumber("reg_alpha", 0.0f);
  sp.min_child_weight = fnumber("min_child_weight", 1.0f);
  sp.max_delta_step = fnumber("max_delta_step", 0.0f);
  sp.min_split_loss = fnumber("min_split_loss", 0.0f);
  sp.eta = fnumber("learning_rate", 0.3f);
  sp.max_depth = depth;
  sp.fma_contract = (uint32_t)integer("fma_contract", 1);
  // Test hook: status bits the device reports for this tree as if it had
  // found them (every kernel still runs normally); drain() then refuses it.
  sp.inject_status = (uint32_t)integer("hip_inject_tree_status", 0);
  DeviceBuffer* margin = margin_cache(data);
  const bool profiling = integer("hip_profile", 0) != 0;
  kcheck(mgb_profile_enable(profiling ? 1 : 0), "profile");
  auto* nodes = reinterpret_cast<MgbTreeNode*>(d_pending_.as<uint8_t>() + slot_offset);
  auto* count = reinterpret_cast<uint32_t*>(d_pending_.as<uint8_t>() + slot_offset + node_bytes);
  const uint32_t* features = sample_columns(data.cols);
  const int32_t* monotone = monotone_constraints(data.cols);
  if (data.sparse) {
    const bool root_columns = integer("hip_csr_root_columns", 1) != 0;
    kcheck(mgb_grow_tree_csr(&shape, &data.csr, data.d_indptr.as<uint64_t>(), data.d_indices.as<uint32_t>(),
                             data.d_codes.get(), root_columns ? data.d_colptr.as<uint64_t>() : nullptr,
                             root_columns ? data.d_csc_rows.as<uint32_t>() : nullptr,
                             root_columns ? data.d_csc_codes.get() : nullptr, data.d_cuts.as<float>(),
                             data.d_counts.as<uint32_t>(),
                             d_grad_.as<float>(), d_scales_.as<float>(), &sp, features, monotone, d_tree_ws_.get(),
                             d_tree_ws_.bytes(), margin->as<float>(), nodes, count),
           "tree growth");
  } else {
    const void* columns = columns_on ? data.d_columns.get() : nullptr;
    kcheck(mgb_grow_tree(&shape, &data.matrix, data.d_bins.get(), columns, data.d_cuts.as<float>(),
                         data.d_counts.as<uint32_t>(), d_grad_.as<float>(), d_scales_.as<float>(), &sp, features,
                         monotone, d_tree_ws_.get(), d_tree_ws_.bytes(), margin->as<float>(), nodes, count),
           "tree growth");
  }
  pending_.push_back(Pending{slot_offset, node_bytes, max_nodes});
  pending_bytes_ += slot_bytes;
  cache_trees_ = boosted_rounds();  // the kernels add the new leaves to the cached margin
  if (profiling) {
    drain();  // profiled rounds stay synchronous: their statistics are read back now
    // Algorithmic histogram bytes per level: rows built x (F codes + 4-byte
    // row id + 8-byte gradient pair) + nodes built x F x (B+1) x 16 bytes.
    kcheck(mgb_profile_collect(), "profile collect");
    uint64_t rows[32] = {0};
    uint32_t built[32] = {0};
    kcheck(mgb_tree_level_stats(&shape, d_tree_ws_.get(), rows, built, 32), "level statistics");
    // CSR rows: their nonzeros (4-byte column + code each) and 8-byte offsets.
    const double row_bytes =
        data.sparse ? (double)data.values.size() / std::max(1u, data.rows) * (4 + data.matrix.bin_bytes) + 8 + 12
                    : (double)data.cols * data.matrix.bin_bytes + 12;
    // Split scan: the root reads its histogram once; below it each sibling
    // pair reads the parent's and the built child's histograms and writes the
    // sibling's (16 bytes per feature and bin each).
    const uint64_t node_hist = (uint64_t)data.cols * (data.hist_bins + 1) * 16;
    // The same with only the tree's column sample (dense matrices): the
    // kernels read, accumulate and write no other feature below the root
    // (the root also builds feature 0 for its totals).
    uint64_t sampled = data.cols;
    if (features && !data.sparse) sampled = std::count(feature_flags_.begin(), feature_flags_.end(), 1u);
    const double row_bytes_s = data.sparse ? row_bytes : (double)sampled * data.matrix.bin_bytes + 12;
    const uint64_t node_hist_s = data.sparse ? node_hist : sampled * (data.hist_bins + 1) * 16;
    level_rows_.assign(rows, rows + std::min<uint32_t>(depth, 32));
    level_nodes_.assign(built, built + std::min<uint32_t>(depth, 32));
    for (uint32_t d = 0; d < depth && d < 32; ++d) {
      hist_bytes_ += (uint64_t)(rows[d] * row_bytes) + (uint64_t)built[d] * node_hist;
      hist_bytes_sampled_ += (uint64_t)(rows[d] * row_bytes_s) + (uint64_t)built[d] * node_hist_s;
      hist_rows_ += rows[d];
      split_bytes_ += (d == 0 ? 1u : 3u) * (uint64_t)built[d] * node_hist;
      split_bytes_sampled_ += (d == 0 ? 1u : 3u) * (uint64_t)built[d] * node_hist_s;
    }
    // Partition (select and apply, and the stable partition's counting pass):
    // a row of a splitting node reads its id, its gradient pair and the split
    // feature's code and writes its id and pair into its child's segment
    // (4 + 8 + s + 4 + 8 bytes); at the last level it reads its id and code
    // and updates its margin (4 + s + 8); a row of a stopping node reads its
    // id and updates its margin (4 + 8).  The code s is one bin code of a
    // dense matrix; a CSR row's lookup reads its offsets, one column index and
    // the code (8 + 4 + s).  A subsample's dropped rows (their walk of the
    // finished tree) are not counted.
    uint32_t moved[32] = {0}, stopped[32] = {0};
    kcheck(mgb_tree_partition_stats(&shape, d_tree_ws_.get(), moved, stopped, 32), "partition statistics");
    const uint64_t code = data.sparse ? 8 + 4 + data.csr.bin_bytes : data.matrix.bin_bytes;
    for (uint32_t d = 0; d < depth && d < 32; ++d) {
      const uint64_t split_row = d + 1 == depth ? 4 + code + 8 : 4 + 8 + code + 4 + 8;
      partition_bytes_ += (uint64_t)moved[d] * split_row + (uint64_t)stopped[d] * (4 + 8);
    }
  }
}

// A round without rows: no gradient and no Hessian, so the root's weight is 0
// and it cannot split (its Hessian sum is below any min_child_weight); the
// tree is that single leaf.  Queued rounds are published first, so the trees
// stay in round order.
void Learner::empty_round() {
  drain();
  MgbTreeNode leaf{};
  leaf.left = leaf.right = leaf.parent = leaf.feature = -1;
  Tree tree;
  tree.nodes.push_back(leaf);
  trees.push_back(std::move(tree));
}

void Learner::drain() {
  if (pending_.empty()) return;
  // One device-to-host copy (it waits for the queued rounds) of every
  // pending slot: node records followed by the node count.  The queue is
  // taken over only once the copy has succeeded.
  kcheck(download_pinned(d_pending_.get(), pending_bytes_, [&](const uint8_t* host) {
    std::vector<Pending> rounds;
    rounds.swap(pending_);
    pending_bytes_ = 0;
    for (const Pending& p : rounds) {
      uint32_t word[2] = {0, 0};  // node count, tree status
      std::memcpy(word, host + p.offset + p.node_bytes, sizeof(word));
      const uint32_t n = std::min(word[0], p.max_nodes);
      const auto* records = reinterpret_cast<const MgbTreeNode*>(host + p.offset);
      const std::string why = tree_violation(records, word[0], word[1], p.max_nodes, num_feature);
      if (!why.empty()) {
        // Every later round took its gradients from this round's margins:
        // drop them with it, and rebuild the training margins from the trees
        // kept (src/learner.cpp:36-61 retire_round).
        const size_t round = trees.size();
        cache_id_ = 0;
        cache_trees_ = 0;
        throw Error("round " + std::to_string(round) + ": the device tree is invalid: " + why +
                    "; this and the " + std::to_string(rounds.size() - 1 - (&p - rounds.data())) +
                    " later queued rounds are dropped");
      }
      Tree tree;
      tree.nodes.assign(records, records + n);
      trees.push_back(std::move(tree));
    }
  }), "device-to-host copy of the queued rounds");
}

void Learner::update(DMatrix& data, int /*iteration*/) {
  configure_check();
  require(data.labels.size() == data.rows, "Labels must be provided for training (one per row).");
  require(data.weights.empty() || data.weights.size() == data.rows, "Number of weights must equal the number of rows.");
  int obj = objective();
  if (obj == 1 || obj == 2) {
    if (data.labels_in_unit < 0) {
      // Checked once per label assignment, not every round.
      data.labels_in_unit = 1;
      for (float y : data.labels)
        if (!(y >= 0 && y <= 1)) { data.labels_in_unit = 0; break; }
    }
    require(data.labels_in_unit == 1, "label must be in [0,1] for logistic loss.");
  }
  data.quantize((uint32_t)integer("max_bin", 256), bin_layout(), (uint32_t)integer("hip_histogram_features", 0));
  auto t0 = std::chrono::steady_clock::now();
  initialize(data, false);
  if (data.rows == 0) return empty_round();
  DeviceBuffer* margin = margin_cache(data);
  d_grad_.ensure((size_t)data.rows * 2 * sizeof(float));
  if (!d_mass_.get()) {
    d_mass_.ensure(MGB_MASS_WORDS * sizeof(uint64_t));
    kcheck(mgb_memset(d_mass_.get(), 0, MGB_MASS_WORDS * sizeof(uint64_t)), "memset");
  }
  d_scales_.ensure(2 * sizeof(float));
  MgbGradParams gp{};
  gp.rows = data.rows;
  gp.objective = (uint32_t)obj;
  gp.has_weight = data.weights.empty() ? 0 : 1;
  gp.scale_pos_weight = fnumber("scale_pos_weight", 1.0f);
  sample_rows(data, gp);
  kcheck(mgb_gradients(&gp, margin->as<float>(), data.d_labels.as<float>(),
                       gp.has_weight ? data.d_weights.as<float>() : nullptr, d_grad_.as<float>(),
                       d_mass_.as<uint64_t>(), d_scales_.as<float>()),
         "gradients");
  // Unit Hessians (every h = 1, so a row count stands in for the Hessian
  // sum) hold for unweighted squared error unless sampling zeroed some rows.
  grow(data, obj == 0 && data.weights.empty() && gp.subsample >= 1.0f, gp.subsample < 1.0f);
  seconds_["train_rounds"] += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  seconds_["quantiles"] = data.sketch_seconds;
  seconds_["bin_matrix"] = data.quantize_seconds;
  ++rounds_timed_;
}

void Learner::boost(DMatrix& data, const float* grad, const float* hess, size_t count) {
  configure_check();
  require(count == data.rows, "Gradient and Hessian must have one entry per row.");
  data.quantize((uint32_t)integer("max_bin", 256), bin_layout(), (uint32_t)integer("hip_histogram_features", 0));
  initialize(data, true);
  if (data.rows == 0) return empty_round();
  std::vector<float> gh(2 * count);
  for (size_t i = 0; i < count; ++i) { gh[2 * i] = grad[i]; gh[2 * i + 1] = hess[i]; }
  d_grad_.upload(gh.data(), gh.size() * sizeof(float));
  if (!d_mass_.get()) {
    d_mass_.ensure(MGB_MASS_WORDS * sizeof(uint64_t));
    kcheck(mgb_memset(d_mass_.get(), 0, MGB_MASS_WORDS * sizeof(uint64_t)), "memset");
  }
  d_scales_.ensure(2 * sizeof(float));
  MgbGradParams gp{};
  gp.rows = data.rows;
  sample_rows(data, gp);
  kcheck(mgb_gradient_mass(&gp, d_grad_.as<float>(), d_mass_.as<uint64_t>(), d_scales_.as<float>()),
         "gradient mass");
  grow(data, false, gp.subsample < 1.0f);
}

const float* Learner::predict_device(DMatrix& data, bool output_margin, uint32_t begin, uint32_t end,
                                    DeviceBuffer& scratch) {
  drain();
  scratch.ensure((size_t)std::max<uint32_t>(data.rows, 1) * sizeof(float));
  float* d_out = scratch.as<float>();
  if (!initialized) {
    // An untrained model predicts its base score.
    kcheck(mgb_fill_f32(d_out, data.rows, output_margin ? base_margin_value() : base_score), "fill");
    return d_out;
  }
  require(data.cols == num_feature, "Feature shape mismatch: expected " + std::to_string(num_feature) + ", got " +
                                        std::to_string(data.cols));
  if (end == 0 || end > trees.size()) end = (uint32_t)trees.size();
  require(begin <= end, "Invalid iteration range.");
  if (begin == 0 && end == trees.size() && data.base_margin.empty() && cache_id_ == data.id &&
      cache_trees_ == trees.size()) {
    if (output_margin || objective() != 1) return d_margin_.as<float>();
    kcheck(mgb_memcpy_d2d(d_out, d_margin_.get(), data.rows * sizeof(float)), "copy");
  } else {
    data.upload();
    if (!data.base_margin.empty()) {
      require(data.base_margin.size() == data.rows, "base_margin must have one value per row.");
      scratch.upload(data.base_margin.data(), data.rows * sizeof(float));
    } else {
      kcheck(mgb_fill_f32(d_out, data.rows, base_margin_value()), "margin fill");
    }
    if (end > begin) {
      upload_model();
      predict_into(data, d_model_offsets_.as<uint32_t>() + begin, end - begin, d_out);
    }
  }
  if (!output_margin) kcheck(mgb_transform(d_out, data.rows, (uint32_t)objective()), "transform");
  return d_out;
}

namespace {

// Cover-weighted mean leaf value of every node of a tree, children before
// parents (a node's children have larger ids), and the tree's depth.
uint32_t node_means(const std::vector<MgbTreeNode>& t, float* means) {
  std::vector<uint32_t> depth(t.size(), 0);
  uint32_t deepest = 0;
  for (size_t i = 0; i < t.size(); ++i) {
    if (t[i].left >= 0) {
      require((size_t)t[i].left > i && (size_t)t[i].right > i && (size_t)t[i].left < t.size() &&
                  (size_t)t[i].right < t.size(),
              "Tree nodes must list children after their parent.");
      depth[t[i].left] = depth[t[i].right] = depth[i] + 1;
      deepest = std::max(deepest, depth[i] + 1);
    }
  }
  for (size_t k = t.size(); k-- > 0;) {
    const MgbTreeNode& n = t[k];
    means[k] = n.left < 0 ? n.leaf
                          : (means[n.left] * t[n.left].cover + means[n.right] * t[n.right].cover) / n.cover;
  }
  return deepest;
}

}  // namespace

std::vector<float> Learner::predict_explain(DMatrix& data, int type, uint32_t end) {
  drain();
  require(type >= 2 && type <= 6, "Prediction type must be 2 to 6 here.");
  const bool interactions = type == 4 || type == 5;
  if (end == 0 || end > trees.size()) end = (uint32_t)trees.size();
  if (initialized)
    require(data.cols == num_feature, "Feature shape mismatch: expected " + std::to_string(num_feature) + ", got " +
                                          std::to_string(data.cols));
  const uint64_t columns = (uint64_t)data.cols + 1;
  const uint64_t width = type == 6 ? end : (interactions ? columns * columns : columns);
  std::vector<float> out((size_t)data.rows * width, 0.0f);
  if (!data.rows) return out;
  if (type == 6 && end == 0) return out;
  data.upload();
  upload_model();
  DeviceBuffer d_out;
  d_out.ensure(out.size() * sizeof(float));
  const uint64_t* indptr = data.sparse ? data.d_indptr.as<uint64_t>() : nullptr;
  const uint32_t* indices = data.sparse ? data.d_indices.as<uint32_t>() : nullptr;
  const float* X = data.sparse ? data.d_values.as<float>() : data.d_data.as<float>();
  if (type == 6) {
    kcheck(mgb_predict_leaf(X, indptr, indices, data.rows, data.cols, d_model_nodes_.as<MgbTreeNode>(),
                            d_model_offsets_.as<uint32_t>(), end, d_out.as<float>()),
           "leaf prediction");
  } else {
    std::vector<float> means;
    uint32_t deepest = 0;
    for (uint32_t t = 0; t < end; ++t) {
      const size_t at = means.size();
      means.resize(at + trees[t].nodes.size());
      deepest = std::max(deepest, node_means(trees[t].nodes, means.data() + at));
    }
    if (means.empty()) means.resize(1);
    d_model_means_.upload(means.data(), means.size() * sizeof(float));
    DeviceBuffer d_base;
    if (!data.base_margin.empty()) {
      require(data.base_margin.size() == data.rows, "base_margin must have one value per row.");
      d_base.upload(data.base_margin.data(), data.rows * sizeof(float));
    }
    kcheck(mgb_predict_contribs(X, indptr, indices, data.rows, data.cols, d_model_nodes_.as<MgbTreeNode>(),
                                d_model_means_.as<float>(), d_model_offsets_.as<uint32_t>(), end, deepest,
                                type == 3 || type == 5 ? 1u : 0u, interactions ? 1u : 0u,
                                d_base.get() ? d_base.as<float>() : nullptr,
                                base_margin_value(), d_out.as<float>()),
           "contribution prediction");
  }
  kcheck(mgb_memcpy_d2h(out.data(), d_out.get(), out.size() * sizeof(float)), "device-to-host copy");
  return out;
}

std::vector<float> Learner::predict(DMatrix& data, bool output_margin, uint32_t begin, uint32_t end) {
  std::vector<float> out(data.rows);
  if (!data.rows) return out;
  DeviceBuffer scratch;
  const float* d_out = predict_device(data, output_margin, begin, end, scratch);
  kcheck(mgb_memcpy_d2h(out.data(), d_out, out.size() * sizeof(float)), "device-to-host copy");
  return out;
}

// Default metric of the objective (src/learner.cpp:1012-1023).
std::string Learner::default_metric() const {
  const int obj = objective();
  return (obj == 1 && objective_name() != "reg:logistic") || obj == 2 ? "logloss" : "rmse";
}

double Learner::metric(DMatrix& d, const float* pred, const std::string& name) {
  static const std::map<std::string, uint32_t> kinds{
      {"rmse", MGB_METRIC_RMSE}, {"mae", MGB_METRIC_MAE}, {"rmsle", MGB_METRIC_RMSLE},
      {"logloss", MGB_METRIC_LOGLOSS}, {"error", MGB_METRIC_ERROR}, {"mape", MGB_METRIC_MAPE},
      {"mphe", MGB_METRIC_MPHE}, {"poisson-nloglik", MGB_METRIC_POISSON},
      {"gamma-deviance", MGB_METRIC_GAMMA_DEVIANCE}, {"tweedie-nloglik", MGB_METRIC_TWEEDIE},
      {"gamma-nloglik", MGB_METRIC_GAMMA_NLOGLIK}, {"auc", 13}, {"aucpr", 14}};
  const size_t sep = name.find('@');
  const std::string base = name.substr(0, sep);
  auto it = kinds.find(base);
  require(base != "merror" && base != "mlogloss", "Multiclass metrics need a multiclass objective: " + name);
  require(it != kinds.end(), "Metric has not been implemented yet: " + name);
  require(d.weights.empty() || d.weights.size() == d.rows, "Evaluation weights must have one entry per row.");
  d.upload_info();
  const float* w = d.weights.empty() ? nullptr : d.d_weights.as<float>();
  d_metric_ws_.ensure(std::max<size_t>(mgb_metric_workspace_bytes(d.rows), 256));
  if (it->second >= 13) {
    for (float y : d.labels) require(y >= 0 && y <= 1, "AUC labels must be in [0,1].");
    if (!d.rows) return std::numeric_limits<double>::quiet_NaN();
    double out[3];
    kcheck(mgb_metric_auc(pred, d.d_labels.as<float>(), w, d.rows, it->second == 14, out, d_metric_ws_.get(),
                          d_metric_ws_.bytes()),
           "auc");
    if (!(out[1] > 0 && out[2] > 0)) return std::numeric_limits<double>::quiet_NaN();
    return it->second == 13 ? out[0] / (out[1] * out[2]) : out[0];
  }
  float parameter = 0;
  if (base == "error") parameter = sep == std::string::npos ? 0.5f : std::stof(name.substr(sep + 1));
  if (base == "mphe") parameter = (float)number("huber_slope", 1);
  if (base == "tweedie-nloglik") {
    require(sep != std::string::npos, "tweedie-nloglik requires a variance power after @.");
    parameter = std::stof(name.substr(sep + 1));
    require(parameter >= 1 && parameter < 2, "Tweedie variance power must be in [1, 2).");
  }
  float out[2];
  kcheck(mgb_metric_sum(pred, d.d_labels.as<float>(), w, d.rows, it->second, parameter, out, d_metric_ws_.get(),
                        d_metric_ws_.bytes()),
         "metric");
  const double mean = out[1] > 0 ? (double)out[0] / (double)out[1] : std::numeric_limits<double>::quiet_NaN();
  return base == "rmse" || base == "rmsle" ? std::sqrt(mean) : mean;
}

std::string Learner::evaluate(int iteration, const std::vector<DMatrix*>& data, const std::vector<std::string>& names) {
  require(initialized, "Model is not yet initialized (not fitted).");
  if (metrics.empty() && integer("disable_default_eval_metric", 0) == 0) metrics.push_back(default_metric());
  std::ostringstream os;
  os << '[' << iteration << ']' << std::setprecision(10);
  for (size_t k = 0; k < data.size(); ++k) {
    DMatrix& d = *data[k];
    const float* pred = predict_device(d, false, 0, 0, d_eval_pred_);
    for (auto const& name : metrics) {
      require(d.labels.size() == d.rows, "Evaluation data requires labels.");
      os << '\t' << names[k] << '-' << name << ':' << metric(d, pred, name);
    }
  }
  return os.str();
}

// ---------------------------------------------------------------------------
// Model (src/model.cpp:28-74: XGBoost JSON schema, version [3, 5, 0])
// ---------------------------------------------------------------------------
Json Learner::model() const {
  Json trees_json = Json::array(), tree_info = Json::array(), indptr = Json::array();
  for (size_t t = 0; t < trees.size(); ++t) {
    const auto& tree = trees[t];
    Json v = Json::object();
    v["id"] = Json((int64_t)t);
    Json tp = Json::object();
    tp["num_deleted"] = "0";
    tp["num_feature"] = std::to_string(num_feature);
    tp["num_nodes"] = std::to_string(tree.nodes.size());
    tp["size_leaf_vector"] = "1";
    v["tree_param"] = tp;
    Json bw = Json::array(), cats = Json::array(), dl = Json::array(), lc = Json::array(), rc = Json::array(),
         loss = Json::array(), parents = Json::array(), cond = Json::array(), idx = Json::array(),
         stype = Json::array(), hess = Json::array();
    for (const auto& n : tree.nodes) {
      bw.push_back(Json(n.base_weight));
      dl.push_back(Json((int64_t)n.default_left));
      lc.push_back(Json((int64_t)n.left));
      rc.push_back(Json((int64_t)n.right));
      loss.push_back(Json(n.gain));
      parents.push_back(Json((int64_t)(n.parent < 0 ? 2147483647 : n.parent)));
      cond.push_back(Json(n.left < 0 ? n.leaf : n.threshold));
      idx.push_back(Json((int64_t)(n.feature < 0 ? 0 : n.feature)));
      stype.push_back(Json((int64_t)0));
      hess.push_back(Json(n.cover));
    }
    v["base_weights"] = bw;
    v["categories"] = Json::array();
    v["categories_nodes"] = Json::array();
    v["categories_segments"] = Json::array();
    v["categories_sizes"] = Json::array();
    v["default_left"] = dl;
    v["left_children"] = lc;
    v["loss_changes"] = loss;
    v["parents"] = parents;
    v["right_children"] = rc;
    v["split_conditions"] = cond;
    v["split_indices"] = idx;
    v["split_type"] = stype;
    v["sum_hessian"] = hess;
    trees_json.push_back(v);
    tree_info.push_back(Json((int64_t)tree.group));
  }
  for (size_t r = 0; r <= trees.size(); ++r) indptr.push_back(Json((int64_t)r));
  Json gbm = Json::object();
  Json gbtree_param = Json::object();
  gbtree_param["num_parallel_tree"] = "1";
  gbtree_param["num_trees"] = std::to_string(trees.size());
  gbm["gbtree_model_param"] = gbtree_param;
  gbm["iteration_indptr"] = indptr;
  gbm["tree_info"] = tree_info;
  gbm["trees"] = trees_json;
  Json booster = Json::object();
  booster["model"] = gbm;
  booster["name"] = "gbtree";
  Json lmp = Json::object();
  lmp["base_score"] = "[" + format_float(base_score) + "]";
  lmp["boost_from_average"] = params_.count("base_score") ? "0" : "1";
  lmp["num_class"] = "0";
  lmp["num_feature"] = std::to_string(num_feature);
  lmp["num_target"] = "1";
  Json objective_json = Json::object();
  objective_json["name"] = objective_name();
  int obj = objective();
  if (obj == 1 || obj == 2) {
    Json rp = Json::object();
    rp["scale_pos_weight"] = param("scale_pos_weight", "1");
    objective_json["reg_loss_param"] = rp;
  } else {
    objective_json["reg_loss_param"] = Json::object();
    objective_json["reg_loss_param"]["scale_pos_weight"] = "1";
  }
  Json attrs = Json::object();
  for (auto const& kv : attributes) attrs[kv.first] = kv.second;
  Json fnames = Json::array(), ftypes = Json::array();
  for (auto const& s : feature_names) fnames.push_back(s);
  for (auto const& s : feature_types) ftypes.push_back(s);
  Json learner = Json::object();
  learner["attributes"] = attrs;
  learner["feature_names"] = fnames;
  learner["feature_types"] = ftypes;
  learner["gradient_booster"] = booster;
  learner["learner_model_param"] = lmp;
  learner["objective"] = objective_json;
  Json root = Json::object();
  root["learner"] = learner;
  Json version = Json::array();
  version.push_back(3); version.push_back(5); version.push_back(0);
  root["version"] = version;
  return root;
}

static float json_float(const Json& v) {
  if (v.is_string()) return std::stof(v.string());
  return (float)v.number();
}

void Learner::load_model(const Json& input) {
  drain();  // queued rounds finish before the model they belong to is replaced
  const Json& learner = input.at("learner");
  const Json& booster = learner.at("gradient_booster");
  require(booster.at("name").string() == "gbtree", "Only gbtree models can be loaded.");
  const Json& mp = learner.at("learner_model_param");
  auto as_uint = [](const Json& v) -> uint32_t {
    return v.is_string() ? (uint32_t)std::stoul(v.string()) : (uint32_t)v.integer();
  };
  num_feature = as_uint(mp.at("num_feature"));
  std::string bs = mp.at("base_score").is_string() ? mp.at("base_score").string() : mp.at("base_score").dump();
  if (!bs.empty() && bs[0] == '[') {
    Json arr = Json::parse(bs);
    require(arr.size() == 1, "Only single-output models are supported.");
    base_score = json_float(arr.items().front());
  } else {
    base_score = std::stof(bs);
  }
  if (learner.contains("objective")) params_["objective"] = learner.at("objective").at("name").string();
  const Json& source = booster.at("model").at("trees");
  std::vector<Tree> loaded;
  for (const Json& t : source.items()) {
    Tree tree;
    const auto& lc = t.at("left_children");
    size_t n = lc.size();
    tree.nodes.resize(n);
    for (size_t i = 0; i < n; ++i) {
      MgbTreeNode& node = tree.nodes[i];
      node.left = (int32_t)t.at("left_children")[i].integer();
      node.right = (int32_t)t.at("right_children")[i].integer();
      int64_t parent = t.at("parents")[i].integer();
      node.parent = parent == 2147483647 ? -1 : (int32_t)parent;
      node.default_left = (uint32_t)t.at("default_left")[i].integer();
      node.gain = json_float(t.at("loss_changes")[i]);
      node.cover = json_float(t.at("sum_hessian")[i]);
      node.base_weight = json_float(t.at("base_weights")[i]);
      float cond = json_float(t.at("split_conditions")[i]);
      if (node.left < 0) {
        node.leaf = cond;
        node.threshold = 0;
        node.feature = -1;
      } else {
        node.threshold = cond;
        node.leaf = 0;
        node.feature = (int32_t)t.at("split_indices")[i].integer();
      }
    }
    loaded.push_back(std::move(tree));
  }
  trees = std::move(loaded);
  feature_names.clear();
  feature_types.clear();
  if (learner.contains("feature_names"))
    for (auto const& s : learner.at("feature_names").items()) feature_names.push_back(s.string());
  if (learner.contains("feature_types"))
    for (auto const& s : learner.at("feature_types").items()) feature_types.push_back(s.string());
  attributes.clear();
  if (learner.contains("attributes"))
    for (auto const& kv : learner.at("attributes").members()) attributes.emplace_back(kv.first, kv.second.string());
  initialized = true;
  cache_id_ = 0;
  cache_trees_ = 0;
  model_version_ = SIZE_MAX;
  metrics.clear();  // src/model.cpp:224
  // A loaded model restarts the engine from seed 0 (src/model.cpp:225).
  rng_.seed(0);
  rng_seed_ = "0";
}

Json Learner::config() const {
  Json p = Json::object();
  for (auto const& kv : params_) p[kv.first] = kv.second;
  Json learner = Json::object();
  learner["params"] = p;
  Json metric_list = Json::array();
  for (auto const& m : metrics) {
    Json entry = Json::object();
    entry["name"] = m;
    metric_list.push_back(entry);
  }
  learner["metrics"] = metric_list;
  Json ltp = Json::object();
  ltp["objective"] = objective_name();
  ltp["booster"] = "gbtree";
  learner["learner_train_param"] = ltp;
  // The engine's state, so a serialised booster continues the same stream.
  std::ostringstream state;
  state << rng_;
  Json generic = Json::object();
  generic["seed"] = rng_seed_;
  generic["rng_state"] = state.str();
  learner["generic_param"] = generic;
  Json root = Json::object();
  root["learner"] = learner;
  Json version = Json::array();
  version.push_back(3); version.push_back(5); version.push_back(0);
  root["version"] = version;
  return root;
}

void Learner::load_config(const Json& cfg) {
  const Json& learner = cfg.at("learner");
  if (learner.contains("params"))
    for (auto const& kv : learner.at("params").members())
      params_[kv.first] = kv.second.is_string() ? kv.second.string() : kv.second.dump();
  if (learner.contains("metrics")) {
    metrics.clear();
    for (auto const& m : learner.at("metrics").items()) metrics.push_back(m.at("name").string());
  }
  if (learner.contains("generic_param")) {
    const Json& generic = learner.at("generic_param");
    if (generic.contains("rng_state") && generic.contains("seed")) {
      std::istringstream state(generic.at("rng_state").string());
      state >> rng_;
      require(!state.fail(), "Invalid rng_state in the booster configuration.");
      rng_seed_ = generic.at("seed").string();
    }
  }
}

void Learner::reset() {
  drain();
  d_margin_.release();
  d_grad_.release();
  d_tree_ws_.release();
  d_pending_.release();
  cache_id_ = 0;
  cache_trees_ = 0;
}

Json Learner::profile() const {
  Json out = Json::object();
  Json secs = Json::object();
  for (auto const& kv : seconds_) secs[kv.first] = Json(kv.second);
  out["seconds"] = secs;
  out["rounds"] = Json((uint64_t)rounds_timed_);
  static const char* names[MGB_PROF_KINDS] = {"gradient", "histogram", "split", "control", "partition", "predict",
                                              "reduce"};
  double ms[MGB_PROF_KINDS] = {0};
  uint64_t launches[MGB_PROF_KINDS] = {0};
  mgb_profile_read(ms, launches, MGB_PROF_KINDS);
  Json kernels = Json::object();
  for (int k = 0; k < MGB_PROF_KINDS; ++k) {
    Json e = Json::object();
    e["ms"] = Json(ms[k]);
    e["launches"] = Json(launches[k]);
    kernels[names[k]] = e;
  }
  out["kernels"] = kernels;
  out["histogram_bytes"] = Json(hist_bytes_);
  out["histogram_rows"] = Json(hist_rows_);
  out["split_bytes"] = Json(split_bytes_);
  out["histogram_bytes_sampled_features"] = Json(hist_bytes_sampled_);
  out["split_bytes_sampled_features"] = Json(split_bytes_sampled_);
  out["partition_bytes"] = Json(partition_bytes_);
  // The last profiled tree, per level: rows and nodes whose histograms were built.
  Json lr = Json::array(), ln = Json::array();
  for (uint64_t v : level_rows_) lr.push_back(Json(v));
  for (uint32_t v : level_nodes_) ln.push_back(Json((uint64_t)v));
  out["level_rows_built"] = lr;
  out["level_nodes_built"] = ln;
  return out;
}

}  // namespace mgb
