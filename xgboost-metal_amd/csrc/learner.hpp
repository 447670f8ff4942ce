// Host side of the hist engine: data matrices, the boosting loop and the
// XGBoost JSON model.  All numeric work on the path runs in the HIP kernels
// behind include/mgb_kernels.h; this layer owns device buffers, parameters,
// tree records and the model format.
//
// Reference counterparts: include/metalgb/engine.hpp:86-427 (Matrix, Tree,
// Learner), src/learner.cpp:207-985 (initialize, update), src/data.cpp
// (dense/CSR ingest, quantize), src/model.cpp:28-74 (JSON model).
#pragma once
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <random>
#include <string>
#include <vector>

#include "json.hpp"
#include "mgb_kernels.h"

namespace mgb {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};
void require(bool ok, const std::string& message);

// Owning device allocation (hipMalloc through the kernel C ABI).
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer() { release(); }
  void* get() const { return ptr_; }
  template <class T> T* as() const { return static_cast<T*>(ptr_); }
  size_t bytes() const { return bytes_; }
  void resize(size_t bytes);          // contents are not preserved
  void ensure(size_t bytes) { if (bytes > bytes_ || !ptr_) resize(bytes); }
  void upload(const void* host, size_t bytes);
  void download(void* host, size_t bytes) const;
  void release();

 private:
  void* ptr_ = nullptr;
  size_t bytes_ = 0;
};

void kcheck(int status, const char* what);

// Copies `bytes` of device memory at `src` into a pinned host buffer the
// library reuses (runtime.hip), waits for the copy, and calls `use` on it
// while holding the buffer; 0, or -1 with the library's error set.
int download_pinned(const void* src, size_t bytes, const std::function<void(const uint8_t*)>& use);

struct DMatrix {
  uint64_t id = 0;                    // unique per matrix; keys the prediction cache
  uint32_t rows = 0, cols = 0;
  std::vector<float> data;            // row-major, NaN marks missing (dense matrices)
  // CSR matrices (sparse = true): rows+1 offsets, strictly increasing column
  // indices within a row, values (NaN marks missing; absent entries too).
  bool sparse = false;
  std::vector<uint64_t> indptr;
  std::vector<uint32_t> indices;
  std::vector<float> values;
  DeviceBuffer d_indptr, d_indices, d_values, d_codes;
  DeviceBuffer d_colptr, d_csc_rows, d_csc_codes;  // column-major copy (root histogram)
  MgbCsrMatrix csr{};
  std::vector<float> labels, weights, base_margin;
  std::vector<std::string> feature_names, feature_types;
  bool is_quantile = false;
  uint32_t quantile_max_bin = 0;

  // Device state.
  DeviceBuffer d_data, d_labels, d_weights;
  bool data_uploaded = false, labels_uploaded = false, weights_uploaded = false;
  int labels_in_unit = -1;            // all labels in [0, 1]: 1 / 0, -1 = not checked since set
  uint32_t quantized_max_bin = 0;     // requested max_bin of the bins below (0: none)
  int quantized_layout = 0;           // layout request the bins below were built for
  uint32_t quantized_group_request = 0;  // hip_histogram_features request (0: rule)
  uint32_t hist_bins = 0;             // bins per feature in histograms = min(max_bin, rows)
  uint32_t features_per_group = 16;
  bool has_missing = false;
  MgbMatrix matrix{};
  DeviceBuffer d_cuts, d_counts, d_bins, d_missing;
  DeviceBuffer d_columns;             // the codes again, column-major, for the row partition
  std::vector<float> cuts_host;        // cols * max_bin, host copy for export
  std::vector<uint32_t> counts_host;
  double sketch_seconds = 0, quantize_seconds = 0;

  DMatrix();
  void upload();
  void upload_info();
  // Cuts and bin matrix for max_bin; layout 0 = automatic (group-major when a
  // row's codes exceed 128 bytes), 1 = row-major, 2 = group-major.
  void quantize(uint32_t max_bin, int layout = 0, uint32_t group_request = 0);
  uint32_t choose_group(uint32_t request) const;
  void relayout(int layout);
  void quantize_sparse(uint32_t max_bin);
  // A matrix without rows: cuts only (no device work, nothing to bin).
  void quantize_empty(uint32_t max_bin, int layout, uint32_t group_request);
  void take_cuts(uint32_t max_bin);
  std::shared_ptr<DMatrix> cut_source;  // QuantileDMatrix ref: take its cuts instead of sketching
  uint64_t nonmissing() const;
  void set_info(const std::string& field, const float* values, size_t count);
  const std::vector<float>& get_info(const std::string& field) const;
};

// std::shuffle of `order` over a 32-bit engine, with the draws of either
// standard library: libstdc++ (x86-64 Linux builds, stock XGBoost's wheels)
// or libc++ (the reference's macOS builds).
enum class ShuffleModel { libstdcxx, libcxx };
void std_shuffle(std::vector<uint32_t>& order, std::mt19937& engine, ShuffleModel model);
// "libstdc++" or "libc++"; anything else throws.
ShuffleModel shuffle_model(const std::string& name);

struct Tree {
  std::vector<MgbTreeNode> nodes;
  uint32_t group = 0;
};

class Learner {
 public:
  Learner();
  ~Learner();
  std::recursive_mutex mutex;

  void set_param(const std::string& name, const std::string& value);
  std::string param(const std::string& name, const std::string& fallback) const;
  double number(const std::string& name, double fallback) const;
  float fnumber(const std::string& name, float fallback) const;
  int64_t integer(const std::string& name, int64_t fallback) const;

  // One boosting round with the configured objective (src/learner.cpp:632-985).
  void update(DMatrix& data, int iteration);
  // One round with caller gradients (custom objective).
  void boost(DMatrix& data, const float* grad, const float* hess, size_t count);
  // Predictions (margin when output_margin) for rounds [begin, end); end 0 = all.
  std::vector<float> predict(DMatrix& data, bool output_margin, uint32_t begin, uint32_t end);
  // Leaf indices (type 6: rows x trees), feature contributions (type 2
  // exact, 3 approximate: rows x (cols + 1), the bias last) or their
  // interactions (4 exact, 5 approximate: rows x (cols + 1)^2) of rounds
  // [0, end); end 0 = all (src/learner.cpp:455-560).
  std::vector<float> predict_explain(DMatrix& data, int type, uint32_t end);
  // The same predictions left on the device: in `scratch`, or in the
  // training-matrix cache when that holds them already.
  const float* predict_device(DMatrix& data, bool output_margin, uint32_t begin, uint32_t end, DeviceBuffer& scratch);
  // "[iteration]\t<name>-<metric>:<value>..." over every metric and matrix
  // (src/learner.cpp:1025-1048).
  std::string evaluate(int iteration, const std::vector<DMatrix*>& data, const std::vector<std::string>& names);
  // One metric of predictions `pred` (device) against data's labels
  // (src/metrics.cpp:8-159).
  double metric(DMatrix& data, const float* pred, const std::string& name);
  std::string default_metric() const;
  // eval_metric values in the order first set, each once.
  std::vector<std::string> metrics;

  Json model() const;
  void load_model(const Json& model);
  Json config() const;
  void load_config(const Json& config);
  void reset();
  Json profile() const;

  // Rounds whose node records are still only on the device: each round's
  // kernels are queued without a host synchronisation; drain() waits for them
  // and appends their trees.  Everything that reads the model drains first.
  void drain();
  uint32_t boosted_rounds() const { return (uint32_t)(trees.size() + pending_.size()); }
  uint32_t num_feature = 0;
  std::vector<Tree> trees;
  std::vector<std::pair<std::string, std::string>> attributes;
  std::vector<std::string> feature_names, feature_types;
  float base_score = 0.5f;
  bool initialized = false;

 private:
  int objective() const;
  std::string objective_name() const;
  void configure_check() const;
  void initialize(DMatrix& data, bool custom);
  // sampled: the round's gradients drop rows (subsample < 1), which leave the row list.
  void grow(DMatrix& data, bool unit_hessian, bool sampled);
  // A round on a matrix without rows: a single leaf of weight 0, no device work.
  void empty_round();
  void configure_rng();
  int bin_layout() const;
  // Per-round row-sampling parameters (src/learner.cpp:679, src/sampling.cpp:11-17).
  void sample_rows(DMatrix& data, MgbGradParams& gp);
  // The tree's column sample as per-feature flags on the device, or NULL.
  const uint32_t* sample_columns(uint32_t cols);
  // Device copy of monotone_constraints for `cols` features (NULL when every
  // feature is unconstrained).
  const int32_t* monotone_constraints(uint32_t cols);
  float base_margin_value() const;
  void upload_model();
  DeviceBuffer* margin_cache(DMatrix& data);
  void predict_into(DMatrix& data, const uint32_t* offsets, uint32_t count, float* margin);

  std::map<std::string, std::string> params_;
  // Training-matrix prediction cache.
  uint64_t cache_id_ = 0;
  size_t cache_trees_ = 0;
  DeviceBuffer d_margin_;
  // Round buffers.
  DeviceBuffer d_grad_, d_mass_, d_scales_, d_tree_ws_, d_node_count_, d_base_;
  // Model on the device for prediction.
  DeviceBuffer d_model_nodes_, d_model_offsets_;
  DeviceBuffer d_model_means_;  // each node's cover-weighted mean leaf value (contributions)
  size_t means_version_ = SIZE_MAX;
  size_t model_version_ = SIZE_MAX, model_trees_ = 0;
  size_t uploaded_trees_ = 0;
  std::map<std::string, double> seconds_;
  uint64_t rounds_timed_ = 0;
  uint64_t hist_bytes_ = 0, hist_rows_ = 0, split_bytes_ = 0, partition_bytes_ = 0;
  uint64_t hist_bytes_sampled_ = 0, split_bytes_sampled_ = 0;  // counting only the column sample's features
  std::vector<uint64_t> level_rows_;
  std::vector<uint32_t> level_nodes_;
  // The learner's engine (src/learner.cpp:94-103): default-constructed state
  // until a "seed" other than the last one applied reseeds it.
  std::mt19937 rng_;
  std::string rng_seed_ = "0";
  DeviceBuffer d_features_;
  std::vector<uint32_t> feature_flags_;
  DeviceBuffer d_monotone_;
  std::vector<int32_t> monotone_;         // parsed constraints, cols entries
  std::string monotone_text_ = "()";      // the parameter they were parsed from
  bool monotone_active_ = false;
  DeviceBuffer d_eval_pred_, d_metric_ws_;
  // Queued rounds: node records (then the node count) at `offset` in d_pending_.
  struct Pending {
    size_t offset, node_bytes;
    uint32_t max_nodes;
  };
  std::vector<Pending> pending_;
  DeviceBuffer d_pending_;
  size_t pending_bytes_ = 0;
};

}  // namespace mgb
