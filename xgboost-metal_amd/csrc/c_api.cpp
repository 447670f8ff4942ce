// XGBoost C API subset for the HIP hist engine (the drop-in boundary).
// Counterpart of the reference's src/c_api.cpp: same entry points, argument
// meaning and error convention (0 / -1 plus a thread-local message), with
// handles owning C++ objects and returned buffers kept in thread-local storage
// until the next call on the same thread.
#include "xgboost_c_api.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <memory>
#include <sstream>

#include "learner.hpp"

using namespace mgb;

namespace {

thread_local std::string g_last_error;
struct Results {
  std::string str, str2;
  std::vector<std::string> strings;
  std::vector<const char*> pointers;
  std::vector<float> floats;
  std::vector<bst_ulong> shape;
  std::vector<uint64_t> indptr;
  std::vector<float> values;
};
thread_local Results g_results;
thread_local Json g_global_config = [] {
  Json j = Json::object();
  j["verbosity"] = Json((int64_t)1);
  j["use_rmm"] = Json(false);
  j["nthread"] = Json((int64_t)0);
  return j;
}();
void (*g_log_callback)(const char*) = nullptr;

using MatrixPtr = std::shared_ptr<DMatrix>;
MatrixPtr& matrix(DMatrixHandle h) {
  require(h != nullptr, "DMatrix handle is null.");
  return *static_cast<MatrixPtr*>(h);
}
Learner& booster(BoosterHandle h) {
  require(h != nullptr, "Booster handle is null.");
  return *static_cast<Learner*>(h);
}

#define API_BEGIN try {
#define API_END                                   \
  }                                               \
  catch (std::exception const& e) {               \
    g_last_error = e.what();                      \
    return -1;                                    \
  }                                               \
  catch (...) {                                   \
    g_last_error = "unknown error";               \
    return -1;                                    \
  }                                               \
  return 0;

// numpy __array_interface__ descriptor -> float32 values (row-major).
struct ArrayView {
  const uint8_t* data = nullptr;
  std::vector<int64_t> shape;
  std::vector<int64_t> strides;  // bytes
  char kind = 'f';
  int itemsize = 4;
};

ArrayView parse_interface(const char* text) {
  Json j = Json::parse(text);
  if (j.is_array()) {
    require(j.size() == 1, "Only a single array interface is supported.");
    j = j.items().front();
  }
  ArrayView v;
  const Json& data = j.at("data");
  v.data = reinterpret_cast<const uint8_t*>((uintptr_t)data.items().front().integer());
  for (auto const& d : j.at("shape").items()) v.shape.push_back(d.integer());
  std::string ts = j.at("typestr").string();
  require(ts.size() >= 3, "Invalid typestr.");
  require(ts[0] != '>', "Big-endian arrays are not supported.");
  v.kind = ts[1];
  v.itemsize = std::stoi(ts.substr(2));
  if (j.contains("strides") && !j.at("strides").is_null()) {
    for (auto const& s : j.at("strides").items()) v.strides.push_back(s.integer());
  } else {
    int64_t step = v.itemsize;
    v.strides.assign(v.shape.size(), 0);
    for (int k = (int)v.shape.size() - 1; k >= 0; --k) {
      v.strides[k] = step;
      step *= v.shape[k];
    }
  }
  if (j.contains("mask") && !j.at("mask").is_null()) throw Error("Masked arrays are not supported.");
  return v;
}

float load_value(const ArrayView& v, int64_t offset) {
  const uint8_t* p = v.data + offset;
  switch (v.kind) {
    case 'f':
      if (v.itemsize == 4) { float f; std::memcpy(&f, p, 4); return f; }
      if (v.itemsize == 8) { double d; std::memcpy(&d, p, 8); return (float)d; }
      if (v.itemsize == 2) {
        uint16_t h; std::memcpy(&h, p, 2);
        uint32_t sign = (h >> 15) & 1, exp = (h >> 10) & 0x1f, mant = h & 0x3ff;
        float f;
        if (exp == 0) f = std::ldexp((float)mant, -24);
        else if (exp == 31) f = mant ? NAN : INFINITY;
        else f = std::ldexp((float)(mant | 0x400), (int)exp - 25);
        return sign ? -f : f;
      }
      break;
    case 'i':
      if (v.itemsize == 1) return (float)*(const int8_t*)p;
      if (v.itemsize == 2) { int16_t x; std::memcpy(&x, p, 2); return (float)x; }
      if (v.itemsize == 4) { int32_t x; std::memcpy(&x, p, 4); return (float)x; }
      if (v.itemsize == 8) { int64_t x; std::memcpy(&x, p, 8); return (float)x; }
      break;
    case 'u':
      if (v.itemsize == 1) return (float)*(const uint8_t*)p;
      if (v.itemsize == 2) { uint16_t x; std::memcpy(&x, p, 2); return (float)x; }
      if (v.itemsize == 4) { uint32_t x; std::memcpy(&x, p, 4); return (float)x; }
      if (v.itemsize == 8) { uint64_t x; std::memcpy(&x, p, 8); return (float)x; }
      break;
    case 'b':
      return *p ? 1.0f : 0.0f;
  }
  throw Error("Unsupported array dtype.");
}

std::vector<float> to_vector(const ArrayView& v) {
  int64_t n = 1;
  for (auto d : v.shape) n *= d;
  std::vector<float> out((size_t)n);
  // C-contiguous float32: one copy.
  bool contiguous = v.kind == 'f' && v.itemsize == 4;
  for (size_t k = 0, step = 4; contiguous && k < v.shape.size(); ++k) {
    const size_t axis = v.shape.size() - 1 - k;
    contiguous = v.shape[axis] <= 1 || v.strides[axis] == (int64_t)step;
    step *= (size_t)v.shape[axis];
  }
  if (contiguous) {
    if (n) std::memcpy(out.data(), v.data, (size_t)n * sizeof(float));
    return out;
  }
  if (v.shape.size() == 1) {
    for (int64_t i = 0; i < n; ++i) out[i] = load_value(v, i * v.strides[0]);
  } else if (v.shape.size() == 2) {
    int64_t cols = v.shape[1];
    for (int64_t r = 0; r < v.shape[0]; ++r)
      for (int64_t c = 0; c < cols; ++c) out[r * cols + c] = load_value(v, r * v.strides[0] + c * v.strides[1]);
  } else {
    throw Error("Only 1- and 2-dimensional arrays are supported.");
  }
  return out;
}

float config_missing(const char* config) {
  if (!config || !*config) return NAN;
  Json c = Json::parse(config);
  if (!c.contains("missing")) return NAN;
  const Json& m = c.at("missing");
  if (m.is_null()) return NAN;
  return (float)m.number();
}

void apply_missing(std::vector<float>& data, float missing) {
  if (std::isnan(missing)) return;
  for (auto& x : data) if (x == missing) x = NAN;
}

void set_quantile(DMatrix& d, const char* config) {
  if (!config || !*config) return;
  Json c = Json::parse(config);
  if (c.contains("max_bin") && c.contains("quantile") && c.at("quantile").is_bool() && c.at("quantile").boolean()) {
    d.is_quantile = true;
    d.quantile_max_bin = (uint32_t)c.at("max_bin").integer();
  }
}

DMatrixHandle new_handle(std::shared_ptr<DMatrix> d) { return new MatrixPtr(std::move(d)); }

std::string array_interface(const void* ptr, size_t n, const char* typestr) {
  Json j = Json::object();
  Json data = Json::array();
  data.push_back(Json((uint64_t)(uintptr_t)ptr));
  data.push_back(Json(true));
  j["data"] = data;
  Json shape = Json::array();
  shape.push_back(Json((uint64_t)n));
  j["shape"] = shape;
  j["strides"] = Json();
  j["typestr"] = typestr;
  j["version"] = Json((int64_t)3);
  return j.dump();
}

}  // namespace

extern "C" {

const char* XGBGetLastError(void) { return g_last_error.c_str(); }

void XGBoostVersion(int* major, int* minor, int* patch) {
  if (major) *major = 3;
  if (minor) *minor = 5;
  if (patch) *patch = 0;
}

int XGBuildInfo(char const** out) {
  API_BEGIN
  Json info = Json::object();
  info["BACKEND"] = "hip";
  info["USE_HIP"] = Json(true);
  info["USE_CUDA"] = Json(false);
  info["USE_NCCL"] = Json(false);
  info["USE_OPENMP"] = Json(false);
  info["HIP_ARCH"] = "gfx950";
  info["DEBUG"] = Json(false);
  g_results.str = info.dump();
  *out = g_results.str.c_str();
  API_END
}

int XGBRegisterLogCallback(void (*callback)(const char*)) {
  API_BEGIN
  g_log_callback = callback;
  API_END
}

int XGBSetGlobalConfig(char const* config) {
  API_BEGIN
  Json c = Json::parse(config);
  for (auto const& kv : c.members()) g_global_config[kv.first] = kv.second;
  API_END
}

int XGBGetGlobalConfig(char const** out_config) {
  API_BEGIN
  g_results.str = g_global_config.dump();
  *out_config = g_results.str.c_str();
  API_END
}

// ---- DMatrix ----------------------------------------------------------------

int XGDMatrixCreateFromDense(char const* data, char const* config, DMatrixHandle* out) {
  API_BEGIN
  ArrayView v = parse_interface(data);
  require(v.shape.size() == 2, "Dense data must be 2-dimensional.");
  auto d = std::make_shared<DMatrix>();
  d->rows = (uint32_t)v.shape[0];
  d->cols = (uint32_t)v.shape[1];
  require((uint64_t)v.shape[0] < (1ull << 32) && (uint64_t)v.shape[1] < (1ull << 32), "Matrix is too large.");
  d->data = to_vector(v);
  apply_missing(d->data, config_missing(config));
  set_quantile(*d, config);
  *out = new_handle(std::move(d));
  API_END
}

int XGDMatrixCreateFromMat(const float* data, bst_ulong nrow, bst_ulong ncol, float missing, DMatrixHandle* out) {
  API_BEGIN
  auto d = std::make_shared<DMatrix>();
  d->rows = (uint32_t)nrow;
  d->cols = (uint32_t)ncol;
  d->data.assign(data, data + nrow * ncol);
  apply_missing(d->data, missing);
  *out = new_handle(std::move(d));
  API_END
}

int XGDMatrixCreateFromCSR(char const* indptr, char const* indices, char const* data, bst_ulong ncol,
                           char const* config, DMatrixHandle* out) {
  API_BEGIN
  ArrayView ip = parse_interface(indptr), ix = parse_interface(indices), dv = parse_interface(data);
  require(ip.shape.size() == 1 && ix.shape.size() == 1 && dv.shape.size() == 1, "CSR arrays must be 1-dimensional.");
  auto d = std::make_shared<DMatrix>();
  int64_t rows = ip.shape[0] - 1;
  require(rows >= 0 && rows < (int64_t)1 << 32, "Invalid CSR indptr.");
  require(ncol < ((bst_ulong)1 << 32), "Too many CSR columns.");
  d->rows = (uint32_t)rows;
  d->cols = (uint32_t)ncol;
  d->sparse = true;
  float missing = config_missing(config);
  // Entries absent from the CSR structure are missing values; stored entries
  // equal to `missing` too (NaN).  Each row's columns are sorted (stable, so
  // a repeated column keeps its first entry's position and is rejected).
  d->indptr.resize((size_t)rows + 1);
  d->indptr[0] = 0;
  std::vector<std::pair<uint32_t, float>> row;
  for (int64_t r = 0; r < rows; ++r) {
    int64_t b = (int64_t)load_value(ip, r * ip.strides[0]);
    int64_t e = (int64_t)load_value(ip, (r + 1) * ip.strides[0]);
    require(b >= 0 && e >= b && e <= ix.shape[0] && e <= dv.shape[0], "Invalid CSR indptr.");
    row.clear();
    bool sorted = true;
    for (int64_t k = b; k < e; ++k) {
      int64_t c = (int64_t)load_value(ix, k * ix.strides[0]);
      require(c >= 0 && (uint64_t)c < ncol, "CSR column index out of range.");
      float x = load_value(dv, k * dv.strides[0]);
      if (!std::isnan(missing) && x == missing) x = NAN;
      if (!row.empty() && (uint32_t)c <= row.back().first) sorted = false;
      row.emplace_back((uint32_t)c, x);
    }
    if (!sorted) {
      std::stable_sort(row.begin(), row.end(), [](const auto& a, const auto& z) { return a.first < z.first; });
      for (size_t i = 1; i < row.size(); ++i)
        require(row[i].first != row[i - 1].first, "CSR row " + std::to_string(r) + " repeats a column index.");
    }
    for (const auto& [c, x] : row) {
      d->indices.push_back(c);
      d->values.push_back(x);
    }
    d->indptr[(size_t)r + 1] = d->indices.size();
  }
  set_quantile(*d, config);
  *out = new_handle(std::move(d));
  API_END
}

int XGDMatrixFree(DMatrixHandle handle) {
  API_BEGIN
  delete static_cast<MatrixPtr*>(handle);
  API_END
}

int XGDMatrixSetInfoFromInterface(DMatrixHandle handle, char const* field, char const* data) {
  API_BEGIN
  ArrayView v = parse_interface(data);
  std::vector<float> values = to_vector(v);
  matrix(handle)->set_info(field, values.data(), values.size());
  API_END
}

int XGDMatrixSetFloatInfo(DMatrixHandle handle, const char* field, const float* array, bst_ulong len) {
  API_BEGIN
  matrix(handle)->set_info(field, array, (size_t)len);
  API_END
}

int XGDMatrixGetFloatInfo(const DMatrixHandle handle, const char* field, bst_ulong* out_len, const float** out_dptr) {
  API_BEGIN
  const auto& v = matrix(handle)->get_info(field);
  *out_len = v.size();
  *out_dptr = v.data();
  API_END
}

int XGDMatrixSetStrFeatureInfo(DMatrixHandle handle, const char* field, const char** features, const bst_ulong size) {
  API_BEGIN
  std::vector<std::string> values(features, features + size);
  std::string f = field;
  if (f == "feature_name") matrix(handle)->feature_names = values;
  else if (f == "feature_type") {
    for (auto const& t : values) require(t != "c", "Categorical features are not supported by this engine.");
    matrix(handle)->feature_types = values;
  } else throw Error("Unknown feature info field: " + f);
  API_END
}

int XGDMatrixGetStrFeatureInfo(DMatrixHandle handle, const char* field, bst_ulong* size, const char*** out_features) {
  API_BEGIN
  std::string f = field;
  g_results.strings = f == "feature_name" ? matrix(handle)->feature_names : matrix(handle)->feature_types;
  g_results.pointers.clear();
  for (auto const& s : g_results.strings) g_results.pointers.push_back(s.c_str());
  *size = g_results.strings.size();
  *out_features = g_results.pointers.data();
  API_END
}

int XGDMatrixNumRow(DMatrixHandle handle, bst_ulong* out) {
  API_BEGIN
  *out = matrix(handle)->rows;
  API_END
}

int XGDMatrixNumCol(DMatrixHandle handle, bst_ulong* out) {
  API_BEGIN
  *out = matrix(handle)->cols;
  API_END
}

int XGDMatrixNumNonMissing(DMatrixHandle handle, bst_ulong* out) {
  API_BEGIN
  *out = matrix(handle)->nonmissing();
  API_END
}

int XGDMatrixGetQuantileCut(DMatrixHandle const handle, char const* config, char const** out_indptr,
                            char const** out_data) {
  API_BEGIN
  auto& d = *matrix(handle);
  uint32_t max_bin = d.quantized_max_bin;
  if (!max_bin && config && *config) {
    Json c = Json::parse(config);
    if (c.contains("max_bin")) max_bin = (uint32_t)c.at("max_bin").integer();
  }
  if (!max_bin && d.is_quantile) max_bin = d.quantile_max_bin;
  require(max_bin != 0, "The DMatrix has no quantile cuts yet; train a booster on it first.");
  const bool same = d.quantized_max_bin == max_bin;
  d.quantize(max_bin, same ? d.quantized_layout : 0, same ? d.quantized_group_request : 0);
  g_results.indptr.assign(1, 0);
  g_results.values.clear();
  for (uint32_t f = 0; f < d.cols; ++f) {
    for (uint32_t i = 0; i < d.counts_host[f]; ++i) g_results.values.push_back(d.cuts_host[(size_t)f * max_bin + i]);
    g_results.indptr.push_back(g_results.values.size());
  }
  g_results.str = array_interface(g_results.indptr.data(), g_results.indptr.size(), "<u8");
  g_results.str2 = array_interface(g_results.values.data(), g_results.values.size(), "<f4");
  *out_indptr = g_results.str.c_str();
  *out_data = g_results.str2.c_str();
  API_END
}

// ---- Booster ------------------------------------------------------------------

int XGBoosterCreate(const DMatrixHandle dmats[], bst_ulong len, BoosterHandle* out) {
  API_BEGIN
  for (bst_ulong i = 0; i < len; ++i) require(dmats[i] != nullptr, "Null DMatrix in the booster cache.");
  *out = new Learner();
  API_END
}

int XGBoosterFree(BoosterHandle handle) {
  API_BEGIN
  delete static_cast<Learner*>(handle);
  API_END
}

int XGBoosterReset(BoosterHandle handle) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  b.reset();
  API_END
}

int XGBoosterSetParam(BoosterHandle handle, const char* name, const char* value) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  b.set_param(name, value ? value : "");
  API_END
}

int XGBoosterSetParams(BoosterHandle handle, char const* config) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  Json c = Json::parse(config);
  for (auto const& kv : c.members()) b.set_param(kv.first, kv.second.is_string() ? kv.second.string() : kv.second.dump());
  API_END
}

int XGBoosterUpdateOneIter(BoosterHandle handle, int iter, DMatrixHandle dtrain) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  b.update(*matrix(dtrain), iter);
  API_END
}

int XGBoosterBoostOneIter(BoosterHandle handle, DMatrixHandle dtrain, float* grad, float* hess, bst_ulong len) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  b.boost(*matrix(dtrain), grad, hess, (size_t)len);
  API_END
}

int XGBoosterTrainOneIter(BoosterHandle handle, DMatrixHandle dtrain, int /*iter*/, char const* grad,
                          char const* hess) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  ArrayView g = parse_interface(grad), h = parse_interface(hess);
  require(g.shape == h.shape, "Gradient and Hessian shapes must match.");
  require(g.shape.size() == 1 || (g.shape.size() == 2 && g.shape[1] == 1),
          "Only single-output custom objectives are supported.");
  if (g.shape.size() == 2) { g.shape.resize(1); h.shape.resize(1); g.strides.resize(1); h.strides.resize(1); }
  auto gv = to_vector(g), hv = to_vector(h);
  b.boost(*matrix(dtrain), gv.data(), hv.data(), gv.size());
  API_END
}

int XGBoosterEvalOneIter(BoosterHandle handle, int iter, DMatrixHandle dmats[], const char* evnames[], bst_ulong len,
                         const char** out_result) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  std::vector<DMatrix*> data;
  std::vector<std::string> names;
  for (bst_ulong i = 0; i < len; ++i) {
    data.push_back(matrix(dmats[i]).get());
    names.push_back(evnames[i]);
  }
  g_results.str = b.evaluate(iter, data, names);
  *out_result = g_results.str.c_str();
  API_END
}

int XGBoosterPredictFromDMatrix(BoosterHandle handle, DMatrixHandle dmat, char const* config,
                                bst_ulong const** out_shape, bst_ulong* out_dim, float const** out_result) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  Json c = config && *config ? Json::parse(config) : Json::object();
  int64_t type = c.contains("type") ? c.at("type").integer() : 0;
  require(type == 0 || type == 1, "Only value (type 0) and margin (type 1) predictions are supported.");
  uint32_t begin = c.contains("iteration_begin") ? (uint32_t)c.at("iteration_begin").integer() : 0;
  uint32_t end = c.contains("iteration_end") ? (uint32_t)c.at("iteration_end").integer() : 0;
  bool strict = c.contains("strict_shape") && c.at("strict_shape").is_bool() && c.at("strict_shape").boolean();
  auto& d = *matrix(dmat);
  g_results.floats = b.predict(d, type == 1, begin, end);
  g_results.shape.clear();
  g_results.shape.push_back(d.rows);
  if (strict) g_results.shape.push_back(1);
  *out_shape = g_results.shape.data();
  *out_dim = g_results.shape.size();
  *out_result = g_results.floats.data();
  API_END
}

int XGBoosterSaveModelToBuffer(BoosterHandle handle, char const* config, bst_ulong* out_len, char const** out_dptr) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  std::string format = "ubj";
  if (config && *config) {
    Json c = Json::parse(config);
    if (c.contains("format")) format = c.at("format").string();
  }
  require(format == "json" || format == "ubj", "Model format must be json or ubj.");
  g_results.str = format == "json" ? b.model().dump() : b.model().dump_ubj();
  *out_len = g_results.str.size();
  *out_dptr = g_results.str.data();
  API_END
}

int XGBoosterLoadModelFromBuffer(BoosterHandle handle, const void* buf, bst_ulong len) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  std::string bytes(static_cast<const char*>(buf), (size_t)len);
  require(!bytes.empty(), "Empty model buffer.");
  b.load_model(bytes[0] == '{' && bytes.size() > 1 && (bytes[1] == '"' || bytes[1] == ' ' || bytes[1] == '\n')
                   ? Json::parse(bytes)
                   : Json::parse_ubj(bytes));
  API_END
}

int XGBoosterSaveModel(BoosterHandle handle, const char* fname) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  std::string name = fname;
  bool json = name.size() >= 5 && name.substr(name.size() - 5) == ".json";
  std::string bytes = json ? b.model().dump() : b.model().dump_ubj();
  std::ofstream out(name, std::ios::binary);
  require(out.good(), "Cannot open " + name);
  out.write(bytes.data(), (std::streamsize)bytes.size());
  API_END
}

int XGBoosterLoadModel(BoosterHandle handle, const char* fname) {
  API_BEGIN
  std::ifstream in(fname, std::ios::binary);
  require(in.good(), std::string("Cannot open ") + fname);
  std::stringstream ss;
  ss << in.rdbuf();
  std::string bytes = ss.str();
  return XGBoosterLoadModelFromBuffer(handle, bytes.data(), bytes.size());
  API_END
}

int XGBoosterSerializeToBuffer(BoosterHandle handle, bst_ulong* out_len, const char** out_dptr) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  Json all = Json::object();
  all["Config"] = b.config();
  all["Model"] = b.model();
  g_results.str = all.dump_ubj();
  *out_len = g_results.str.size();
  *out_dptr = g_results.str.data();
  API_END
}

int XGBoosterUnserializeFromBuffer(BoosterHandle handle, const void* buf, bst_ulong len) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  Json all = Json::parse_ubj(std::string(static_cast<const char*>(buf), (size_t)len));
  // Model first: loading a model restarts the engine, the configuration then
  // restores the serialised engine state.
  b.load_model(all.at("Model"));
  b.load_config(all.at("Config"));
  API_END
}

int XGBoosterSaveJsonConfig(BoosterHandle handle, bst_ulong* out_len, char const** out_str) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  g_results.str = b.config().dump();
  *out_len = g_results.str.size();
  *out_str = g_results.str.c_str();
  API_END
}

int XGBoosterLoadJsonConfig(BoosterHandle handle, char const* config) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  b.load_config(Json::parse(config));
  API_END
}

int XGBoosterBoostedRounds(BoosterHandle handle, int* out) {
  API_BEGIN
  *out = (int)booster(handle).boosted_rounds();
  API_END
}

int XGBoosterGetNumFeature(BoosterHandle handle, bst_ulong* out) {
  API_BEGIN
  *out = booster(handle).num_feature;
  API_END
}

int XGBoosterGetAttr(BoosterHandle handle, const char* key, const char** out, int* success) {
  API_BEGIN
  *success = 0;
  for (auto const& kv : booster(handle).attributes)
    if (kv.first == key) {
      g_results.str = kv.second;
      *out = g_results.str.c_str();
      *success = 1;
    }
  API_END
}

int XGBoosterSetAttr(BoosterHandle handle, const char* key, const char* value) {
  API_BEGIN
  auto& attrs = booster(handle).attributes;
  for (size_t i = 0; i < attrs.size(); ++i)
    if (attrs[i].first == key) {
      if (value) attrs[i].second = value;
      else attrs.erase(attrs.begin() + (long)i);
      return 0;
    }
  if (value) attrs.emplace_back(key, value);
  API_END
}

int XGBoosterGetAttrNames(BoosterHandle handle, bst_ulong* out_len, const char*** out) {
  API_BEGIN
  g_results.strings.clear();
  for (auto const& kv : booster(handle).attributes) g_results.strings.push_back(kv.first);
  g_results.pointers.clear();
  for (auto const& s : g_results.strings) g_results.pointers.push_back(s.c_str());
  *out_len = g_results.strings.size();
  *out = g_results.pointers.data();
  API_END
}

int XGBoosterSetStrFeatureInfo(BoosterHandle handle, const char* field, const char** features, const bst_ulong size) {
  API_BEGIN
  std::vector<std::string> values(features, features + size);
  std::string f = field;
  if (f == "feature_name") booster(handle).feature_names = values;
  else if (f == "feature_type") booster(handle).feature_types = values;
  else throw Error("Unknown feature info field: " + f);
  API_END
}

int XGBoosterGetStrFeatureInfo(BoosterHandle handle, const char* field, bst_ulong* len, const char*** out_features) {
  API_BEGIN
  std::string f = field;
  g_results.strings = f == "feature_name" ? booster(handle).feature_names : booster(handle).feature_types;
  g_results.pointers.clear();
  for (auto const& s : g_results.strings) g_results.pointers.push_back(s.c_str());
  *len = g_results.strings.size();
  *out_features = g_results.pointers.data();
  API_END
}

int XGBoosterHipProfile(BoosterHandle handle, const char** out) {
  API_BEGIN
  g_results.str = booster(handle).profile().dump();
  *out = g_results.str.c_str();
  API_END
}

}  // extern "C"
