// XGBoost C API subset for the HIP hist engine (the drop-in boundary).
// Counterpart of the reference's src/c_api.cpp: same entry points, argument
// meaning and error convention (0 / -1 plus a thread-local message), with
// handles owning C++ objects and returned buffers kept in thread-local storage
// until the next call on the same thread.
#include "xgboost_c_api.h"

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstring>
#include <fstream>
#include <functional>
#include <iomanip>
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
  j["std_shuffle"] = Json("libstdc++");  // xgb.cv's fold shuffle (XGDMatrixBuildCVFolds)
  return j;
}();
void (*g_log_callback)(const char*) = nullptr;

using MatrixPtr = std::shared_ptr<DMatrix>;
MatrixPtr& matrix(DMatrixHandle h) {
  require(h != nullptr, "DMatrix handle is null.");
  return *static_cast<MatrixPtr*>(h);
}
// The booster with its queued rounds completed: every entry point that reads
// the model uses this one.
Learner& booster(BoosterHandle h) {
  require(h != nullptr, "Booster handle is null.");
  Learner& b = *static_cast<Learner*>(h);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  b.drain();
  return b;
}

// The booster as it is, rounds possibly still queued on the device: for the
// per-round entry points (updates, parameters, attributes), which never read
// the trees and must not wait for the device.
Learner& booster_queued(BoosterHandle h) {
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

// Dense matrix from an __array_interface__ (one feature per column).
std::shared_ptr<DMatrix> dense_matrix(const char* interface, float missing) {
  ArrayView v = parse_interface(interface);
  require(v.shape.size() == 2, "Dense data must be 2-dimensional.");
  require((uint64_t)v.shape[0] < (1ull << 32) && (uint64_t)v.shape[1] < (1ull << 32), "Matrix is too large.");
  auto d = std::make_shared<DMatrix>();
  d->rows = (uint32_t)v.shape[0];
  d->cols = (uint32_t)v.shape[1];
  d->data = to_vector(v);
  apply_missing(d->data, missing);
  return d;
}

// Dense matrix from a JSON list of per-column array interfaces.
std::shared_ptr<DMatrix> columnar_matrix(const char* text, float missing) {
  Json columns = Json::parse(text);
  require(columns.is_array() && columns.size() > 0, "Columnar data must be a non-empty list of array interfaces.");
  auto d = std::make_shared<DMatrix>();
  d->cols = (uint32_t)columns.size();
  std::vector<std::vector<float>> cols;
  for (auto const& c : columns.items()) {
    std::string one = c.dump();
    ArrayView v = parse_interface(one.c_str());
    require(v.shape.size() == 1, "Each column of columnar data must be 1-dimensional.");
    cols.push_back(to_vector(v));
    require(cols.back().size() == cols.front().size(), "Columns of columnar data differ in length.");
  }
  d->rows = (uint32_t)cols.front().size();
  d->data.resize((size_t)d->rows * d->cols);
  for (uint32_t f = 0; f < d->cols; ++f)
    for (uint32_t r = 0; r < d->rows; ++r) d->data[(size_t)r * d->cols + f] = cols[f][r];
  apply_missing(d->data, missing);
  return d;
}

// CSR matrix from per-row entry lists: stored entries equal to `missing`
// become NaN (missing); each row's columns are sorted (stable) and a repeated
// column is rejected.  `row_entries(r, out)` appends row r's (column, value)
// pairs.
template <typename RowFn>
std::shared_ptr<DMatrix> csr_matrix(uint64_t rows, uint64_t ncol, float missing, RowFn row_entries) {
  require(rows < (1ull << 32), "Too many rows.");
  require(ncol < (1ull << 32), "Too many columns.");
  auto d = std::make_shared<DMatrix>();
  d->rows = (uint32_t)rows;
  d->cols = (uint32_t)ncol;
  d->sparse = true;
  d->indptr.resize(rows + 1);
  d->indptr[0] = 0;
  std::vector<std::pair<uint32_t, float>> row;
  for (uint64_t r = 0; r < rows; ++r) {
    row.clear();
    row_entries(r, row);
    bool sorted = true;
    for (size_t i = 0; i < row.size(); ++i) {
      require(row[i].first < ncol, "Sparse column index out of range.");
      if (!std::isnan(missing) && row[i].second == missing) row[i].second = NAN;
      if (i && row[i].first <= row[i - 1].first) sorted = false;
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
    d->indptr[r + 1] = d->indices.size();
  }
  return d;
}

std::shared_ptr<DMatrix> csr_from_interfaces(const char* indptr, const char* indices, const char* data, uint64_t ncol,
                                             float missing) {
  ArrayView ip = parse_interface(indptr), ix = parse_interface(indices), dv = parse_interface(data);
  require(ip.shape.size() == 1 && ix.shape.size() == 1 && dv.shape.size() == 1, "CSR arrays must be 1-dimensional.");
  const int64_t rows = ip.shape[0] - 1;
  require(rows >= 0, "Invalid CSR indptr.");
  return csr_matrix((uint64_t)rows, ncol, missing, [&](uint64_t r, std::vector<std::pair<uint32_t, float>>& row) {
    const int64_t b = (int64_t)load_value(ip, (int64_t)r * ip.strides[0]);
    const int64_t e = (int64_t)load_value(ip, (int64_t)(r + 1) * ip.strides[0]);
    require(b >= 0 && e >= b && e <= ix.shape[0] && e <= dv.shape[0], "Invalid CSR indptr.");
    for (int64_t k = b; k < e; ++k) {
      const int64_t c = (int64_t)load_value(ix, k * ix.strides[0]);
      require(c >= 0, "CSR column index out of range.");
      row.emplace_back((uint32_t)c, load_value(dv, k * dv.strides[0]));
    }
  });
}

// Batches of a data iterator appended in order (src/c_api.cpp:140-157): one
// dense matrix when every batch is dense, else one CSR matrix (a dense
// batch's NaN entries are absent); labels, weights and base margins are
// concatenated when every batch has them.
std::shared_ptr<DMatrix> concatenate(const std::vector<std::shared_ptr<DMatrix>>& batches, float missing) {
  require(!batches.empty(), "The iterator produced no batch.");
  const uint32_t cols = batches.front()->cols;
  bool any_sparse = false;
  uint64_t rows = 0;
  for (auto const& b : batches) {
    require(b->cols == cols, "Iterator batches differ in their number of features.");
    any_sparse = any_sparse || b->sparse;
    rows += b->rows;
  }
  require(cols > 0, "The iterator produced no feature data.");
  std::shared_ptr<DMatrix> out;
  if (!any_sparse) {
    out = std::make_shared<DMatrix>();
    out->rows = (uint32_t)rows;
    out->cols = cols;
    out->data.reserve((size_t)rows * cols);
    for (auto const& b : batches) out->data.insert(out->data.end(), b->data.begin(), b->data.end());
    apply_missing(out->data, missing);
  } else {
    size_t bi = 0;
    uint64_t base = 0;
    out = csr_matrix(rows, cols, missing, [&](uint64_t r, std::vector<std::pair<uint32_t, float>>& row) {
      while (r - base >= batches[bi]->rows) base += batches[bi++]->rows;
      const DMatrix& b = *batches[bi];
      const uint64_t lr = r - base;
      if (b.sparse) {
        for (uint64_t k = b.indptr[lr]; k < b.indptr[lr + 1]; ++k) row.emplace_back(b.indices[k], b.values[k]);
      } else {
        for (uint32_t c = 0; c < cols; ++c) {
          const float x = b.data[(size_t)lr * cols + c];
          if (!std::isnan(x)) row.emplace_back(c, x);
        }
      }
    });
  }
  auto info = [&](auto field) {
    size_t have = 0;
    for (auto const& b : batches) have += !(b.get()->*field).empty();
    require(have == 0 || have == batches.size(), "Some iterator batches carry labels, weights or base margins and "
                                                 "others do not.");
    if (!have) return;
    for (auto const& b : batches) {
      require((b.get()->*field).size() == b->rows, "An iterator batch's meta info length differs from its rows.");
      (out.get()->*field).insert((out.get()->*field).end(), (b.get()->*field).begin(), (b.get()->*field).end());
    }
  };
  info(&DMatrix::labels);
  info(&DMatrix::weights);
  info(&DMatrix::base_margin);
  out->feature_names = batches.front()->feature_names;
  out->feature_types = batches.front()->feature_types;
  return out;
}

std::shared_ptr<DMatrix> from_iterator(DataIterHandle iter, DMatrixHandle proxy, DataIterResetCallback* reset,
                                       XGDMatrixCallbackNext* next, const char* config) {
  require(reset && next && proxy, "Iterator callbacks and proxy must be provided.");
  Json c = config && *config ? Json::parse(config) : Json::object();
  require(!c.contains("cache_prefix") || c.at("cache_prefix").is_null() || c.at("cache_prefix").string().empty(),
          "External memory (cache_prefix) is not supported by this engine.");
  std::vector<std::shared_ptr<DMatrix>> batches;
  reset(iter);
  for (;;) {
    const int status = next(iter);
    require(status >= 0, "Data iterator callback failed.");
    if (!status) break;
    batches.push_back(matrix(proxy));
  }
  reset(iter);
  return concatenate(batches, config_missing(config));
}

// Feature map file: "<index> <name> <type>" per line (XGBoost's text format);
// the names it lists replace those in `names`.
void read_feature_map(const std::string& path, std::vector<std::string>& names) {
  std::ifstream in(path);
  require(in.good(), "Cannot open feature map " + path);
  std::string line;
  while (std::getline(in, line)) {
    std::istringstream fields(line);
    long idx;
    std::string name;
    if (!(fields >> idx >> name)) continue;
    require(idx >= 0, "Negative index in the feature map.");
    if ((size_t)idx >= names.size()) names.resize((size_t)idx + 1);
    names[(size_t)idx] = name;
  }
}

// Rows `index` of `source` with their labels, weights and base margins
// (src/data.cpp:1451); a slice of a quantile matrix keeps the source's cuts.
std::shared_ptr<DMatrix> slice_rows(const std::shared_ptr<DMatrix>& source, const int* index, size_t len) {
  const DMatrix& src = *source;
  for (size_t i = 0; i < len; ++i)
    require(index[i] >= 0 && (uint32_t)index[i] < src.rows, "Slice index out of range.");
  std::shared_ptr<DMatrix> d;
  if (src.sparse) {
    d = csr_matrix(len, src.cols, NAN, [&](uint64_t i, std::vector<std::pair<uint32_t, float>>& row) {
      const uint32_t r = (uint32_t)index[i];
      for (uint64_t k = src.indptr[r]; k < src.indptr[r + 1]; ++k) row.emplace_back(src.indices[k], src.values[k]);
    });
  } else {
    d = std::make_shared<DMatrix>();
    d->rows = (uint32_t)len;
    d->cols = src.cols;
    d->data.resize(len * src.cols);
    for (size_t i = 0; i < len; ++i)
      std::memcpy(d->data.data() + i * src.cols, src.data.data() + (size_t)index[i] * src.cols, src.cols * 4);
  }
  auto pick = [&](const std::vector<float>& v, std::vector<float>& o) {
    if (v.empty()) return;
    o.resize(len);
    for (size_t i = 0; i < len; ++i) o[i] = v[(size_t)index[i]];
  };
  pick(src.labels, d->labels);
  pick(src.weights, d->weights);
  pick(src.base_margin, d->base_margin);
  d->feature_names = src.feature_names;
  d->feature_types = src.feature_types;
  if (src.is_quantile) {
    d->is_quantile = true;
    d->quantile_max_bin = src.quantile_max_bin;
    d->cut_source = source;
  }
  return d;
}

std::vector<std::string> feature_names_of(const Learner& b) {
  std::vector<std::string> names = b.feature_names;
  if (names.empty())
    for (uint32_t f = 0; f < b.num_feature; ++f) names.push_back("f" + std::to_string(f));
  return names;
}

std::string number_text(double v) {
  std::ostringstream out;
  out << std::setprecision(9) << v;
  return out.str();
}

// A float widened to double in the number layout of the reference's JSON
// writer (nlohmann::json, include/metalgb/engine.hpp:22): the shortest digits
// that round-trip the double; plain decimals for decimal exponents in
// (-4, 15], otherwise d.ddde+XX with at least two exponent digits; integral
// values keep ".0"; non-finite values print as nan / inf (src/data.cpp:69-99).
std::string json_number(double v) {
  if (std::isnan(v)) return "nan";
  if (std::isinf(v)) return v < 0 ? "-inf" : "inf";
  std::string out;
  if (std::signbit(v)) { out += '-'; v = -v; }
  if (v == 0) return out + "0.0";
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof buf, v, std::chars_format::scientific);
  const std::string sci(buf, r.ptr);  // d[.ddd]e±XX
  const size_t e = sci.find('e');
  std::string digits = sci.substr(0, e);
  digits.erase(std::remove(digits.begin(), digits.end(), '.'), digits.end());
  const int k = (int)digits.size();
  const int n = std::stoi(sci.substr(e + 1)) + 1;  // decimal point position after `digits`[0..n)
  if (k <= n && n <= 15) return out + digits + std::string(n - k, '0') + ".0";
  if (0 < n && n <= 15) return out + digits.substr(0, n) + "." + digits.substr(n);
  if (-4 < n && n <= 0) return out + "0." + std::string(-n, '0') + digits;
  out += digits.substr(0, 1);
  if (k > 1) out += "." + digits.substr(1);
  const int x = n - 1;
  out += x < 0 ? "e-" : "e+";
  const int a = x < 0 ? -x : x;
  if (a < 10) out += '0';
  return out + std::to_string(a);
}

std::string json_string(const std::string& s) {
  std::string out = "\"";
  for (unsigned char c : s) {
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\n': out += "\\n"; break;
      case '\t': out += "\\t"; break;
      case '\r': out += "\\r"; break;
      case '\b': out += "\\b"; break;
      case '\f': out += "\\f"; break;
      default:
        if (c < 0x20) {
          char u[8];
          std::snprintf(u, sizeof u, "\\u%04x", c);
          out += u;
        } else {
          out += (char)c;
        }
    }
  }
  return out + "\"";
}

// Text, JSON and dot dumps of one tree in the reference's formats
// (src/model.cpp:334-428).  The JSON dump is indented by 2 with its keys in
// byte order, as the reference's JSON object (a sorted map) prints them.
std::string dump_tree(const Tree& tree, const std::vector<std::string>& names, const std::string& format, bool stats) {
  const auto& n = tree.nodes;
  auto name = [&](int32_t f) { return f >= 0 && (size_t)f < names.size() ? names[f] : "f" + std::to_string(f); };
  std::ostringstream out;
  if (format == "json") {
    std::function<void(int32_t, uint32_t, size_t)> node = [&](int32_t id, uint32_t depth, size_t level) {
      const MgbTreeNode& x = n.at(id);
      const std::string pad(2 * level, ' '), inner(2 * level + 2, ' ');
      std::vector<std::pair<const char*, std::string>> members;  // byte order of the keys
      const bool split = x.left >= 0;
      if (split) members.emplace_back("children", "");
      if (stats) members.emplace_back("cover", json_number(x.cover));
      if (split) {
        members.emplace_back("depth", std::to_string(depth));
        if (stats) members.emplace_back("gain", json_number(x.gain));
        members.emplace_back("missing", std::to_string(x.default_left ? x.left : x.right));
        members.emplace_back("no", std::to_string(x.right));
      } else {
        members.emplace_back("leaf", json_number(x.leaf));
      }
      members.emplace_back("nodeid", std::to_string(id));
      if (split) {
        members.emplace_back("split", json_string(name(x.feature)));
        members.emplace_back("split_condition", json_number(x.threshold));
        members.emplace_back("yes", std::to_string(x.left));
      }
      out << "{";
      for (size_t i = 0; i < members.size(); ++i) {
        out << (i ? ",\n" : "\n") << inner << '"' << members[i].first << "\": ";
        if (std::strcmp(members[i].first, "children") == 0) {
          const std::string item(2 * level + 4, ' ');
          out << "[\n" << item;
          node(x.left, depth + 1, level + 2);
          out << ",\n" << item;
          node(x.right, depth + 1, level + 2);
          out << "\n" << inner << "]";
        } else {
          out << members[i].second;
        }
      }
      out << "\n" << pad << "}";
    };
    node(0, 0, 0);
    return out.str();
  }
  require(format == "text" || format == "dot", "Unknown dump format: " + format);
  if (format == "dot") out << "digraph {\n    graph [ rankdir=TB ]\n";
  std::function<void(int32_t, int)> node = [&](int32_t id, int depth) {
    const MgbTreeNode& x = n.at(id);
    if (format == "dot") {
      out << "    " << id << " [ label=\"";
      if (x.left < 0) out << "leaf=" << number_text(x.leaf);
      else out << name(x.feature) << '<' << number_text(x.threshold);
      if (stats) out << "\\ncover=" << number_text(x.cover);
      out << "\" ]\n";
      if (x.left >= 0) {
        out << "    " << id << " -> " << x.left << " [ label=\"yes" << (x.default_left ? ", missing" : "") << "\" ]\n";
        out << "    " << id << " -> " << x.right << " [ label=\"no" << (!x.default_left ? ", missing" : "") << "\" ]\n";
      }
    } else {
      out << std::string(depth, '\t') << id << ':';
      if (x.left < 0) out << "leaf=" << number_text(x.leaf);
      else
        out << '[' << name(x.feature) << '<' << number_text(x.threshold) << "] yes=" << x.left << ",no=" << x.right
            << ",missing=" << (x.default_left ? x.left : x.right);
      if (stats) {
        if (x.left >= 0) out << ",gain=" << number_text(x.gain);
        out << ",cover=" << number_text(x.cover);
      }
      out << '\n';
    }
    if (x.left >= 0) {
      node(x.left, depth + 1);
      node(x.right, depth + 1);
    }
  };
  node(0, 0);
  if (format == "dot") out << "}\n";
  return out.str();
}

void string_output(std::vector<std::string> strings, bst_ulong* len, const char*** out) {
  g_results.strings = std::move(strings);
  g_results.pointers.clear();
  for (auto const& s : g_results.strings) g_results.pointers.push_back(s.c_str());
  *len = g_results.strings.size();
  *out = g_results.pointers.data();
}

// Value (type 0) or margin (type 1) predictions of d into g_results
// (c_api.cpp:499-518): iteration_begin/end select rounds, strict_shape adds
// the output dimension.
void predict_into_results(Learner& b, DMatrix& d, const char* config) {
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  Json c = config && *config ? Json::parse(config) : Json::object();
  const int64_t type = c.contains("type") ? c.at("type").integer() : 0;
  require(type >= 0 && type <= 6, "Invalid prediction type.");
  const uint32_t begin = c.contains("iteration_begin") ? (uint32_t)c.at("iteration_begin").integer() : 0;
  const uint32_t end = c.contains("iteration_end") ? (uint32_t)c.at("iteration_end").integer() : 0;
  const bool strict = c.contains("strict_shape") && c.at("strict_shape").is_bool() && c.at("strict_shape").boolean();
  g_results.shape.clear();
  g_results.shape.push_back(d.rows);
  if (type >= 2) {
    // Leaf and contribution predictions cover rounds [0, end) only
    // (src/learner.cpp:467-469).
    require(begin == 0 || b.trees.empty(),
            "Leaf and contribution predictions support only iteration end; use model slicing for a nonzero start.");
    g_results.floats = b.predict_explain(d, (int)type, end);
    if (type == 6) {
      // (src/learner.cpp:549-551): one tree gives a vector, strict_shape
      // rows x rounds x groups x parallel trees.
      const uint64_t n = d.rows ? g_results.floats.size() / d.rows : (uint64_t)b.trees.size();
      if (strict) {
        g_results.shape.push_back(n);
        g_results.shape.push_back(1);
        g_results.shape.push_back(1);
      } else if (n != 1) {
        g_results.shape.push_back(n);
      }
    } else {
      if (strict) g_results.shape.push_back(1);
      g_results.shape.push_back((uint64_t)d.cols + 1);
      if (type == 4 || type == 5) g_results.shape.push_back((uint64_t)d.cols + 1);
    }
    return;
  }
  g_results.floats = b.predict(d, type == 1, begin, end);
  if (strict) g_results.shape.push_back(1);
}

int unsupported(const std::string& what) {
  g_last_error = what + " is not supported by the MI355X hist engine.";
  return -1;
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
  auto d = dense_matrix(data, config_missing(config));
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
  // Entries absent from the CSR structure are missing values; stored entries
  // equal to `missing` too (NaN).
  auto d = csr_from_interfaces(indptr, indices, data, ncol, config_missing(config));
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
  auto& b = booster_queued(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  b.set_param(name, value ? value : "");
  API_END
}

int XGBoosterSetParams(BoosterHandle handle, char const* config) {
  API_BEGIN
  auto& b = booster_queued(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  Json c = Json::parse(config);
  for (auto const& kv : c.members()) b.set_param(kv.first, kv.second.is_string() ? kv.second.string() : kv.second.dump());
  API_END
}

int XGBoosterUpdateOneIter(BoosterHandle handle, int iter, DMatrixHandle dtrain) {
  API_BEGIN
  auto& b = booster_queued(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  b.update(*matrix(dtrain), iter);
  API_END
}

int XGBoosterBoostOneIter(BoosterHandle handle, DMatrixHandle dtrain, float* grad, float* hess, bst_ulong len) {
  API_BEGIN
  auto& b = booster_queued(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  b.boost(*matrix(dtrain), grad, hess, (size_t)len);
  API_END
}

int XGBoosterTrainOneIter(BoosterHandle handle, DMatrixHandle dtrain, int /*iter*/, char const* grad,
                          char const* hess) {
  API_BEGIN
  auto& b = booster_queued(handle);
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
  predict_into_results(booster(handle), *matrix(dmat), config);
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
  for (auto const& kv : booster_queued(handle).attributes)
    if (kv.first == key) {
      g_results.str = kv.second;
      *out = g_results.str.c_str();
      *success = 1;
    }
  API_END
}

int XGBoosterSetAttr(BoosterHandle handle, const char* key, const char* value) {
  API_BEGIN
  auto& attrs = booster_queued(handle).attributes;
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
  for (auto const& kv : booster_queued(handle).attributes) g_results.strings.push_back(kv.first);
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

// Engine extension: the matrix's values, labels and weights are copied to the
// device when first used (quantization, prediction); this copies them now and
// waits, so that a caller can time training on device-resident input, as the
// reference's DMatrix construction fills its device buffers up front
// (src/data.cpp:485-520).
int XGDMatrixHipUpload(DMatrixHandle handle) {
  API_BEGIN
  auto& m = matrix(handle);
  m->upload();
  m->upload_info();
  kcheck(mgb_synchronize(), "synchronize");
  API_END
}

// ---------------------------------------------------------------------------
// Other layouts, iterators, slicing (c_api.cpp:195-313)
// ---------------------------------------------------------------------------
int XGDMatrixCreateFromCSC(char const* indptr, char const* indices, char const* data, bst_ulong nrow,
                           char const* config, DMatrixHandle* out) {
  API_BEGIN
  ArrayView cp = parse_interface(indptr), ri = parse_interface(indices), dv = parse_interface(data);
  require(cp.shape.size() == 1 && ri.shape.size() == 1 && dv.shape.size() == 1, "CSC arrays must be 1-dimensional.");
  const int64_t ncol = cp.shape[0] - 1;
  require(ncol >= 0, "Invalid CSC indptr.");
  // Column order: each row receives its entries with increasing columns.
  std::vector<std::vector<std::pair<uint32_t, float>>> rows((size_t)nrow);
  for (int64_t c = 0; c < ncol; ++c) {
    const int64_t b = (int64_t)load_value(cp, c * cp.strides[0]), e = (int64_t)load_value(cp, (c + 1) * cp.strides[0]);
    require(b >= 0 && e >= b && e <= ri.shape[0] && e <= dv.shape[0], "Invalid CSC indptr.");
    for (int64_t k = b; k < e; ++k) {
      const int64_t r = (int64_t)load_value(ri, k * ri.strides[0]);
      require(r >= 0 && (uint64_t)r < nrow, "CSC row index out of range.");
      rows[(size_t)r].emplace_back((uint32_t)c, load_value(dv, k * dv.strides[0]));
    }
  }
  auto d = csr_matrix(nrow, (uint64_t)ncol, config_missing(config),
                      [&](uint64_t r, std::vector<std::pair<uint32_t, float>>& row) { row = std::move(rows[r]); });
  set_quantile(*d, config);
  *out = new_handle(std::move(d));
  API_END
}

int XGDMatrixCreateFromCOO(char const* row_idx, char const* col_idx, char const* data, bst_ulong nrow, bst_ulong ncol,
                           char const* config, DMatrixHandle* out) {
  API_BEGIN
  ArrayView ri = parse_interface(row_idx), ci = parse_interface(col_idx), dv = parse_interface(data);
  require(ri.shape.size() == 1 && ci.shape.size() == 1 && dv.shape.size() == 1, "COO arrays must be 1-dimensional.");
  require(ri.shape[0] == ci.shape[0] && ri.shape[0] == dv.shape[0], "COO arrays differ in length.");
  std::vector<std::vector<std::pair<uint32_t, float>>> rows((size_t)nrow);
  for (int64_t k = 0; k < ri.shape[0]; ++k) {
    const int64_t r = (int64_t)load_value(ri, k * ri.strides[0]), c = (int64_t)load_value(ci, k * ci.strides[0]);
    require(r >= 0 && (uint64_t)r < nrow && c >= 0 && (uint64_t)c < ncol, "COO index out of range.");
    rows[(size_t)r].emplace_back((uint32_t)c, load_value(dv, k * dv.strides[0]));
  }
  auto d = csr_matrix(nrow, ncol, config_missing(config),
                      [&](uint64_t r, std::vector<std::pair<uint32_t, float>>& row) { row = std::move(rows[r]); });
  set_quantile(*d, config);
  *out = new_handle(std::move(d));
  API_END
}

int XGDMatrixCreateFromColumnar(char const* data, char const* config, DMatrixHandle* out) {
  API_BEGIN
  auto d = columnar_matrix(data, config_missing(config));
  set_quantile(*d, config);
  *out = new_handle(std::move(d));
  API_END
}

int XGProxyDMatrixCreate(DMatrixHandle* out) {
  API_BEGIN
  *out = new_handle(std::make_shared<DMatrix>());
  API_END
}

int XGProxyDMatrixSetDataDense(DMatrixHandle handle, char const* data) {
  API_BEGIN
  matrix(handle) = dense_matrix(data, NAN);
  API_END
}

int XGProxyDMatrixSetDataColumnar(DMatrixHandle handle, char const* data) {
  API_BEGIN
  matrix(handle) = columnar_matrix(data, NAN);
  API_END
}

int XGProxyDMatrixSetDataCSR(DMatrixHandle handle, char const* indptr, char const* indices, char const* data,
                             bst_ulong ncol) {
  API_BEGIN
  matrix(handle) = csr_from_interfaces(indptr, indices, data, ncol, NAN);
  API_END
}

int XGDMatrixCreateFromCallback(DataIterHandle iter, DMatrixHandle proxy, DataIterResetCallback* reset,
                                XGDMatrixCallbackNext* next, char const* config, DMatrixHandle* out) {
  API_BEGIN
  *out = new_handle(from_iterator(iter, proxy, reset, next, config));
  API_END
}

int XGQuantileDMatrixCreateFromCallback(DataIterHandle iter, DMatrixHandle proxy, DataIterHandle ref,
                                        DataIterResetCallback* reset, XGDMatrixCallbackNext* next, char const* config,
                                        DMatrixHandle* out) {
  API_BEGIN
  Json c = config && *config ? Json::parse(config) : Json::object();
  uint32_t bins = 256;
  if (c.contains("max_bin") && !c.at("max_bin").is_null()) {
    const int64_t v = c.at("max_bin").integer();
    require(v >= 2 && v <= 4096, "max_bin must be in [2, 4096].");
    bins = (uint32_t)v;
  }
  auto d = from_iterator(iter, proxy, reset, next, config);
  d->is_quantile = true;
  d->quantile_max_bin = bins;
  if (ref) d->cut_source = matrix(ref);
  *out = new_handle(std::move(d));
  API_END
}

int XGDMatrixSliceDMatrixEx(DMatrixHandle handle, int const* idxset, bst_ulong len, DMatrixHandle* out,
                            int allow_groups) {
  API_BEGIN
  (void)allow_groups;  // no query groups in this engine
  require(idxset || !len, "Null slice indices.");
  *out = new_handle(slice_rows(matrix(handle), idxset, len));
  API_END
}

int XGDMatrixSliceDMatrix(DMatrixHandle handle, int const* idxset, bst_ulong len, DMatrixHandle* out) {
  return XGDMatrixSliceDMatrixEx(handle, idxset, len, out, 0);
}

int XGDMatrixGetDataAsCSR(DMatrixHandle handle, char const* config, bst_ulong* out_indptr, unsigned* out_indices,
                          float* out_data) {
  API_BEGIN
  (void)config;
  const DMatrix& m = *matrix(handle);
  bst_ulong n = 0;
  out_indptr[0] = 0;
  for (uint32_t r = 0; r < m.rows; ++r) {
    if (m.sparse) {
      for (uint64_t k = m.indptr[r]; k < m.indptr[r + 1]; ++k)
        if (!std::isnan(m.values[k])) { out_indices[n] = m.indices[k]; out_data[n++] = m.values[k]; }
    } else {
      for (uint32_t c = 0; c < m.cols; ++c) {
        const float x = m.data[(size_t)r * m.cols + c];
        if (!std::isnan(x)) { out_indices[n] = c; out_data[n++] = x; }
      }
    }
    out_indptr[r + 1] = n;
  }
  API_END
}

int XGDMatrixGetInfoRef(DMatrixHandle handle, char const* field, char const** out) {
  API_BEGIN
  const std::vector<float>& v = matrix(handle)->get_info(field);
  g_results.str = array_interface(v.data(), v.size(), "<f4");
  *out = g_results.str.c_str();
  API_END
}

int XGDMatrixWasZeroCopied(DMatrixHandle handle, int* out) {
  API_BEGIN
  matrix(handle);
  require(out != nullptr, "Null output pointer.");
  *out = 0;
  API_END
}

// ---------------------------------------------------------------------------
// In-place prediction, importance, slicing, dumps (c_api.cpp:503-598)
// ---------------------------------------------------------------------------
int XGBoosterPredictFromDense(BoosterHandle handle, char const* values, char const* config, DMatrixHandle proxy,
                              bst_ulong const** out_shape, bst_ulong* out_dim, float const** out_result) {
  API_BEGIN
  (void)proxy;
  auto d = dense_matrix(values, config_missing(config));
  predict_into_results(booster(handle), *d, config);
  *out_shape = g_results.shape.data();
  *out_dim = g_results.shape.size();
  *out_result = g_results.floats.data();
  API_END
}

int XGBoosterPredictFromColumnar(BoosterHandle handle, char const* values, char const* config, DMatrixHandle proxy,
                                 bst_ulong const** out_shape, bst_ulong* out_dim, float const** out_result) {
  API_BEGIN
  (void)proxy;
  auto d = columnar_matrix(values, config_missing(config));
  predict_into_results(booster(handle), *d, config);
  *out_shape = g_results.shape.data();
  *out_dim = g_results.shape.size();
  *out_result = g_results.floats.data();
  API_END
}

int XGBoosterPredictFromCSR(BoosterHandle handle, char const* indptr, char const* indices, char const* values,
                            bst_ulong ncol, char const* config, DMatrixHandle proxy, bst_ulong const** out_shape,
                            bst_ulong* out_dim, float const** out_result) {
  API_BEGIN
  (void)proxy;
  auto d = csr_from_interfaces(indptr, indices, values, ncol, config_missing(config));
  predict_into_results(booster(handle), *d, config);
  *out_shape = g_results.shape.data();
  *out_dim = g_results.shape.size();
  *out_result = g_results.floats.data();
  API_END
}

int XGBoosterPredictToBuffer(BoosterHandle handle, DMatrixHandle dmat, char const* config, float* out_buffer,
                             bst_ulong out_capacity, bst_ulong const** out_shape, bst_ulong* out_dim) {
  API_BEGIN
  require(out_shape && out_dim, "Null output shape pointers.");
  predict_into_results(booster(handle), *matrix(dmat), config);
  *out_shape = g_results.shape.data();
  *out_dim = g_results.shape.size();
  require(g_results.floats.size() <= out_capacity, "Output buffer capacity (" + std::to_string(out_capacity) +
                                                       ") is smaller than the prediction size (" +
                                                       std::to_string(g_results.floats.size()) + ").");
  if (!g_results.floats.empty()) {
    require(out_buffer != nullptr, "Null output buffer for a nonempty prediction.");
    std::memcpy(out_buffer, g_results.floats.data(), g_results.floats.size() * sizeof(float));
  }
  API_END
}

int XGBoosterFeatureScore(BoosterHandle handle, char const* config, bst_ulong* out_n_features,
                          char const*** out_features, bst_ulong* out_dim, bst_ulong const** out_shape,
                          float const** out_scores) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  Json c = config && *config ? Json::parse(config) : Json::object();
  const std::string kind = c.contains("importance_type") ? c.at("importance_type").string() : "weight";
  require(kind == "weight" || kind == "gain" || kind == "cover" || kind == "total_gain" || kind == "total_cover",
          "Unknown importance type: " + kind);
  std::vector<std::string> names = b.feature_names;
  if (c.contains("feature_names") && c.at("feature_names").is_array()) {
    names.clear();
    for (auto const& v : c.at("feature_names").items()) names.push_back(v.string());
  }
  if (c.contains("feature_map") && c.at("feature_map").is_string() && !c.at("feature_map").string().empty())
    read_feature_map(c.at("feature_map").string(), names);
  uint32_t nf = b.num_feature;
  for (auto const& t : b.trees)
    for (auto const& n : t.nodes)
      if (n.left >= 0) nf = std::max(nf, (uint32_t)n.feature + 1);
  require(names.empty() || names.size() >= nf, "Feature name length is invalid.");
  std::vector<double> total(nf, 0.0);
  std::vector<uint32_t> count(nf, 0);
  for (auto const& t : b.trees)
    for (auto const& n : t.nodes) {
      if (n.left < 0) continue;
      ++count[n.feature];
      total[n.feature] += kind == "weight" ? 1.0 : (kind == "gain" || kind == "total_gain") ? n.gain : n.cover;
    }
  std::vector<std::string> used;
  g_results.floats.clear();
  for (uint32_t f = 0; f < nf; ++f) {
    if (!count[f]) continue;
    used.push_back(names.empty() ? "f" + std::to_string(f) : names[f]);
    g_results.floats.push_back((float)(total[f] / ((kind == "gain" || kind == "cover") ? count[f] : 1)));
  }
  string_output(std::move(used), out_n_features, out_features);
  g_results.shape.assign(1, *out_n_features);
  *out_dim = 1;
  *out_shape = g_results.shape.data();
  *out_scores = g_results.floats.data();
  API_END
}

// Trees [begin, end) with a stride; end 0 means all rounds (src/model.cpp:430).
// An empty or out-of-range slice returns -2 (src/c_api.cpp:503-506), which the
// Python package turns into IndexError.
int XGBoosterSlice(BoosterHandle handle, int begin_layer, int end_layer, int step, BoosterHandle* out) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  const int rounds = (int)b.trees.size();
  if (end_layer == 0) end_layer = rounds;
  require(step > 0 && begin_layer >= 0, "Invalid model slice.");
  if (end_layer > rounds || begin_layer >= end_layer) {
    g_last_error = "Model slice index out of range.";
    return -2;
  }
  auto copy = std::make_unique<Learner>();
  copy->load_model(b.model());
  copy->load_config(b.config());
  auto& attrs = copy->attributes;
  attrs.erase(std::remove_if(attrs.begin(), attrs.end(),
                             [](auto const& kv) { return kv.first == "best_iteration" || kv.first == "best_score"; }),
              attrs.end());
  std::vector<Tree> kept;
  for (int i = begin_layer; i < end_layer; i += step) kept.push_back(b.trees[(size_t)i]);
  copy->trees = std::move(kept);
  *out = copy.release();
  API_END
}

int XGBoosterDumpModelEx(BoosterHandle handle, char const* fmap, int with_stats, char const* format,
                         bst_ulong* out_len, char const*** out_dump_array) {
  API_BEGIN
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  std::vector<std::string> names = feature_names_of(b);
  if (fmap && *fmap) read_feature_map(fmap, names);
  const std::string fmt = format && *format ? format : "text";
  std::vector<std::string> dumps;
  for (auto const& t : b.trees) dumps.push_back(dump_tree(t, names, fmt, with_stats != 0));
  string_output(std::move(dumps), out_len, out_dump_array);
  API_END
}

int XGBoosterDumpModel(BoosterHandle handle, char const* fmap, int with_stats, bst_ulong* out_len,
                       char const*** out_dump_array) {
  return XGBoosterDumpModelEx(handle, fmap, with_stats, "text", out_len, out_dump_array);
}

int XGBoosterDumpModelExWithFeatures(BoosterHandle handle, int fnum, char const** fname, char const** ftype,
                                     int with_stats, char const* format, bst_ulong* out_len,
                                     char const*** out_models) {
  API_BEGIN
  (void)ftype;
  auto& b = booster(handle);
  std::lock_guard<std::recursive_mutex> lock(b.mutex);
  std::vector<std::string> names(fname, fname + fnum);
  const std::string fmt = format && *format ? format : "text";
  std::vector<std::string> dumps;
  for (auto const& t : b.trees) dumps.push_back(dump_tree(t, names, fmt, with_stats != 0));
  string_output(std::move(dumps), out_len, out_models);
  API_END
}

// ---------------------------------------------------------------------------
// One process; inputs and features this engine does not take
// ---------------------------------------------------------------------------
int XGCommunicatorInit(char const* config) {
  API_BEGIN
  Json c = config && *config ? Json::parse(config) : Json::object();
  require(!c.is_object() || c.members().empty(), "Distributed training is not supported by this engine.");
  API_END
}
int XGCommunicatorFinalize(void) { return 0; }
int XGCommunicatorGetRank(void) { return 0; }
int XGCommunicatorGetWorldSize(void) { return 1; }
int XGCommunicatorIsDistributed(void) { return 0; }
int XGCommunicatorPrint(char const* message) {
  if (g_log_callback) g_log_callback(message);
  else std::fprintf(stderr, "%s\n", message);
  return 0;
}
int XGCommunicatorGetProcessorName(char const** name_str) {
  API_BEGIN
  g_results.str = "localhost";
  *name_str = g_results.str.c_str();
  API_END
}
int XGCommunicatorBroadcast(void*, size_t, int root) {
  API_BEGIN
  require(root == 0, "A single process broadcasts from root 0.");
  API_END
}
int XGCommunicatorAllreduce(void*, size_t, int, int) { return 0; }
int XGCommunicatorSignalError(void) { return unsupported("Distributed error signalling"); }
int XGTrackerCreate(char const*, TrackerHandle*) { return unsupported("Distributed trackers"); }
int XGTrackerWorkerArgs(TrackerHandle, char const**) { return unsupported("Distributed trackers"); }
int XGTrackerRun(TrackerHandle, char const*) { return unsupported("Distributed trackers"); }
int XGTrackerWaitFor(TrackerHandle, char const*) { return unsupported("Distributed trackers"); }
int XGTrackerFree(TrackerHandle) { return 0; }
int XGDMatrixCreateFromCudaArrayInterface(char const*, char const*, DMatrixHandle*) { return unsupported("CUDA input"); }
int XGDMatrixCreateFromCudaColumnar(char const*, char const*, DMatrixHandle*) { return unsupported("CUDA input"); }
int XGProxyDMatrixSetDataCudaArrayInterface(DMatrixHandle, char const*) { return unsupported("CUDA input"); }
int XGProxyDMatrixSetDataCudaColumnar(DMatrixHandle, char const*) { return unsupported("CUDA input"); }
int XGBoosterPredictFromCudaArray(BoosterHandle, char const*, char const*, DMatrixHandle, bst_ulong const**,
                                  bst_ulong*, const float**) {
  return unsupported("CUDA input");
}
int XGBoosterPredictFromCudaColumnar(BoosterHandle, char const*, char const*, DMatrixHandle, bst_ulong const**,
                                     bst_ulong*, const float**) {
  return unsupported("CUDA input");
}
int XGDMatrixCreateFromArrow(void const*, void const*, float, DMatrixHandle*) { return unsupported("Arrow input"); }
int XGDMatrixCreateFromDLPack(void*, int, float, DMatrixHandle*) { return unsupported("DLPack input"); }
int XGDMatrixCreateFromURI(char const*, DMatrixHandle*) { return unsupported("Loading text or binary data files"); }
int XGDMatrixCreateFromBufferDescriptor(void const*, float, DMatrixHandle*) {
  return unsupported("Device buffer-descriptor input");
}
int XGDMatrixSetInfoFromBufferDescriptor(DMatrixHandle, char const*, void const*) {
  return unsupported("Device buffer-descriptor input");
}
int XGBoosterPredictFromBufferDescriptor(BoosterHandle, void const*, char const*, DMatrixHandle, bst_ulong const**,
                                         bst_ulong*, const float**) {
  return unsupported("Device buffer-descriptor input");
}
int XGExtMemQuantileDMatrixCreateFromCallback(DataIterHandle, DMatrixHandle, DataIterHandle, DataIterResetCallback*,
                                              XGDMatrixCallbackNext*, char const*, DMatrixHandle*) {
  return unsupported("External-memory training");
}
int XGBoosterTrainOneIterWithSplitGrad(BoosterHandle, DMatrixHandle, int, char const*, char const*, char const*,
                                       char const*) {
  return unsupported("Separate split and leaf gradients");
}
// Row folds for xgboost.cv (src/c_api.cpp:1018-1110): rows shuffled by
// std::shuffle over mt19937(seed) when `shuffle` (libstdc++'s draws, as an
// x86-64 build of that function makes them); plain folds take
// consecutive chunks of that order (the first nrows % nfold folds one row
// longer), stratified folds deal the order, stably sorted by label, round
// robin.  Fold k tests its rows and trains on the others, both in row order.
int XGDMatrixBuildCVFolds(DMatrixHandle handle, int nfold, unsigned seed, int shuffle, int stratified,
                          DMatrixHandle* out_train, DMatrixHandle* out_test) {
  API_BEGIN
  require(out_train && out_test, "Null CV fold output arrays.");
  require(nfold >= 2, "nfold must be at least 2.");
  std::shared_ptr<DMatrix> m = matrix(handle);
  const uint32_t nrows = m->rows;
  require((uint32_t)nfold <= nrows, "Number of folds cannot exceed number of rows.");
  // The shuffle draws follow the standard library the global config's
  // "std_shuffle" names, as the column sample follows the booster parameter
  // of that name: "libstdc++" (the default, stock XGBoost's x86-64 builds)
  // or "libc++" (the reference's macOS builds).
  ShuffleModel model = ShuffleModel::libstdcxx;
  if (g_global_config.contains("std_shuffle")) {
    const Json& name = g_global_config.at("std_shuffle");
    require(name.is_string(), "std_shuffle must be \"libstdc++\" or \"libc++\".");
    model = shuffle_model(name.string());
  }
  std::mt19937 rng(seed);
  std::vector<uint32_t> order(nrows);
  for (uint32_t r = 0; r < nrows; ++r) order[r] = r;
  if (shuffle && nrows > 1) std_shuffle(order, rng, model);
  std::vector<int> fold(nrows, 0);
  if (stratified) {
    const auto& y = m->labels;
    require(y.size() == nrows, "Stratified CV requires 1D labels matching the number of rows.");
    std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) { return y[a] < y[b]; });
    for (uint32_t pos = 0; pos < nrows; ++pos) fold[order[pos]] = (int)(pos % (uint32_t)nfold);
  } else {
    uint32_t pos = 0;
    for (int k = 0; k < nfold; ++k) {
      const uint32_t chunk = nrows / (uint32_t)nfold + ((uint32_t)k < nrows % (uint32_t)nfold ? 1u : 0u);
      for (uint32_t j = 0; j < chunk; ++j) fold[order[pos++]] = k;
    }
  }
  std::vector<std::shared_ptr<DMatrix>> train(nfold), test(nfold);
  for (int k = 0; k < nfold; ++k) {
    std::vector<int> train_rows, test_rows;
    for (uint32_t r = 0; r < nrows; ++r) (fold[r] == k ? test_rows : train_rows).push_back((int)r);
    train[k] = slice_rows(m, train_rows.data(), train_rows.size());
    test[k] = slice_rows(m, test_rows.data(), test_rows.size());
  }
  for (int k = 0; k < nfold; ++k) {
    out_train[k] = new_handle(std::move(train[k]));
    out_test[k] = new_handle(std::move(test[k]));
  }
  API_END
}
int XGDMatrixSaveBinary(DMatrixHandle, char const*, int) { return unsupported("Saving a DMatrix"); }
int XGDMatrixGetCategories(DMatrixHandle handle, char const*, CategoriesHandle* out) {
  API_BEGIN
  matrix(handle);
  *out = nullptr;
  API_END
}
int XGDMatrixGetCategoriesExportToArrow(DMatrixHandle handle, char const*, CategoriesHandle* out,
                                        char const** export_out) {
  API_BEGIN
  matrix(handle);
  *out = nullptr;
  if (export_out) *export_out = nullptr;
  API_END
}
int XGBoosterGetCategories(BoosterHandle handle, char const*, CategoriesHandle* out) {
  API_BEGIN
  booster(handle);
  *out = nullptr;
  API_END
}
int XGBoosterGetCategoriesExportToArrow(BoosterHandle handle, char const*, CategoriesHandle* out,
                                        char const** export_out) {
  API_BEGIN
  booster(handle);
  *out = nullptr;
  if (export_out) *export_out = nullptr;
  API_END
}
int XGBCategoriesFree(CategoriesHandle handle) {
  API_BEGIN
  require(handle == nullptr, "Unknown categories handle.");
  API_END
}

}  // extern "C"
