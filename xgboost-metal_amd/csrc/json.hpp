// Minimal JSON value, parser and writer for the C API boundary: array
// interface descriptors, booster configuration and the XGBoost JSON model.
#pragma once
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace mgb {

class Json {
 public:
  enum class Type { Null, Bool, Number, String, Array, Object };
  Json() = default;
  Json(std::nullptr_t) {}
  Json(bool b) : type_(Type::Bool), bool_(b) {}
  Json(int v) : type_(Type::Number), num_(v), int_(v), is_int_(true) {}
  Json(int64_t v) : type_(Type::Number), num_((double)v), int_(v), is_int_(true) {}
  Json(uint64_t v) : type_(Type::Number), num_((double)v), int_((int64_t)v), is_int_(true) {}
  Json(uint32_t v) : type_(Type::Number), num_(v), int_(v), is_int_(true) {}
  Json(double v) : type_(Type::Number), num_(v), int_((int64_t)v) {}
  Json(float v) : type_(Type::Number), num_(v), int_((int64_t)v), is_float_(true) {}
  Json(const char* s) : type_(Type::String), str_(s) {}
  Json(std::string s) : type_(Type::String), str_(std::move(s)) {}

  static Json array() { Json j; j.type_ = Type::Array; return j; }
  static Json object() { Json j; j.type_ = Type::Object; return j; }
  static Json parse(const std::string& text);

  Type type() const { return type_; }
  bool is_null() const { return type_ == Type::Null; }
  bool is_number() const { return type_ == Type::Number; }
  bool is_string() const { return type_ == Type::String; }
  bool is_array() const { return type_ == Type::Array; }
  bool is_object() const { return type_ == Type::Object; }
  bool is_bool() const { return type_ == Type::Bool; }

  double number() const { expect(Type::Number); return num_; }
  int64_t integer() const { expect(Type::Number); return is_int_ ? int_ : (int64_t)num_; }
  bool boolean() const { expect(Type::Bool); return bool_; }
  const std::string& string() const { expect(Type::String); return str_; }

  // Arrays.
  void push_back(Json v) { expect(Type::Array); arr_.push_back(std::move(v)); }
  size_t size() const { return type_ == Type::Array ? arr_.size() : type_ == Type::Object ? obj_.size() : 0; }
  const Json& operator[](size_t i) const { expect(Type::Array); return arr_.at(i); }
  const std::vector<Json>& items() const { expect(Type::Array); return arr_; }

  // Objects (insertion order is kept for stable output).
  Json& operator[](const std::string& key);
  const Json& at(const std::string& key) const;
  bool contains(const std::string& key) const;
  const std::vector<std::pair<std::string, Json>>& members() const { expect(Type::Object); return obj_; }

  std::string dump() const;
  // Universal Binary JSON (the default XGBoost model format).
  std::string dump_ubj() const;
  static Json parse_ubj(const std::string& bytes);

 private:
  void expect(Type t) const {
    if (type_ != t) throw std::runtime_error("JSON value has an unexpected type");
  }
  void dump_to(std::string& out) const;
  void ubj_to(std::string& out) const;
  Type type_ = Type::Null;
  bool bool_ = false;
  double num_ = 0;
  int64_t int_ = 0;
  bool is_int_ = false;
  bool is_float_ = false;
  std::string str_;
  std::vector<Json> arr_;
  std::vector<std::pair<std::string, Json>> obj_;
};

std::string format_float(float v);

}  // namespace mgb
