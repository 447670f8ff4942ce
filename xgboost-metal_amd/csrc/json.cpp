#include "json.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace mgb {
namespace {

struct Parser {
  const std::string& s;
  size_t i = 0;
  explicit Parser(const std::string& text) : s(text) {}

  [[noreturn]] void fail(const char* what) {
    throw std::runtime_error(std::string("invalid JSON: ") + what + " at offset " + std::to_string(i));
  }
  void ws() {
    while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\t' || s[i] == '\r')) ++i;
  }
  bool lit(const char* word) {
    size_t n = std::strlen(word);
    if (s.compare(i, n, word) == 0) { i += n; return true; }
    return false;
  }
  Json value() {
    ws();
    if (i >= s.size()) fail("unexpected end");
    char c = s[i];
    if (c == '{') return object();
    if (c == '[') return array();
    if (c == '"') return Json(string());
    if (lit("true")) return Json(true);
    if (lit("false")) return Json(false);
    if (lit("null")) return Json();
    if (lit("NaN")) return Json(std::nan(""));
    if (lit("Infinity")) return Json(INFINITY);
    if (lit("-Infinity")) return Json(-INFINITY);
    return number();
  }
  Json number() {
    size_t start = i;
    if (s[i] == '-' || s[i] == '+') ++i;
    bool is_int = true;
    while (i < s.size() && (std::isdigit((unsigned char)s[i]) || s[i] == '.' || s[i] == 'e' || s[i] == 'E' ||
                            s[i] == '-' || s[i] == '+')) {
      if (s[i] == '.' || s[i] == 'e' || s[i] == 'E') is_int = false;
      ++i;
    }
    if (start == i) fail("expected a value");
    std::string text = s.substr(start, i - start);
    if (is_int) {
      errno = 0;
      long long v = std::strtoll(text.c_str(), nullptr, 10);
      if (errno == 0) return Json((int64_t)v);
      unsigned long long u = std::strtoull(text.c_str(), nullptr, 10);
      return Json((uint64_t)u);
    }
    return Json(std::strtod(text.c_str(), nullptr));
  }
  std::string string() {
    if (s[i] != '"') fail("expected a string");
    ++i;
    std::string out;
    while (i < s.size() && s[i] != '"') {
      char c = s[i++];
      if (c == '\\') {
        if (i >= s.size()) fail("bad escape");
        char e = s[i++];
        switch (e) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'r': out += '\r'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'u': {
            if (i + 4 > s.size()) fail("bad unicode escape");
            unsigned code = (unsigned)std::strtoul(s.substr(i, 4).c_str(), nullptr, 16);
            i += 4;
            if (code < 0x80) out += (char)code;
            else if (code < 0x800) { out += (char)(0xC0 | (code >> 6)); out += (char)(0x80 | (code & 0x3F)); }
            else {
              out += (char)(0xE0 | (code >> 12));
              out += (char)(0x80 | ((code >> 6) & 0x3F));
              out += (char)(0x80 | (code & 0x3F));
            }
            break;
          }
          default: out += e;
        }
      } else {
        out += c;
      }
    }
    if (i >= s.size()) fail("unterminated string");
    ++i;
    return out;
  }
  Json array() {
    ++i;
    Json out = Json::array();
    ws();
    if (i < s.size() && s[i] == ']') { ++i; return out; }
    for (;;) {
      out.push_back(value());
      ws();
      if (i < s.size() && s[i] == ',') { ++i; continue; }
      if (i < s.size() && s[i] == ']') { ++i; return out; }
      fail("expected , or ]");
    }
  }
  Json object() {
    ++i;
    Json out = Json::object();
    ws();
    if (i < s.size() && s[i] == '}') { ++i; return out; }
    for (;;) {
      ws();
      std::string key = string();
      ws();
      if (i >= s.size() || s[i] != ':') fail("expected :");
      ++i;
      out[key] = value();
      ws();
      if (i < s.size() && s[i] == ',') { ++i; continue; }
      if (i < s.size() && s[i] == '}') { ++i; return out; }
      fail("expected , or }");
    }
  }
};

void escape(const std::string& in, std::string& out) {
  out += '"';
  for (char c : in) {
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\n': out += "\\n"; break;
      case '\t': out += "\\t"; break;
      case '\r': out += "\\r"; break;
      default:
        if ((unsigned char)c < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof(buf), "\\u%04x", (unsigned char)c);
          out += buf;
        } else {
          out += c;
        }
    }
  }
  out += '"';
}

}  // namespace

Json Json::parse(const std::string& text) {
  Parser p(text);
  Json v = p.value();
  p.ws();
  if (p.i != text.size()) p.fail("trailing characters");
  return v;
}

Json& Json::operator[](const std::string& key) {
  if (type_ == Type::Null) type_ = Type::Object;
  expect(Type::Object);
  for (auto& kv : obj_) if (kv.first == key) return kv.second;
  obj_.emplace_back(key, Json());
  return obj_.back().second;
}

const Json& Json::at(const std::string& key) const {
  expect(Type::Object);
  for (auto& kv : obj_) if (kv.first == key) return kv.second;
  throw std::runtime_error("JSON object has no key '" + key + "'");
}

bool Json::contains(const std::string& key) const {
  if (type_ != Type::Object) return false;
  for (auto& kv : obj_) if (kv.first == key) return true;
  return false;
}

std::string format_float(float v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v > 0 ? "Infinity" : "-Infinity";
  char buf[40];
  std::snprintf(buf, sizeof(buf), "%.9g", (double)v);
  // Keep a float literal ("-0" would read back as the integer 0 and lose
  // the sign of zero).
  std::string out = buf;
  if (out.find_first_of(".eE") == std::string::npos) out += ".0";
  return out;
}

void Json::dump_to(std::string& out) const {
  switch (type_) {
    case Type::Null: out += "null"; break;
    case Type::Bool: out += bool_ ? "true" : "false"; break;
    case Type::Number: {
      if (is_int_) {
        out += std::to_string(int_);
      } else if (is_float_) {
        out += format_float((float)num_);
      } else if (std::isnan(num_)) {
        out += "NaN";
      } else if (std::isinf(num_)) {
        out += num_ > 0 ? "Infinity" : "-Infinity";
      } else {
        char buf[40];
        std::snprintf(buf, sizeof(buf), "%.17g", num_);
        out += buf;
      }
      break;
    }
    case Type::String: escape(str_, out); break;
    case Type::Array: {
      out += '[';
      for (size_t k = 0; k < arr_.size(); ++k) {
        if (k) out += ',';
        arr_[k].dump_to(out);
      }
      out += ']';
      break;
    }
    case Type::Object: {
      out += '{';
      for (size_t k = 0; k < obj_.size(); ++k) {
        if (k) out += ',';
        escape(obj_[k].first, out);
        out += ':';
        obj_[k].second.dump_to(out);
      }
      out += '}';
      break;
    }
  }
}

// ---------------------------------------------------------------------------
// UBJSON: integers as int8/int32/int64 ('i','l','L'), binary32 values as 'd',
// other numbers as 'D', strings 'S' with an integer length.
// ---------------------------------------------------------------------------
namespace {
void put_be(std::string& out, uint64_t v, int bytes) {
  for (int i = bytes - 1; i >= 0; --i) out += (char)((v >> (8 * i)) & 0xff);
}
void put_int(std::string& out, int64_t v) {
  if (v >= -128 && v <= 127) { out += 'i'; out += (char)(int8_t)v; }
  else if (v >= INT32_MIN && v <= INT32_MAX) { out += 'l'; put_be(out, (uint32_t)(int32_t)v, 4); }
  else { out += 'L'; put_be(out, (uint64_t)v, 8); }
}
void put_str(std::string& out, const std::string& s) {
  put_int(out, (int64_t)s.size());
  out += s;
}
struct UbjReader {
  const std::string& b;
  size_t i = 0;
  explicit UbjReader(const std::string& bytes) : b(bytes) {}
  [[noreturn]] void fail(const char* what) { throw std::runtime_error(std::string("invalid UBJSON: ") + what); }
  uint8_t byte() { if (i >= b.size()) fail("truncated"); return (uint8_t)b[i++]; }
  uint64_t be(int n) { uint64_t v = 0; for (int k = 0; k < n; ++k) v = (v << 8) | byte(); return v; }
  int64_t integer_of(char t) {
    switch (t) {
      case 'i': return (int8_t)byte();
      case 'U': return byte();
      case 'I': return (int16_t)be(2);
      case 'l': return (int32_t)be(4);
      case 'L': return (int64_t)be(8);
    }
    fail("expected an integer");
  }
  std::string str() { int64_t n = integer_of((char)byte()); std::string s = b.substr(i, (size_t)n); i += (size_t)n; return s; }
  Json value_of(char t) {
    switch (t) {
      case 'Z': return Json();
      case 'T': return Json(true);
      case 'F': return Json(false);
      case 'i': case 'U': case 'I': case 'l': case 'L': return Json(integer_of(t));
      case 'd': { uint32_t v = (uint32_t)be(4); float f; std::memcpy(&f, &v, 4); return Json(f); }
      case 'D': { uint64_t v = be(8); double d; std::memcpy(&d, &v, 8); return Json(d); }
      case 'S': return Json(str());
      case 'C': return Json(std::string(1, (char)byte()));
      case '[': return array();
      case '{': return object();
    }
    fail("unknown marker");
  }
  Json array() {
    Json out = Json::array();
    char type = 0;
    int64_t count = -1;
    if (i < b.size() && b[i] == '$') { ++i; type = (char)byte(); }
    if (i < b.size() && b[i] == '#') { ++i; count = integer_of((char)byte()); }
    if (count >= 0) {
      for (int64_t k = 0; k < count; ++k) out.push_back(value_of(type ? type : (char)byte()));
      return out;
    }
    for (;;) {
      char t = (char)byte();
      if (t == ']') return out;
      out.push_back(value_of(t));
    }
  }
  Json object() {
    Json out = Json::object();
    char type = 0;
    int64_t count = -1;
    if (i < b.size() && b[i] == '$') { ++i; type = (char)byte(); }
    if (i < b.size() && b[i] == '#') { ++i; count = integer_of((char)byte()); }
    for (int64_t k = 0; count < 0 || k < count; ++k) {
      if (count < 0 && i < b.size() && b[i] == '}') { ++i; return out; }
      std::string key = str();
      out[key] = value_of(type ? type : (char)byte());
    }
    return out;
  }
};
}  // namespace

void Json::ubj_to(std::string& out) const {
  switch (type_) {
    case Type::Null: out += 'Z'; break;
    case Type::Bool: out += bool_ ? 'T' : 'F'; break;
    case Type::Number:
      if (is_int_) put_int(out, int_);
      else if (is_float_) {
        float f = (float)num_;
        uint32_t v;
        std::memcpy(&v, &f, 4);
        out += 'd';
        put_be(out, v, 4);
      } else {
        uint64_t v;
        std::memcpy(&v, &num_, 8);
        out += 'D';
        put_be(out, v, 8);
      }
      break;
    case Type::String: out += 'S'; put_str(out, str_); break;
    case Type::Array:
      out += '[';
      for (auto const& v : arr_) v.ubj_to(out);
      out += ']';
      break;
    case Type::Object:
      out += '{';
      for (auto const& kv : obj_) { put_str(out, kv.first); kv.second.ubj_to(out); }
      out += '}';
      break;
  }
}

std::string Json::dump_ubj() const {
  std::string out;
  ubj_to(out);
  return out;
}

Json Json::parse_ubj(const std::string& bytes) {
  UbjReader r(bytes);
  return r.value_of((char)r.byte());
}

std::string Json::dump() const {
  std::string out;
  dump_to(out);
  return out;
}

}  // namespace mgb
