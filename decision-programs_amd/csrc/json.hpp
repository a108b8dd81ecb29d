// Minimal JSON reader/writer for array interfaces, parameters and models.
// Accepts the bare NaN / Infinity / -Infinity tokens that XGBoost's text
// format and the reference's DMatrix config ({"missing":NaN}) use
// (native/class_native_training.cuh:51, native/class_native_model_json.hpp:14).
#pragma once

#include <charconv>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <limits>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

#include "dp_internal.hpp"

namespace dp::json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object };
  Kind kind = Null;
  bool boolean = false;
  std::string text;  // number token or string contents
  std::vector<Value> items;
  std::vector<std::pair<std::string, Value>> members;

  const Value* find(std::string_view key) const {
    for (const auto& m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
  const Value& at(std::string_view key) const {
    const Value* v = find(key);
    need(v != nullptr, "missing JSON key: " + std::string(key));
    return *v;
  }
  double number() const {
    need(kind == Number, "JSON value is not a number");
    if (text == "NaN") return std::numeric_limits<double>::quiet_NaN();
    if (text == "Infinity" || text == "+Infinity") return std::numeric_limits<double>::infinity();
    if (text == "-Infinity") return -std::numeric_limits<double>::infinity();
    return std::strtod(text.c_str(), nullptr);
  }
  uint64_t u64() const {
    need(kind == Number, "JSON value is not an integer");
    uint64_t v = 0;
    auto r = std::from_chars(text.data(), text.data() + text.size(), v);
    need(r.ec == std::errc() && r.ptr == text.data() + text.size(),
         "JSON value is not a non-negative integer: " + text);
    return v;
  }
  int64_t i64() const {
    need(kind == Number, "JSON value is not an integer");
    int64_t v = 0;
    auto r = std::from_chars(text.data(), text.data() + text.size(), v);
    need(r.ec == std::errc() && r.ptr == text.data() + text.size(),
         "JSON value is not an integer: " + text);
    return v;
  }
};

class Parser {
 public:
  explicit Parser(std::string_view s) : s_(s) {}
  Value parse() {
    Value v = value();
    ws();
    need(i_ == s_.size(), "trailing characters after JSON value");
    return v;
  }

 private:
  std::string_view s_;
  size_t i_ = 0;
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
  }
  bool lit(std::string_view w) {
    if (s_.substr(i_, w.size()) == w) { i_ += w.size(); return true; }
    return false;
  }
  // Objects and arrays nest at most this deep: the descent is recursive, so a
  // hostile '[[[[...' document is refused before it exhausts the host stack.
  static constexpr int kMaxDepth = 512;
  int depth_ = 0;
  struct Nest {
    int& d;
    explicit Nest(int& depth) : d(depth) {
      need(++d <= kMaxDepth, "JSON nesting deeper than " + std::to_string(kMaxDepth) + " levels");
    }
    ~Nest() { --d; }
  };
  Value value() {
    ws();
    need(i_ < s_.size(), "unexpected end of JSON");
    Value v;
    const char c = s_[i_];
    if (c == '{' || c == '[') {
      Nest nest(depth_);
      return container(c);
    }
    if (c == '"') {
      v.kind = Value::String;
      v.text = string();
      return v;
    }
    return scalar();
  }
  Value container(char c) {
    Value v;
    if (c == '{') {
      v.kind = Value::Object;
      ++i_;
      ws();
      if (i_ < s_.size() && s_[i_] == '}') { ++i_; return v; }
      for (;;) {
        ws();
        need(i_ < s_.size() && s_[i_] == '"', "expected JSON object key");
        std::string key = string();
        ws();
        need(i_ < s_.size() && s_[i_] == ':', "expected ':' in JSON object");
        ++i_;
        v.members.emplace_back(std::move(key), value());
        ws();
        need(i_ < s_.size(), "unterminated JSON object");
        if (s_[i_] == ',') { ++i_; continue; }
        need(s_[i_] == '}', "expected ',' or '}' in JSON object");
        ++i_;
        return v;
      }
    }
    if (c == '[') {
      v.kind = Value::Array;
      ++i_;
      ws();
      if (i_ < s_.size() && s_[i_] == ']') { ++i_; return v; }
      for (;;) {
        v.items.push_back(value());
        ws();
        need(i_ < s_.size(), "unterminated JSON array");
        if (s_[i_] == ',') { ++i_; continue; }
        need(s_[i_] == ']', "expected ',' or ']' in JSON array");
        ++i_;
        return v;
      }
    }
    return v;
  }
  Value scalar() {
    Value v;
    if (lit("true")) { v.kind = Value::Bool; v.boolean = true; return v; }
    if (lit("false")) { v.kind = Value::Bool; v.boolean = false; return v; }
    if (lit("null")) return v;
    for (std::string_view w : {"NaN", "Infinity", "+Infinity", "-Infinity"})
      if (lit(w)) { v.kind = Value::Number; v.text = std::string(w); return v; }
    const size_t b = i_;
    if (i_ < s_.size() && (s_[i_] == '-' || s_[i_] == '+')) ++i_;
    while (i_ < s_.size() && (std::isdigit(static_cast<unsigned char>(s_[i_])) || s_[i_] == '.' ||
                              s_[i_] == 'e' || s_[i_] == 'E' || s_[i_] == '-' || s_[i_] == '+'))
      ++i_;
    need(i_ > b, "invalid JSON token");
    v.kind = Value::Number;
    v.text = std::string(s_.substr(b, i_ - b));
    return v;
  }
  std::string string() {
    ++i_;  // opening quote
    std::string out;
    while (i_ < s_.size() && s_[i_] != '"') {
      char c = s_[i_++];
      if (c == '\\') {
        need(i_ < s_.size(), "bad JSON escape");
        char e = s_[i_++];
        switch (e) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'r': out += '\r'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'u': {
            need(i_ + 4 <= s_.size(), "bad JSON unicode escape");
            unsigned code = std::stoul(std::string(s_.substr(i_, 4)), nullptr, 16);
            i_ += 4;
            if (code < 0x80) out += char(code);
            else if (code < 0x800) { out += char(0xC0 | (code >> 6)); out += char(0x80 | (code & 0x3F)); }
            else { out += char(0xE0 | (code >> 12)); out += char(0x80 | ((code >> 6) & 0x3F)); out += char(0x80 | (code & 0x3F)); }
            break;
          }
          default: out += e;
        }
      } else {
        out += c;
      }
    }
    need(i_ < s_.size(), "unterminated JSON string");
    ++i_;
    return out;
  }
};

inline Value parse(std::string_view s) { return Parser(s).parse(); }

// ---- writing ------------------------------------------------------------
inline void put_string(std::string& o, std::string_view s) {
  o += '"';
  for (char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\n': o += "\\n"; break;
      case '\t': o += "\\t"; break;
      case '\r': o += "\\r"; break;
      default:
        if (static_cast<unsigned char>(c) < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof buf, "\\u%04x", c);
          o += buf;
        } else {
          o += c;
        }
    }
  }
  o += '"';
}

// Shortest decimal text that reads back as the same float; non-finite values
// use XGBoost's bare tokens.
inline void put_float(std::string& o, float x) {
  if (std::isnan(x)) { o += "NaN"; return; }
  if (std::isinf(x)) { o += x > 0 ? "Infinity" : "-Infinity"; return; }
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof buf, x);
  o.append(buf, r.ptr);
}

inline void put_double(std::string& o, double x) {
  if (std::isnan(x)) { o += "NaN"; return; }
  if (std::isinf(x)) { o += x > 0 ? "Infinity" : "-Infinity"; return; }
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof buf, x);
  o.append(buf, r.ptr);
}

template <class T>
inline void put_int_array(std::string& o, const std::vector<T>& v) {
  o += '[';
  for (size_t i = 0; i < v.size(); ++i) {
    if (i) o += ',';
    o += std::to_string(v[i]);
  }
  o += ']';
}

inline void put_float_array(std::string& o, const std::vector<float>& v) {
  o += '[';
  for (size_t i = 0; i < v.size(); ++i) {
    if (i) o += ',';
    put_float(o, v[i]);
  }
  o += ']';
}

// Text of a parsed (or built) value: compact when indent < 0, else one
// member / item per line indented by `indent` spaces per level.  Number
// tokens are written as they were read.
inline void dump_to(std::string& o, const Value& v, int indent, int level = 0) {
  auto newline = [&](int lvl) {
    if (indent < 0) return;
    o += '\n';
    o.append(size_t(indent) * size_t(lvl), ' ');
  };
  switch (v.kind) {
    case Value::Null: o += "null"; break;
    case Value::Bool: o += v.boolean ? "true" : "false"; break;
    case Value::Number: o += v.text; break;
    case Value::String: put_string(o, v.text); break;
    case Value::Array:
      if (v.items.empty()) { o += "[]"; break; }
      o += '[';
      for (size_t i = 0; i < v.items.size(); ++i) {
        if (i) o += ',';
        newline(level + 1);
        dump_to(o, v.items[i], indent, level + 1);
      }
      newline(level);
      o += ']';
      break;
    case Value::Object:
      if (v.members.empty()) { o += "{}"; break; }
      o += '{';
      for (size_t i = 0; i < v.members.size(); ++i) {
        if (i) o += ',';
        newline(level + 1);
        put_string(o, v.members[i].first);
        o += indent < 0 ? ":" : ": ";
        dump_to(o, v.members[i].second, indent, level + 1);
      }
      newline(level);
      o += '}';
      break;
  }
}

inline std::string dump(const Value& v, int indent = -1) {
  std::string o;
  dump_to(o, v, indent);
  return o;
}

// Builders for values written by the host tools.
inline Value null_value() { return Value{}; }
inline Value boolean(bool b) {
  Value v;
  v.kind = Value::Bool;
  v.boolean = b;
  return v;
}
inline Value string(std::string s) {
  Value v;
  v.kind = Value::String;
  v.text = std::move(s);
  return v;
}
inline Value number(double x) {
  Value v;
  v.kind = Value::Number;
  put_double(v.text, x);
  return v;
}
inline Value integer(int64_t x) {
  Value v;
  v.kind = Value::Number;
  v.text = std::to_string(x);
  return v;
}
inline Value object() {
  Value v;
  v.kind = Value::Object;
  return v;
}
inline Value array() {
  Value v;
  v.kind = Value::Array;
  return v;
}
// Sets (replacing) member `key` of object `o`.
inline void set(Value& o, const std::string& key, Value value) {
  for (auto& m : o.members)
    if (m.first == key) {
      m.second = std::move(value);
      return;
    }
  o.members.emplace_back(key, std::move(value));
}

}  // namespace dp::json
