// Minimal JSON reader for the engine's module configs (the reference's
// serialized `__config__` schema, src/inference_serialization.cpp:762-860).
// Supports objects, arrays, numbers, strings, true/false/null.
#pragma once

#include <cctype>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace mh {
namespace json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<Value> arr;
  std::map<std::string, Value> obj;

  bool has(const std::string &k) const { return kind == Object && obj.count(k); }
  const Value &at(const std::string &k) const {
    auto it = obj.find(k);
    if (kind != Object || it == obj.end()) throw std::runtime_error("config: missing key '" + k + "'");
    return it->second;
  }
  int as_int() const {
    if (kind == Bool) return b ? 1 : 0;
    if (kind != Number) throw std::runtime_error("config: expected a number");
    return int(num);
  }
  double as_num() const {
    if (kind != Number) throw std::runtime_error("config: expected a number");
    return num;
  }
  bool as_bool() const {
    if (kind == Number) return num != 0;
    if (kind != Bool) throw std::runtime_error("config: expected a boolean");
    return b;
  }
  const std::string &as_str() const {
    if (kind != String) throw std::runtime_error("config: expected a string");
    return str;
  }
  int get_int(const std::string &k, int def) const { return has(k) ? at(k).as_int() : def; }
  double get_num(const std::string &k, double def) const { return has(k) ? at(k).as_num() : def; }
  bool get_bool(const std::string &k, bool def) const { return has(k) ? at(k).as_bool() : def; }
  std::string get_str(const std::string &k, const std::string &def) const { return has(k) ? at(k).as_str() : def; }
};

class Parser {
 public:
  explicit Parser(const std::string &s) : s_(s) {}
  Value parse() {
    Value v = value();
    ws();
    if (i_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  const std::string &s_;
  size_t i_ = 0;
  [[noreturn]] void fail(const char *m) { throw std::runtime_error(std::string("config json: ") + m); }
  void ws() {
    while (i_ < s_.size() && std::isspace(static_cast<unsigned char>(s_[i_]))) ++i_;
  }
  bool lit(const char *t) {
    size_t n = std::char_traits<char>::length(t);
    if (s_.compare(i_, n, t) == 0) { i_ += n; return true; }
    return false;
  }
  Value value() {
    ws();
    if (i_ >= s_.size()) fail("unexpected end");
    const char c = s_[i_];
    Value v;
    if (c == '{') {
      v.kind = Value::Object;
      ++i_;
      ws();
      if (i_ < s_.size() && s_[i_] == '}') { ++i_; return v; }
      for (;;) {
        ws();
        Value k = value();
        if (k.kind != Value::String) fail("object key must be a string");
        ws();
        if (i_ >= s_.size() || s_[i_] != ':') fail("expected ':'");
        ++i_;
        v.obj[k.str] = value();
        ws();
        if (i_ < s_.size() && s_[i_] == ',') { ++i_; continue; }
        if (i_ < s_.size() && s_[i_] == '}') { ++i_; return v; }
        fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = Value::Array;
      ++i_;
      ws();
      if (i_ < s_.size() && s_[i_] == ']') { ++i_; return v; }
      for (;;) {
        v.arr.push_back(value());
        ws();
        if (i_ < s_.size() && s_[i_] == ',') { ++i_; continue; }
        if (i_ < s_.size() && s_[i_] == ']') { ++i_; return v; }
        fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Value::String;
      ++i_;
      while (i_ < s_.size() && s_[i_] != '"') {
        if (s_[i_] == '\\' && i_ + 1 < s_.size()) {
          ++i_;
          const char e = s_[i_];
          v.str += (e == 'n') ? '\n' : (e == 't') ? '\t' : e;
        } else {
          v.str += s_[i_];
        }
        ++i_;
      }
      if (i_ >= s_.size()) fail("unterminated string");
      ++i_;
      return v;
    }
    if (lit("true")) { v.kind = Value::Bool; v.b = true; return v; }
    if (lit("false")) { v.kind = Value::Bool; v.b = false; return v; }
    if (lit("null")) return v;
    char *end = nullptr;
    v.num = std::strtod(s_.c_str() + i_, &end);
    if (end == s_.c_str() + i_) fail("bad value");
    v.kind = Value::Number;
    i_ = size_t(end - s_.c_str());
    return v;
  }
};

inline Value parse(const std::string &s) { return Parser(s).parse(); }

}  // namespace json
}  // namespace mh
