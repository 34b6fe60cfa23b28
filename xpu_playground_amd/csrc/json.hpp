// Minimal strict JSON reader for config.json, model.safetensors.index.json
// and safetensors headers (the reference hand-writes one too,
// qwen3/model.cpp:16-215). Numbers are kept as double and as their source
// text so integer fields can be checked exactly.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace xpu::json {

struct Value {
  enum class Kind { Null, Bool, Number, String, Array, Object } kind = Kind::Null;
  bool boolean = false;
  double number = 0;
  std::string text;  // string value, or the literal text of a number
  std::vector<Value> array;
  std::map<std::string, Value> object;

  const Value &at(const std::string &key) const {
    if (kind != Kind::Object) throw std::runtime_error("JSON value is not an object (looking for '" + key + "')");
    auto it = object.find(key);
    if (it == object.end()) throw std::runtime_error("missing JSON field '" + key + "'");
    return it->second;
  }
  const Value *find(const std::string &key) const {
    if (kind != Kind::Object) return nullptr;
    auto it = object.find(key);
    return it == object.end() ? nullptr : &it->second;
  }
  // exact unsigned integer (no fraction or exponent in the source text)
  uint64_t as_u64(const std::string &what) const {
    if (kind != Kind::Number || text.empty() || text.find_first_not_of("0123456789") != std::string::npos)
      throw std::runtime_error(what + " must be an unsigned integer");
    return std::strtoull(text.c_str(), nullptr, 10);
  }
};

class Parser {
 public:
  explicit Parser(const std::string &s) : s_(s) {}
  Value parse() {
    Value v = value();
    ws();
    if (i_ != s_.size()) fail("trailing content");
    return v;
  }

 private:
  [[noreturn]] void fail(const std::string &m) const {
    throw std::runtime_error("invalid JSON at byte " + std::to_string(i_) + ": " + m);
  }
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
  }
  char peek() {
    if (i_ >= s_.size()) fail("unexpected end");
    return s_[i_];
  }
  bool take(const char *lit) {
    size_t n = 0;
    while (lit[n]) ++n;
    if (s_.compare(i_, n, lit) != 0) return false;
    i_ += n;
    return true;
  }
  Value value() {
    ws();
    Value v;
    const char c = peek();
    if (c == '{') return object();
    if (c == '[') return array();
    if (c == '"') {
      v.kind = Value::Kind::String;
      v.text = string();
      return v;
    }
    if (take("true")) { v.kind = Value::Kind::Bool; v.boolean = true; return v; }
    if (take("false")) { v.kind = Value::Kind::Bool; return v; }
    if (take("null")) return v;
    return number();
  }
  Value number() {
    const size_t b = i_;
    if (s_[i_] == '-') ++i_;
    while (i_ < s_.size() && ((s_[i_] >= '0' && s_[i_] <= '9') || s_[i_] == '.' || s_[i_] == 'e' ||
                              s_[i_] == 'E' || s_[i_] == '+' || s_[i_] == '-'))
      ++i_;
    if (b == i_) fail("expected a value");
    Value v;
    v.kind = Value::Kind::Number;
    v.text = s_.substr(b, i_ - b);
    char *end = nullptr;
    v.number = std::strtod(v.text.c_str(), &end);
    if (end != v.text.c_str() + v.text.size()) fail("invalid number");
    return v;
  }
  std::string string() {
    if (s_[i_] != '"') fail("expected string");
    ++i_;
    std::string out;
    while (true) {
      const char c = peek();
      ++i_;
      if (c == '"') return out;
      if (static_cast<unsigned char>(c) < 0x20) fail("control character in string");
      if (c != '\\') { out += c; continue; }
      const char e = peek();
      ++i_;
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          if (i_ + 4 > s_.size()) fail("short unicode escape");
          const unsigned code = static_cast<unsigned>(std::stoul(s_.substr(i_, 4), nullptr, 16));
          i_ += 4;
          if (code < 0x80) out += static_cast<char>(code);
          else if (code < 0x800) {
            out += static_cast<char>(0xc0 | (code >> 6));
            out += static_cast<char>(0x80 | (code & 0x3f));
          } else {
            out += static_cast<char>(0xe0 | (code >> 12));
            out += static_cast<char>(0x80 | ((code >> 6) & 0x3f));
            out += static_cast<char>(0x80 | (code & 0x3f));
          }
          break;
        }
        default: fail("invalid escape");
      }
    }
  }
  Value array() {
    ++i_;
    Value v;
    v.kind = Value::Kind::Array;
    ws();
    if (peek() == ']') { ++i_; return v; }
    while (true) {
      v.array.push_back(value());
      ws();
      const char c = peek();
      ++i_;
      if (c == ']') return v;
      if (c != ',') fail("expected , or ]");
    }
  }
  Value object() {
    ++i_;
    Value v;
    v.kind = Value::Kind::Object;
    ws();
    if (peek() == '}') { ++i_; return v; }
    while (true) {
      ws();
      std::string key = string();
      ws();
      if (peek() != ':') fail("expected :");
      ++i_;
      if (!v.object.emplace(key, value()).second) fail("duplicate key " + key);
      ws();
      const char c = peek();
      ++i_;
      if (c == '}') return v;
      if (c != ',') fail("expected , or }");
    }
  }
  const std::string &s_;
  size_t i_ = 0;
};

inline Value parse(const std::string &text) { return Parser(text).parse(); }

}  // namespace xpu::json
