// Strict JSON reader for the three documents the checkpoint loader reads:
// config.json, model.safetensors.index.json and each safetensors header.
//
// The text is parsed once into a flat tape: one entry per value in document
// order, a container's children directly after it, and each entry records
// where its subtree ends, so walking an object or array is a skip along the
// tape and no value owns heap nodes. Strings are unescaped into one shared
// buffer; numbers keep their source lexeme so integer fields can be read
// exactly (digits only, overflow rejected) rather than through a double.
#pragma once

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

namespace xpu::json {

enum class Type : uint8_t { Null, True, False, Number, String, Array, Object };

class Document;

// A view of one value of a Document (valid while the Document lives).
class Node {
public:
  Node() = default;
  Node(const Document *doc, uint32_t at) : doc_(doc), at_(at) {}

  explicit operator bool() const { return doc_ != nullptr; }
  Type type() const;
  bool is(Type t) const { return doc_ && type() == t; }
  bool is_bool() const { return is(Type::True) || is(Type::False); }
  bool truth() const { return is(Type::True); }

  std::string_view string() const;  // String values
  double number() const;            // Number values
  // Number written as a plain unsigned integer (no sign, fraction or
  // exponent) that fits 64 bits; false otherwise.
  bool exact_u64(uint64_t &out) const;

  size_t size() const;                         // Array elements or Object members
  Node element(size_t i) const;                // i-th Array element (i < size())
  Node member(std::string_view key) const;     // empty Node when absent or not an Object
  // calls f(key, value) for every Object member in document order
  template <typename F> void each_member(F &&f) const;
  template <typename F> void each_element(F &&f) const;

private:
  const Document *doc_ = nullptr;
  uint32_t at_ = 0;
};

class Document {
public:
  // source names the document in error messages
  Document(std::string_view text, std::string source) : source_(std::move(source)) { Parser(*this, text).run(); }
  Node root() const { return Node(this, 0); }
  const std::string &source() const { return source_; }

private:
  friend class Node;
  struct Entry {
    Type type;
    uint32_t end;    // tape index just past this value's subtree
    uint32_t count;  // Array elements / Object members
    uint32_t off;    // String: offset into text_; Number: offset of the lexeme
    uint32_t len;
    double value;    // Number
  };
  std::vector<Entry> tape_;
  std::string text_;  // unescaped strings and number lexemes, back to back
  std::string source_;

  class Parser {
  public:
    Parser(Document &d, std::string_view in) : d_(d), in_(in) {}

    void run() {
      // explicit stack of open containers: tape index of each
      std::vector<uint32_t> open;
      skip_space();
      parse_value(open);
      while (!open.empty()) {
        Entry &c = d_.tape_[open.back()];
        skip_space();
        const char close = c.type == Type::Array ? ']' : '}';
        if (peek() == close) {
          ++pos_;
          c.end = static_cast<uint32_t>(d_.tape_.size());
          if (c.type == Type::Object) unique_names(open.back());
          open.pop_back();
          continue;
        }
        if (c.count) {
          expect(',', c.type == Type::Array ? "',' or ']' in an array" : "',' or '}' in an object");
          skip_space();
        }
        ++c.count;
        if (c.type == Type::Object) {
          if (peek() != '"') fail("a member name (string)");
          parse_string();
          skip_space();
          expect(':', "':' after a member name");
          skip_space();
        }
        parse_value(open);
      }
      skip_space();
      if (pos_ != in_.size()) fail("end of document");
    }

  private:
    Document &d_;
    std::string_view in_;
    size_t pos_ = 0;

    [[noreturn]] void fail(const char *wanted) const {
      std::string got = pos_ < in_.size() ? std::string("'") + in_[pos_] + "'" : std::string("end of input");
      throw std::runtime_error(d_.source_ + ": malformed JSON at offset " + std::to_string(pos_) + ": expected " +
                               wanted + ", found " + got);
    }
    char peek() const { return pos_ < in_.size() ? in_[pos_] : '\0'; }
    void expect(char c, const char *wanted) {
      if (peek() != c) fail(wanted);
      ++pos_;
    }
    void skip_space() {
      while (pos_ < in_.size() && (in_[pos_] == ' ' || in_[pos_] == '\t' || in_[pos_] == '\n' || in_[pos_] == '\r'))
        ++pos_;
    }
    // An object whose member names repeat is rejected, as the reference's
    // reader does (qwen3/model.cpp:204-205): the names are sorted and
    // compared neighbour to neighbour once the object is closed.
    void unique_names(uint32_t object) const {
      std::vector<std::string_view> names;
      names.reserve(d_.tape_[object].count);
      const uint32_t end = d_.tape_[object].end;
      for (uint32_t k = object + 1; k < end; k = d_.tape_[k + 1].end)
        names.push_back(std::string_view(d_.text_).substr(d_.tape_[k].off, d_.tape_[k].len));
      std::sort(names.begin(), names.end());
      for (size_t i = 1; i < names.size(); ++i)
        if (names[i] == names[i - 1])
          throw std::runtime_error(d_.source_ + ": malformed JSON: duplicate object key \"" +
                                   std::string(names[i]) + "\" in the object that ends at offset " +
                                   std::to_string(pos_ - 1));
    }

    uint32_t push(Type t) {
      if (d_.tape_.size() >= 0xfffffff0u) fail("a smaller document");
      d_.tape_.push_back(Entry{t, static_cast<uint32_t>(d_.tape_.size() + 1), 0, 0, 0, 0.0});
      return static_cast<uint32_t>(d_.tape_.size() - 1);
    }

    // scalars get their whole entry; containers are left open on the stack
    void parse_value(std::vector<uint32_t> &open) {
      const char c = peek();
      if (c == '{' || c == '[') {
        ++pos_;
        if (open.size() >= 256) fail("nesting of at most 256 levels");
        open.push_back(push(c == '{' ? Type::Object : Type::Array));
      } else if (c == '"') {
        parse_string();
      } else if (c == '-' || (c >= '0' && c <= '9')) {
        parse_number();
      } else if (!literal("true", Type::True) && !literal("false", Type::False) && !literal("null", Type::Null)) {
        fail("a value");
      }
    }

    bool literal(std::string_view word, Type t) {
      if (in_.substr(pos_, word.size()) != word) return false;
      pos_ += word.size();
      push(t);
      return true;
    }

    void parse_number() {
      const size_t start = pos_;
      auto digits = [&] {
        const size_t from = pos_;
        while (peek() >= '0' && peek() <= '9') ++pos_;
        return pos_ - from;
      };
      if (peek() == '-') ++pos_;
      if (peek() == '0') ++pos_;
      else if (!digits()) fail("a digit");
      if (peek() == '.') {
        ++pos_;
        if (!digits()) fail("a digit after '.'");
      }
      if (peek() == 'e' || peek() == 'E') {
        ++pos_;
        if (peek() == '+' || peek() == '-') ++pos_;
        if (!digits()) fail("an exponent digit");
      }
      const uint32_t e = push(Type::Number);
      Entry &n = d_.tape_[e];
      n.off = static_cast<uint32_t>(d_.text_.size());
      n.len = static_cast<uint32_t>(pos_ - start);
      d_.text_.append(in_.substr(start, pos_ - start));
      n.value = std::strtod(d_.text_.c_str() + n.off, nullptr);
    }

    unsigned hex4() {
      unsigned v = 0;
      for (int i = 0; i < 4; ++i, ++pos_) {
        const char c = peek();
        const int d = c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10 : c >= 'A' && c <= 'F' ? c - 'A' + 10 : -1;
        if (d < 0) fail("four hex digits after \\u");
        v = v * 16 + static_cast<unsigned>(d);
      }
      return v;
    }

    // code point -> UTF-8: the lead byte carries the length, each
    // continuation byte 6 bits
    void put_utf8(uint32_t cp) {
      if (cp < 0x80) {
        d_.text_.push_back(static_cast<char>(cp));
        return;
      }
      const int tail = cp < 0x800 ? 1 : cp < 0x10000 ? 2 : 3;
      static const unsigned char lead[] = {0, 0xc0, 0xe0, 0xf0};
      d_.text_.push_back(static_cast<char>(lead[tail] | (cp >> (6 * tail))));
      for (int i = tail - 1; i >= 0; --i) d_.text_.push_back(static_cast<char>(0x80 | ((cp >> (6 * i)) & 0x3f)));
    }

    void parse_string() {
      ++pos_;  // opening quote
      const uint32_t e = push(Type::String);
      const size_t off = d_.text_.size();
      for (;;) {
        if (pos_ >= in_.size()) fail("a closing '\"'");
        const char c = in_[pos_++];
        if (c == '"') break;
        if (static_cast<unsigned char>(c) < 0x20) {
          --pos_;
          fail("no raw control character inside a string");
        }
        if (c != '\\') {
          d_.text_.push_back(c);
          continue;
        }
        const char esc = peek();
        ++pos_;
        static constexpr std::string_view from = "\"\\/bfnrt", to = "\"\\/\b\f\n\r\t";
        if (const size_t k = from.find(esc); esc && k != std::string_view::npos) {
          d_.text_.push_back(to[k]);
        } else if (esc == 'u') {
          uint32_t cp = hex4();
          if (cp >= 0xd800 && cp < 0xdc00 && in_.substr(pos_, 2) == "\\u") {  // surrogate pair
            pos_ += 2;
            const uint32_t low = hex4();
            if (low < 0xdc00 || low >= 0xe000) fail("a low surrogate");
            cp = 0x10000 + ((cp - 0xd800) << 10) + (low - 0xdc00);
          }
          put_utf8(cp);
        } else {
          --pos_;
          fail("a valid escape character");
        }
      }
      d_.tape_[e].off = static_cast<uint32_t>(off);
      d_.tape_[e].len = static_cast<uint32_t>(d_.text_.size() - off);
    }
  };
};

inline Type Node::type() const { return doc_->tape_[at_].type; }

inline std::string_view Node::string() const {
  const auto &e = doc_->tape_[at_];
  return e.type == Type::String ? std::string_view(doc_->text_).substr(e.off, e.len) : std::string_view();
}

inline double Node::number() const {
  const auto &e = doc_->tape_[at_];
  return e.type == Type::Number ? e.value : 0.0;
}

inline bool Node::exact_u64(uint64_t &out) const {
  if (!is(Type::Number)) return false;
  const auto &e = doc_->tape_[at_];
  const std::string_view lex = std::string_view(doc_->text_).substr(e.off, e.len);
  uint64_t v = 0;
  for (const char c : lex) {
    if (c < '0' || c > '9') return false;
    const uint64_t d = static_cast<uint64_t>(c - '0');
    if (v > (UINT64_MAX - d) / 10) return false;
    v = v * 10 + d;
  }
  out = v;
  return true;
}

inline size_t Node::size() const {
  const auto &e = doc_->tape_[at_];
  return e.type == Type::Array || e.type == Type::Object ? e.count : 0;
}

template <typename F> void Node::each_element(F &&f) const {
  if (!is(Type::Array)) return;
  const uint32_t end = doc_->tape_[at_].end;
  for (uint32_t i = at_ + 1; i < end; i = doc_->tape_[i].end) f(Node(doc_, i));
}

inline Node Node::element(size_t i) const {
  Node found;
  size_t n = 0;
  each_element([&](Node v) {
    if (n++ == i) found = v;
  });
  return found;
}

template <typename F> void Node::each_member(F &&f) const {
  if (!is(Type::Object)) return;
  const uint32_t end = doc_->tape_[at_].end;
  for (uint32_t k = at_ + 1; k < end;) {
    const uint32_t v = k + 1;  // a member name is a one-entry String
    f(Node(doc_, k).string(), Node(doc_, v));
    k = doc_->tape_[v].end;
  }
}

inline Node Node::member(std::string_view key) const {
  Node found;
  each_member([&](std::string_view k, Node v) {
    if (!found && k == key) found = v;
  });
  return found;
}

}  // namespace xpu::json
