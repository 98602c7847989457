// Minimal JSON reader for config.json and safetensors headers (no external dependencies).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace q3t {
namespace json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<Value> arr;
  std::map<std::string, Value> obj;

  const Value &at(const std::string &key) const {
    if (kind != Object) throw std::runtime_error("json: not an object when reading '" + key + "'");
    auto it = obj.find(key);
    if (it == obj.end()) throw std::runtime_error("json: missing key '" + key + "'");
    return it->second;
  }
  bool has(const std::string &key) const { return kind == Object && obj.count(key) != 0; }
  double number() const {
    if (kind != Number) throw std::runtime_error("json: expected a number");
    return num;
  }
  // An integral number within +-2^53 (exact in a double); anything else is an error, so a
  // crafted header cannot reach an out-of-range conversion.
  int64_t integer() const {
    const double x = number();
    if (!(x >= -9007199254740992.0 && x <= 9007199254740992.0) || x != (double)(int64_t)x)
      throw std::runtime_error("json: expected an integer");
    return (int64_t)x;
  }
};

class Parser {
 public:
  // Nesting deeper than this is rejected: value() -> object() / array() recurse, so an
  // unbounded depth would let a crafted header overflow the host stack.
  static constexpr int kMaxDepth = 64;

  explicit Parser(const std::string &text) : s_(text) {}
  Value parse() {
    Value v = value();
    ws();
    if (i_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  const std::string &s_;
  size_t i_ = 0;
  int depth_ = 0;

  // Counts one level of object / array nesting for the lifetime of the guard.
  struct Nest {
    Parser &p;
    explicit Nest(Parser &parser) : p(parser) {
      if (++p.depth_ > kMaxDepth) p.fail("nesting too deep");
    }
    ~Nest() { --p.depth_; }
  };

  [[noreturn]] void fail(const char *what) {
    throw std::runtime_error(std::string("json: ") + what + " at offset " + std::to_string(i_));
  }
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
  }
  char peek() {
    ws();
    if (i_ >= s_.size()) fail("unexpected end");
    return s_[i_];
  }
  void expect(char c) {
    if (peek() != c) fail("unexpected character");
    ++i_;
  }
  Value value() {
    const char c = peek();
    if (c == '{') return object();
    if (c == '[') return array();
    if (c == '"') {
      Value v;
      v.kind = Value::String;
      v.str = string();
      return v;
    }
    if (s_.compare(i_, 4, "true") == 0) {
      i_ += 4;
      Value v;
      v.kind = Value::Bool;
      v.b = true;
      return v;
    }
    if (s_.compare(i_, 5, "false") == 0) {
      i_ += 5;
      Value v;
      v.kind = Value::Bool;
      return v;
    }
    if (s_.compare(i_, 4, "null") == 0) {
      i_ += 4;
      return Value();
    }
    return number();
  }
  Value object() {
    Nest nest(*this);
    Value v;
    v.kind = Value::Object;
    expect('{');
    if (peek() == '}') {
      ++i_;
      return v;
    }
    while (true) {
      if (peek() != '"') fail("expected key");
      std::string key = string();
      expect(':');
      v.obj[key] = value();
      const char c = peek();
      ++i_;
      if (c == '}') break;
      if (c != ',') fail("expected , or }");
    }
    return v;
  }
  Value array() {
    Nest nest(*this);
    Value v;
    v.kind = Value::Array;
    expect('[');
    if (peek() == ']') {
      ++i_;
      return v;
    }
    while (true) {
      v.arr.push_back(value());
      const char c = peek();
      ++i_;
      if (c == ']') break;
      if (c != ',') fail("expected , or ]");
    }
    return v;
  }
  std::string string() {
    expect('"');
    std::string out;
    while (i_ < s_.size() && s_[i_] != '"') {
      char c = s_[i_++];
      if (c == '\\') {
        if (i_ >= s_.size()) fail("bad escape");
        const char e = s_[i_++];
        switch (e) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'r': out += '\r'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'u': {
            if (i_ + 4 > s_.size()) fail("bad \\u escape");
            const unsigned cp = (unsigned)std::stoul(s_.substr(i_, 4), nullptr, 16);
            i_ += 4;
            if (cp < 0x80) {
              out += (char)cp;
            } else if (cp < 0x800) {
              out += (char)(0xC0 | (cp >> 6));
              out += (char)(0x80 | (cp & 0x3F));
            } else {
              out += (char)(0xE0 | (cp >> 12));
              out += (char)(0x80 | ((cp >> 6) & 0x3F));
              out += (char)(0x80 | (cp & 0x3F));
            }
            break;
          }
          default: out += e;
        }
      } else {
        out += c;
      }
    }
    if (i_ >= s_.size()) fail("unterminated string");
    ++i_;
    return out;
  }
  Value number() {
    const size_t start = i_;
    if (i_ < s_.size() && (s_[i_] == '-' || s_[i_] == '+')) ++i_;
    while (i_ < s_.size() && (isdigit((unsigned char)s_[i_]) || s_[i_] == '.' || s_[i_] == 'e' ||
                              s_[i_] == 'E' || s_[i_] == '-' || s_[i_] == '+'))
      ++i_;
    if (start == i_) fail("expected a value");
    Value v;
    v.kind = Value::Number;
    v.num = std::stod(s_.substr(start, i_ - start));
    return v;
  }
};

inline Value parse(const std::string &text) { return Parser(text).parse(); }

}  // namespace json
}  // namespace q3t
