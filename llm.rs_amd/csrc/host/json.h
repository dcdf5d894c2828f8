// json.h - the small JSON reader the weight loaders need (config.json,
// safetensors headers and shard indexes): objects, arrays, strings (with
// escapes; \u outside ASCII becomes UTF-8), numbers, booleans and null.
#pragma once
#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace llmrs {
namespace json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<Value> arr;
  std::map<std::string, Value> obj;

  bool has(const std::string& k) const { return kind == Object && obj.count(k) != 0; }
  const Value& at(const std::string& k) const {
    auto it = obj.find(k);
    if (kind != Object || it == obj.end()) throw std::runtime_error("JSON: missing key \"" + k + "\"");
    return it->second;
  }
  double number() const {
    if (kind != Number) throw std::runtime_error("JSON: expected a number");
    return num;
  }
  const std::string& string() const {
    if (kind != String) throw std::runtime_error("JSON: expected a string");
    return str;
  }
};

class Parser {
 public:
  Parser(const char* p, size_t n) : p_(p), end_(p + n) {}
  Value parse() {
    Value v = value();
    ws();
    if (p_ != end_) fail("trailing characters");
    return v;
  }

 private:
  const char* p_;
  const char* end_;

  [[noreturn]] void fail(const char* what) { throw std::runtime_error(std::string("JSON: ") + what); }
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool eat(char c) {
    ws();
    if (p_ < end_ && *p_ == c) {
      ++p_;
      return true;
    }
    return false;
  }
  void expect(char c) {
    if (!eat(c)) fail("unexpected character");
  }
  bool word(const char* w) {
    size_t n = 0;
    while (w[n]) ++n;
    if ((size_t)(end_ - p_) >= n && std::string(p_, n) == w) {
      p_ += n;
      return true;
    }
    return false;
  }
  static void utf8(std::string& out, unsigned cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += (char)(0xE0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    } else {
      out += (char)(0xF0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3F));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    }
  }
  unsigned hex4() {
    if (end_ - p_ < 4) fail("short \\u escape");
    unsigned v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
      else fail("bad \\u escape");
    }
    return v;
  }
  std::string string_body() {
    std::string out;
    while (true) {
      if (p_ >= end_) fail("unterminated string");
      const char c = *p_++;
      if (c == '"') return out;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (p_ >= end_) fail("unterminated escape");
      const char e = *p_++;
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
          unsigned cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
            p_ += 2;
            const unsigned lo = hex4();
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(out, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
  }
  // Nesting deeper than this is refused (a crafted header cannot exhaust
  // the host stack); configs and safetensors headers nest two levels.
  static constexpr int kMaxDepth = 64;

  Value value(int depth = 0) {
    ws();
    if (p_ >= end_) fail("unexpected end");
    if (depth >= kMaxDepth) fail("nesting too deep");
    Value v;
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v.kind = Value::Object;
      if (eat('}')) return v;
      do {
        expect('"');
        std::string k = string_body();
        expect(':');
        v.obj[k] = value(depth + 1);
      } while (eat(','));
      expect('}');
    } else if (c == '[') {
      ++p_;
      v.kind = Value::Array;
      if (eat(']')) return v;
      do v.arr.push_back(value(depth + 1));
      while (eat(','));
      expect(']');
    } else if (c == '"') {
      ++p_;
      v.kind = Value::String;
      v.str = string_body();
    } else if (word("true")) {
      v.kind = Value::Bool;
      v.b = true;
    } else if (word("false")) {
      v.kind = Value::Bool;
    } else if (word("null")) {
      v.kind = Value::Null;
    } else {
      char* stop = nullptr;
      const std::string tok(p_, (size_t)std::min<ptrdiff_t>(end_ - p_, 64));
      v.num = std::strtod(tok.c_str(), &stop);
      if (stop == tok.c_str()) fail("bad value");
      p_ += stop - tok.c_str();
      v.kind = Value::Number;
    }
    return v;
  }
};

inline Value parse(const char* p, size_t n) { return Parser(p, n).parse(); }
inline Value parse(const std::string& s) { return parse(s.data(), s.size()); }

}  // namespace json
}  // namespace llmrs
