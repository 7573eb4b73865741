// Small JSON reader for safetensors headers and checkpoint config files.
//
// Accepts RFC 8259 JSON (objects, arrays, strings with escapes and surrogate
// pairs, numbers, true/false/null) with a nesting limit of 128, and rejects
// trailing data other than whitespace.  Integers that fit an unsigned 64-bit
// value are kept exactly (safetensors data offsets exceed 2^53 in principle);
// every number also carries its double value.  Objects keep their members in
// order; lookups return the last member of a repeated key.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace exl3 {
namespace json {

enum class Kind { Null, Bool, Number, String, Array, Object };

struct Value {
  Kind kind = Kind::Null;
  bool b = false;
  double num = 0.0;
  bool is_uint = false;  // number is a non-negative integer that fits u64
  uint64_t u = 0;
  std::string str;
  std::vector<Value> arr;
  std::vector<std::pair<std::string, Value>> obj;

  bool is_object() const { return kind == Kind::Object; }
  bool is_array() const { return kind == Kind::Array; }
  bool is_string() const { return kind == Kind::String; }
  bool is_number() const { return kind == Kind::Number; }

  // Last member named `key`, or nullptr (also for non-objects).
  const Value* find(const std::string& key) const {
    if (kind != Kind::Object) return nullptr;
    for (size_t i = obj.size(); i-- > 0;)
      if (obj[i].first == key) return &obj[i].second;
    return nullptr;
  }
  bool string_equals(const char* s) const { return kind == Kind::String && str == s; }
};

class Parser {
 public:
  Parser(const char* data, size_t size) : p_(data), end_(data + size) {}

  // Parses one document; on failure returns false and sets error().
  bool parse(Value& out) {
    skip_ws();
    if (!value(out, 0)) return false;
    skip_ws();
    if (p_ != end_) return fail("trailing characters");
    return true;
  }
  const std::string& error() const { return err_; }

 private:
  static constexpr int kMaxDepth = 128;
  const char* p_;
  const char* end_;
  std::string err_;

  bool fail(const char* what) {
    if (err_.empty()) err_ = what;
    return false;
  }
  void skip_ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool literal(const char* word) {
    size_t n = strlen(word);
    if ((size_t)(end_ - p_) < n || memcmp(p_, word, n) != 0) return fail("expected value");
    p_ += n;
    return true;
  }

  bool value(Value& v, int depth) {
    if (p_ >= end_) return fail("EOF while parsing a value");
    switch (*p_) {
      case '{': return object(v, depth + 1);
      case '[': return array(v, depth + 1);
      case '"': v.kind = Kind::String; return string(v.str);
      case 't': v.kind = Kind::Bool; v.b = true; return literal("true");
      case 'f': v.kind = Kind::Bool; v.b = false; return literal("false");
      case 'n': v.kind = Kind::Null; return literal("null");
      default: return number(v);
    }
  }

  bool object(Value& v, int depth) {
    if (depth > kMaxDepth) return fail("recursion limit exceeded");
    v.kind = Kind::Object;
    ++p_;
    skip_ws();
    if (p_ < end_ && *p_ == '}') { ++p_; return true; }
    for (;;) {
      skip_ws();
      if (p_ >= end_ || *p_ != '"') return fail("key must be a string");
      std::string key;
      if (!string(key)) return false;
      skip_ws();
      if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
      ++p_;
      skip_ws();
      v.obj.emplace_back(std::move(key), Value());
      if (!value(v.obj.back().second, depth)) return false;
      skip_ws();
      if (p_ < end_ && *p_ == ',') { ++p_; continue; }
      if (p_ < end_ && *p_ == '}') { ++p_; return true; }
      return fail("expected ',' or '}'");
    }
  }

  bool array(Value& v, int depth) {
    if (depth > kMaxDepth) return fail("recursion limit exceeded");
    v.kind = Kind::Array;
    ++p_;
    skip_ws();
    if (p_ < end_ && *p_ == ']') { ++p_; return true; }
    for (;;) {
      skip_ws();
      v.arr.emplace_back();
      if (!value(v.arr.back(), depth)) return false;
      skip_ws();
      if (p_ < end_ && *p_ == ',') { ++p_; continue; }
      if (p_ < end_ && *p_ == ']') { ++p_; return true; }
      return fail("expected ',' or ']'");
    }
  }

  static void put_utf8(std::string& s, uint32_t c) {
    if (c < 0x80) {
      s += (char)c;
    } else if (c < 0x800) {
      s += (char)(0xC0 | (c >> 6));
      s += (char)(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      s += (char)(0xE0 | (c >> 12));
      s += (char)(0x80 | ((c >> 6) & 0x3F));
      s += (char)(0x80 | (c & 0x3F));
    } else {
      s += (char)(0xF0 | (c >> 18));
      s += (char)(0x80 | ((c >> 12) & 0x3F));
      s += (char)(0x80 | ((c >> 6) & 0x3F));
      s += (char)(0x80 | (c & 0x3F));
    }
  }

  bool hex4(uint32_t& c) {
    if (end_ - p_ < 4) return fail("EOF in escape");
    c = 0;
    for (int i = 0; i < 4; ++i) {
      char h = *p_++;
      c <<= 4;
      if (h >= '0' && h <= '9') c |= (uint32_t)(h - '0');
      else if (h >= 'a' && h <= 'f') c |= (uint32_t)(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') c |= (uint32_t)(h - 'A' + 10);
      else return fail("invalid escape");
    }
    return true;
  }

  // Length of the UTF-8 sequence starting at p (0 if invalid).
  size_t utf8_len(const unsigned char* p) const {
    const unsigned char* e = (const unsigned char*)end_;
    unsigned char c = p[0];
    size_t n;
    uint32_t cp;
    if (c < 0x80) return 1;
    if ((c & 0xE0) == 0xC0) { n = 2; cp = c & 0x1F; }
    else if ((c & 0xF0) == 0xE0) { n = 3; cp = c & 0x0F; }
    else if ((c & 0xF8) == 0xF0) { n = 4; cp = c & 0x07; }
    else return 0;
    if ((size_t)(e - p) < n) return 0;
    for (size_t i = 1; i < n; ++i) {
      if ((p[i] & 0xC0) != 0x80) return 0;
      cp = (cp << 6) | (p[i] & 0x3F);
    }
    static const uint32_t kMin[5] = {0, 0, 0x80, 0x800, 0x10000};
    if (cp < kMin[n] || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return 0;
    return n;
  }

  bool string(std::string& s) {
    ++p_;  // opening quote
    for (;;) {
      if (p_ >= end_) return fail("EOF while parsing a string");
      unsigned char c = (unsigned char)*p_;
      if (c == '"') { ++p_; return true; }
      if (c < 0x20) return fail("control character in string");
      if (c == '\\') {
        ++p_;
        if (p_ >= end_) return fail("EOF in escape");
        char e = *p_++;
        switch (e) {
          case '"': s += '"'; break;
          case '\\': s += '\\'; break;
          case '/': s += '/'; break;
          case 'b': s += '\b'; break;
          case 'f': s += '\f'; break;
          case 'n': s += '\n'; break;
          case 'r': s += '\r'; break;
          case 't': s += '\t'; break;
          case 'u': {
            uint32_t c1;
            if (!hex4(c1)) return false;
            if (c1 >= 0xDC00 && c1 <= 0xDFFF) return fail("lone trailing surrogate");
            if (c1 >= 0xD800 && c1 <= 0xDBFF) {
              uint32_t c2;
              if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone leading surrogate");
              p_ += 2;
              if (!hex4(c2)) return false;
              if (c2 < 0xDC00 || c2 > 0xDFFF) return fail("invalid surrogate pair");
              c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
            }
            put_utf8(s, c1);
            break;
          }
          default: return fail("invalid escape");
        }
        continue;
      }
      size_t n = utf8_len((const unsigned char*)p_);
      if (n == 0) return fail("invalid UTF-8");
      s.append(p_, n);
      p_ += n;
    }
  }

  bool number(Value& v) {
    const char* start = p_;
    bool neg = false, integral = true;
    if (p_ < end_ && *p_ == '-') { neg = true; ++p_; }
    if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("expected value");
    if (*p_ == '0') {
      ++p_;
    } else {
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && *p_ == '.') {
      integral = false;
      ++p_;
      if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("invalid number");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      integral = false;
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("invalid number");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    std::string text(start, p_);
    v.kind = Kind::Number;
    v.num = strtod(text.c_str(), nullptr);
    v.is_uint = false;
    if (integral && !neg) {
      uint64_t u = 0;
      bool fits = true;
      for (char c : text) {
        uint64_t d = (uint64_t)(c - '0');
        if (u > (UINT64_MAX - d) / 10) { fits = false; break; }
        u = u * 10 + d;
      }
      v.is_uint = fits;
      v.u = fits ? u : 0;
    }
    return true;
  }
};

// Convenience: parse a whole buffer.
inline bool parse(const char* data, size_t size, Value& out, std::string& error) {
  Parser p(data, size);
  if (!p.parse(out)) {
    error = p.error();
    return false;
  }
  return true;
}

}  // namespace json
}  // namespace exl3
