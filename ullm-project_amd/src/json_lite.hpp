// json_lite.hpp -- the JSON subset a safetensors header uses, host side.
//
// RFC 8259 values: objects, arrays, strings (all escapes, \u surrogate pairs
// decoded to UTF-8), integers, true/false/null.  Fractions and exponents are
// rejected: a safetensors header carries only integer shapes and offsets and
// string metadata.  Duplicate object keys are an error, as an ambiguous
// header must not load.  Nesting is bounded.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace ullm {
namespace json {

struct Value {
  enum Kind { kNull, kBool, kInt, kString, kArray, kObject } kind = kNull;
  bool b = false;
  bool negative = false;
  uint64_t u = 0;  // magnitude of an integer
  std::string s;
  std::vector<Value> a;
  std::map<std::string, Value> o;
};

class Parser {
 public:
  Parser(const char *p, std::size_t n) : p_(p), end_(p + n) {}

  Value parse_document() {
    ws();
    Value v = value(0);
    ws();
    if (p_ != end_) {
      fail("trailing characters after the JSON value");
    }
    return v;
  }

 private:
  [[noreturn]] void fail(const char *what) {
    throw std::runtime_error(std::string("header JSON: ") + what);
  }
  void ws() {
    while (p_ != end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) {
      ++p_;
    }
  }
  char peek() {
    if (p_ == end_) {
      fail("unexpected end");
    }
    return *p_;
  }
  void expect(const char *lit) {
    for (; *lit != '\0'; ++lit, ++p_) {
      if (p_ == end_ || *p_ != *lit) {
        fail("invalid literal");
      }
    }
  }

  Value value(int depth) {
    if (depth > 64) {
      fail("nesting too deep");
    }
    Value v;
    const char c = peek();
    if (c == '{') {
      v.kind = Value::kObject;
      ++p_;
      ws();
      if (peek() == '}') {
        ++p_;
        return v;
      }
      for (;;) {
        ws();
        if (peek() != '"') {
          fail("object key must be a string");
        }
        std::string key = string();
        ws();
        if (peek() != ':') {
          fail("expected ':'");
        }
        ++p_;
        ws();
        Value item = value(depth + 1);
        if (!v.o.emplace(std::move(key), std::move(item)).second) {
          fail("duplicate object key");
        }
        ws();
        if (peek() == ',') {
          ++p_;
          continue;
        }
        if (peek() == '}') {
          ++p_;
          return v;
        }
        fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = Value::kArray;
      ++p_;
      ws();
      if (peek() == ']') {
        ++p_;
        return v;
      }
      for (;;) {
        ws();
        v.a.push_back(value(depth + 1));
        ws();
        if (peek() == ',') {
          ++p_;
          continue;
        }
        if (peek() == ']') {
          ++p_;
          return v;
        }
        fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Value::kString;
      v.s = string();
      return v;
    }
    if (c == 't') {
      expect("true");
      v.kind = Value::kBool;
      v.b = true;
      return v;
    }
    if (c == 'f') {
      expect("false");
      v.kind = Value::kBool;
      return v;
    }
    if (c == 'n') {
      expect("null");
      return v;
    }
    if (c == '-' || (c >= '0' && c <= '9')) {
      v.kind = Value::kInt;
      if (c == '-') {
        v.negative = true;
        ++p_;
      }
      if (peek() < '0' || peek() > '9') {
        fail("invalid number");
      }
      if (peek() == '0' && p_ + 1 != end_ && p_[1] >= '0' && p_[1] <= '9') {
        fail("leading zero in a number");
      }
      while (p_ != end_ && *p_ >= '0' && *p_ <= '9') {
        const uint64_t d = uint64_t(*p_ - '0');
        if (v.u > (UINT64_MAX - d) / 10) {
          fail("integer out of range");
        }
        v.u = v.u * 10 + d;
        ++p_;
      }
      if (p_ != end_ && (*p_ == '.' || *p_ == 'e' || *p_ == 'E')) {
        fail("only integers are expected in a safetensors header");
      }
      return v;
    }
    fail("unexpected character");
  }

  static void put_utf8(std::string &out, uint32_t cp) {
    if (cp < 0x80) {
      out += char(cp);
    } else if (cp < 0x800) {
      out += char(0xc0 | (cp >> 6));
      out += char(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
      out += char(0xe0 | (cp >> 12));
      out += char(0x80 | ((cp >> 6) & 0x3f));
      out += char(0x80 | (cp & 0x3f));
    } else {
      out += char(0xf0 | (cp >> 18));
      out += char(0x80 | ((cp >> 12) & 0x3f));
      out += char(0x80 | ((cp >> 6) & 0x3f));
      out += char(0x80 | (cp & 0x3f));
    }
  }

  uint32_t hex4() {
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = peek();
      ++p_;
      v <<= 4;
      if (c >= '0' && c <= '9') {
        v |= uint32_t(c - '0');
      } else if (c >= 'a' && c <= 'f') {
        v |= uint32_t(c - 'a' + 10);
      } else if (c >= 'A' && c <= 'F') {
        v |= uint32_t(c - 'A' + 10);
      } else {
        fail("invalid \\u escape");
      }
    }
    return v;
  }

  std::string string() {
    ++p_;  // opening quote
    std::string out;
    for (;;) {
      const char c = peek();
      ++p_;
      if (c == '"') {
        return out;
      }
      if (static_cast<unsigned char>(c) < 0x20) {
        fail("control character in a string");
      }
      if (c != '\\') {
        out += c;
        continue;
      }
      const char e = peek();
      ++p_;
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
          uint32_t cp = hex4();
          if (cp >= 0xd800 && cp <= 0xdbff) {
            if (peek() != '\\') {
              fail("unpaired surrogate");
            }
            ++p_;
            if (peek() != 'u') {
              fail("unpaired surrogate");
            }
            ++p_;
            const uint32_t lo = hex4();
            if (lo < 0xdc00 || lo > 0xdfff) {
              fail("unpaired surrogate");
            }
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          } else if (cp >= 0xdc00 && cp <= 0xdfff) {
            fail("unpaired surrogate");
          }
          put_utf8(out, cp);
          break;
        }
        default: fail("invalid escape");
      }
    }
  }

  const char *p_;
  const char *end_;
};

// JSON string literal with the escapes a reader needs (quote, backslash,
// control characters); other bytes, UTF-8 included, pass through.
inline std::string quote(const std::string &s) {
  static const char kHex[] = "0123456789abcdef";
  std::string out = "\"";
  for (const unsigned char c : s) {
    if (c == '"' || c == '\\') {
      out += '\\';
      out += char(c);
    } else if (c < 0x20) {
      out += "\\u00";
      out += kHex[c >> 4];
      out += kHex[c & 15];
    } else {
      out += char(c);
    }
  }
  return out + "\"";
}

}  // namespace json
}  // namespace ullm
