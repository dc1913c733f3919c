// json.cpp -- recursive-descent JSON reader (see json.hpp).
#include "json.hpp"

#include <cmath>
#include <cstdlib>
#include <limits>

namespace osm::json {

namespace {

constexpr int kMaxDepth = 64;

class Parser {
 public:
  explicit Parser(std::string_view text) : s_(text) {}

  Value document() {
    Value v = value(0);
    skip_ws();
    if (i_ != s_.size()) fail("trailing characters after the document");
    return v;
  }

 private:
  std::string_view s_;
  std::size_t i_ = 0;

  [[noreturn]] void fail(const std::string& what) const {
    throw JsonError("JSON parse error at byte " + std::to_string(i_) + ": " + what);
  }
  void skip_ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
  }
  char peek() const { return i_ < s_.size() ? s_[i_] : '\0'; }
  void expect_word(std::string_view w) {
    if (s_.substr(i_, w.size()) != w) fail("unexpected token");
    i_ += w.size();
  }

  Value value(int depth) {
    if (depth > kMaxDepth) fail("nesting deeper than 64");
    skip_ws();
    Value v;
    switch (peek()) {
      case '{': object(v, depth); break;
      case '[': array(v, depth); break;
      case '"':
        v.kind = Value::Kind::string;
        v.str = string();
        break;
      case 't':
        expect_word("true");
        v.kind = Value::Kind::boolean;
        v.b = true;
        break;
      case 'f':
        expect_word("false");
        v.kind = Value::Kind::boolean;
        break;
      case 'n': expect_word("null"); break;
      default: number(v); break;
    }
    return v;
  }

  void object(Value& v, int depth) {
    v.kind = Value::Kind::object;
    ++i_;  // '{'
    skip_ws();
    if (peek() == '}') {
      ++i_;
      return;
    }
    for (;;) {
      skip_ws();
      if (peek() != '"') fail("expected a string key");
      std::string key = string();
      skip_ws();
      if (peek() != ':') fail("expected ':'");
      ++i_;
      Value member = value(depth + 1);
      if (!v.members.emplace(std::move(key), std::move(member)).second) fail("duplicate key");
      skip_ws();
      if (peek() == ',') {
        ++i_;
        continue;
      }
      if (peek() == '}') {
        ++i_;
        return;
      }
      fail("expected ',' or '}'");
    }
  }

  void array(Value& v, int depth) {
    v.kind = Value::Kind::array;
    ++i_;  // '['
    skip_ws();
    if (peek() == ']') {
      ++i_;
      return;
    }
    for (;;) {
      v.items.push_back(value(depth + 1));
      skip_ws();
      if (peek() == ',') {
        ++i_;
        continue;
      }
      if (peek() == ']') {
        ++i_;
        return;
      }
      fail("expected ',' or ']'");
    }
  }

  unsigned hex4() {
    if (i_ + 4 > s_.size()) fail("short \\u escape");
    unsigned v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = s_[i_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= static_cast<unsigned>(c - '0');
      else if (c >= 'a' && c <= 'f') v |= static_cast<unsigned>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= static_cast<unsigned>(c - 'A' + 10);
      else fail("bad \\u escape");
    }
    return v;
  }

  static void utf8(std::string& out, unsigned cp) {
    if (cp < 0x80) {
      out += static_cast<char>(cp);
    } else if (cp < 0x800) {
      out += static_cast<char>(0xC0 | (cp >> 6));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += static_cast<char>(0xE0 | (cp >> 12));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
      out += static_cast<char>(0xF0 | (cp >> 18));
      out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    }
  }

  std::string string() {
    ++i_;  // '"'
    std::string out;
    for (;;) {
      if (i_ >= s_.size()) fail("unterminated string");
      const char c = s_[i_++];
      if (c == '"') return out;
      if (static_cast<unsigned char>(c) < 0x20) fail("control character in string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i_ >= s_.size()) fail("unterminated escape");
      const char e = s_[i_++];
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
          if (cp >= 0xD800 && cp <= 0xDBFF) {
            if (s_.substr(i_, 2) != "\\u") fail("unpaired surrogate");
            i_ += 2;
            const unsigned lo = hex4();
            if (lo < 0xDC00 || lo > 0xDFFF) fail("unpaired surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
            fail("unpaired surrogate");
          }
          utf8(out, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
  }

  void number(Value& v) {
    const std::size_t begin = i_;
    if (peek() == '-') ++i_;
    if (peek() == '0') {
      ++i_;
    } else if (peek() >= '1' && peek() <= '9') {
      while (peek() >= '0' && peek() <= '9') ++i_;
    } else {
      fail("unexpected character");
    }
    bool integral = true;
    if (peek() == '.') {
      integral = false;
      ++i_;
      if (!(peek() >= '0' && peek() <= '9')) fail("digit expected after '.'");
      while (peek() >= '0' && peek() <= '9') ++i_;
    }
    if (peek() == 'e' || peek() == 'E') {
      integral = false;
      ++i_;
      if (peek() == '+' || peek() == '-') ++i_;
      if (!(peek() >= '0' && peek() <= '9')) fail("digit expected in exponent");
      while (peek() >= '0' && peek() <= '9') ++i_;
    }
    const std::string text(s_.substr(begin, i_ - begin));
    v.kind = Value::Kind::number;
    v.num = std::strtod(text.c_str(), nullptr);
    v.integral = integral;
    v.negative = text[0] == '-';
    if (integral) {
      std::uint64_t mag = 0;
      for (std::size_t k = v.negative ? 1 : 0; k < text.size(); ++k) {
        const std::uint64_t d = static_cast<std::uint64_t>(text[k] - '0');
        if (mag > (std::numeric_limits<std::uint64_t>::max() - d) / 10U) {
          mag = std::numeric_limits<std::uint64_t>::max();
          break;
        }
        mag = mag * 10U + d;
      }
      v.u = mag;
    }
  }
};

}  // namespace

const Value& Value::at(std::string_view key) const {
  if (kind != Kind::object) throw JsonError("not an object where key '" + std::string(key) + "' was expected");
  const auto it = members.find(key);
  if (it == members.end()) throw JsonError("key '" + std::string(key) + "' not found");
  return it->second;
}

std::uint64_t Value::as_u64() const {
  if (kind != Kind::number) throw JsonError("type must be number");
  if (!integral || negative) {
    // A whole value written with a fraction or exponent is accepted, as a
    // number cast to an integer would be; negative or fractional is not.
    if (negative || num < 0.0 || std::floor(num) != num || num >= 18446744073709551616.0)
      throw JsonError("number is not an unsigned integer");
    return static_cast<std::uint64_t>(num);
  }
  if (u == std::numeric_limits<std::uint64_t>::max()) throw JsonError("number out of range");
  return u;
}

std::uint32_t Value::as_u32() const {
  const std::uint64_t v = as_u64();
  if (v > std::numeric_limits<std::uint32_t>::max()) throw JsonError("number out of range of uint32");
  return static_cast<std::uint32_t>(v);
}

const std::string& Value::as_string() const {
  if (kind != Kind::string) throw JsonError("type must be string");
  return str;
}

bool Value::as_bool() const {
  if (kind != Kind::boolean) throw JsonError("type must be boolean");
  return b;
}

Value parse(std::string_view text) { return Parser(text).document(); }

}  // namespace osm::json
