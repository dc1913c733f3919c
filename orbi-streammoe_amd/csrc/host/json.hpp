// json.hpp -- a small JSON reader for the qpack container's manifest.json and
// layout.json (the reference parses them with nlohmann/json v3.11.3,
// src/container/qpack.cpp:19-97). RFC 8259 text: objects, arrays, strings
// (with escapes, \u pairs to UTF-8), numbers, true, false, null. Malformed
// text, duplicate keys and nesting deeper than 64 throw JsonError with the
// byte offset.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace osm::json {

struct JsonError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

struct Value {
  enum class Kind { null, boolean, number, string, array, object };
  Kind kind = Kind::null;
  bool b = false;
  double num = 0.0;
  bool integral = false;   // the number was written without fraction or exponent
  bool negative = false;
  std::uint64_t u = 0;     // its magnitude when integral (saturated past 2^64 - 1)
  std::string str;
  std::vector<Value> items;
  std::map<std::string, Value, std::less<>> members;

  [[nodiscard]] bool is_object() const { return kind == Kind::object; }
  [[nodiscard]] bool is_array() const { return kind == Kind::array; }
  [[nodiscard]] bool is_null() const { return kind == Kind::null; }
  [[nodiscard]] bool contains(std::string_view key) const {
    return kind == Kind::object && members.find(key) != members.end();
  }
  // Member `key` of an object; throws JsonError when absent or not an object.
  [[nodiscard]] const Value& at(std::string_view key) const;
  // Typed reads; each throws JsonError on a kind or range mismatch.
  [[nodiscard]] std::uint64_t as_u64() const;
  [[nodiscard]] std::uint32_t as_u32() const;
  [[nodiscard]] const std::string& as_string() const;
  [[nodiscard]] bool as_bool() const;
};

[[nodiscard]] Value parse(std::string_view text);

}  // namespace osm::json
