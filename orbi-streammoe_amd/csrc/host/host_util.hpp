// host_util.hpp -- small helpers shared by the host translation units.
#pragma once

#include <cmath>
#include <cstddef>
#include <limits>
#include <span>
#include <string>

#include "../device/osm_device.h"

namespace osm {

inline void set_diag(std::string* target, std::string message) {
  if (target != nullptr) *target = std::move(message);
}

inline std::string hip_error(const char* what, int rc) {
  return std::string(what) + ": " + osmd_error_string(rc);
}

inline bool all_finite(std::span<const float> v) {
  for (float f : v)
    if (!std::isfinite(f)) return false;
  return true;
}

// a * b without overflow, or false.
inline bool mul_ok(std::size_t a, std::size_t b, std::size_t& out) {
  if (a != 0 && b > std::numeric_limits<std::size_t>::max() / a) return false;
  out = a * b;
  return true;
}

}  // namespace osm
