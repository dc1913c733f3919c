"""The selection's exp key against the host C library, bit for bit.

The reference ranks experts by std::exp(fl(L - m)) / S
(src/cpu/reference_ops.cpp:141-150). The device computes that exp with
orbi-streammoe_amd/csrc/device/libm_expf.h, a restatement of the host
libm's expf. Here the header itself, compiled with g++, is checked against
std::exp(float) of this host over every float <= 0 (2^31 inputs, -0 to -inf)
and the largest positive keys a selection can see (never: keys are <= 0, but
the boundary cases of the special-value branch are covered too).
"""

import os
import subprocess
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER_DIR = os.path.join(ROOT, "orbi-streammoe_amd", "csrc", "device")

PROGRAM = r"""
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>
#include "libm_expf.h"

static float from_bits(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
static uint32_t to_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

int main() {
  // Every non-positive float (sign bit set, exponent below all-ones) and -inf,
  // then the positive side up to the overflow threshold and +inf.
  struct Range { uint64_t lo, hi; };
  const Range ranges[] = {{0x80000000ull, 0xFF800001ull}, {0x00000000ull, 0x42B20000ull},
                          {0x7F800000ull, 0x7F800001ull}};
  const unsigned nt = std::thread::hardware_concurrency() ? std::thread::hardware_concurrency() : 8;
  unsigned long long total = 0, bad = 0;
  for (const Range& r : ranges) {
    std::vector<unsigned long long> miss(nt, 0), first(nt, ~0ull);
    std::vector<std::thread> th;
    for (unsigned i = 0; i < nt; ++i)
      th.emplace_back([&, i] {
        const uint64_t lo = r.lo + (r.hi - r.lo) * i / nt, hi = r.lo + (r.hi - r.lo) * (i + 1) / nt;
        for (uint64_t u = lo; u < hi; ++u) {
          const float x = from_bits(static_cast<uint32_t>(u));
          const float want = std::exp(x);
          if (to_bits(osm_libm_expf(x)) != to_bits(want)) {
            if (!miss[i]) first[i] = u;
            ++miss[i];
          }
        }
      });
    for (auto& t : th) t.join();
    for (unsigned i = 0; i < nt; ++i) {
      bad += miss[i];
      if (miss[i]) std::printf("first mismatch at 0x%08llx\n", first[i]);
    }
    total += r.hi - r.lo;
  }
  std::printf("checked %llu mismatches %llu\n", total, bad);
  return bad == 0 ? 0 : 1;
}
"""


def test_restated_expf_equals_host_libm_everywhere():
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "expf_check.cpp"), os.path.join(d, "expf_check")
        with open(src, "w") as f:
            f.write(PROGRAM)
        # The reference's own compile flags for its CPU path (-O2, no fast-math).
        subprocess.run(["g++", "-O2", "-std=c++20", "-I", HEADER_DIR, "-o", exe, src, "-lpthread"], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches 0" in out.stdout, out.stdout
