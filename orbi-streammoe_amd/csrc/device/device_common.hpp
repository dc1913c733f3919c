// device_common.hpp -- helpers shared by the gfx950 kernels of libosm_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "libm_expf.h"
#include "osm_device.h"

namespace osmk {

constexpr int kWave = 64;

// ---- router GEMM bounds -----------------------------------------------------
// Per K range of the MFMA router GEMM, a logit's bound plane holds
// sum_i (32 (|s_{i-1}| + a_i) + |s_i|) + c(D) sum_i a_i over its 32-column
// steps i, s_i the fp32 running sum after step i (s_0 = 0) and a_i the step's
// |w_chunk| |x_chunk|: the reference's 32 partial sums within a step are at
// most 32 (|s_{i-1}| + a_i), adding a step sum errs by at most u |s_i|, and
// c(D) = 112 + D^2 u (u = 2^-24) covers the MFMAs' own rounding (66 u of the
// operands' absolute sum per step) and the reference's rounded products.
// The selection adds R |running sum at the start| for every range after the
// first and scales the total by (1 + 2^-9) u.
__device__ __forceinline__ float router_gemm_bound_coef(uint32_t hidden) {
  return 112.0f + static_cast<float>(hidden) * static_cast<float>(hidden) * 0x1p-24f;
}

// ---- metadata widening (bf16 -> f32 is a 16-bit shift, f16 -> f32 exact) --
__device__ __forceinline__ float bf16_to_f32(uint32_t bits) {
  return __uint_as_float(bits << 16);
}
__device__ __forceinline__ float f16_to_f32(uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

template <int META>
__device__ __forceinline__ float meta_at(const void* p, size_t i) {
  if constexpr (META == OSM_META_F32) {
    return static_cast<const float*>(p)[i];
  } else if constexpr (META == OSM_META_BF16) {
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else {
    return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
}

// ---- wavefront reductions (64 lanes) --------------------------------------
// Within a 16-lane row the steps are DPP moves (VALU latency, no LDS
// round trip): quad_perm [1,0,3,2] (xor 1), quad_perm [2,3,0,1] (xor 2),
// row_half_mirror (lane i <-> 7-i) and row_mirror (lane i <-> 15-i). Across
// rows, row_bcast:15 / row_bcast:31 fold rows into lane 63, which readlane
// then broadcasts as a wave-uniform value.
enum : int {
  kDppXor1 = 0xB1,
  kDppXor2 = 0x4E,
  kDppRowHalfMirror = 0x141,
  kDppRowMirror = 0x140,
  kDppRowBcast15 = 0x142,
  kDppRowBcast31 = 0x143,
};

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, v), CTRL,
                                                               ROW_MASK, 0xF, false));
}

// Sum over each aligned group of WIDTH lanes (WIDTH in {1,2,4,8,16}); every
// lane of the group holds the result.
template <int WIDTH>
__device__ __forceinline__ float row_sum(float v) {
  if constexpr (WIDTH >= 2) v += dpp<kDppXor1>(0.0f, v);
  if constexpr (WIDTH >= 4) v += dpp<kDppXor2>(0.0f, v);
  if constexpr (WIDTH >= 8) v += dpp<kDppRowHalfMirror>(0.0f, v);
  if constexpr (WIDTH >= 16) v += dpp<kDppRowMirror>(0.0f, v);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum<16>(v);
  v += dpp<kDppRowBcast15, 0xA>(0.0f, v);
  v += dpp<kDppRowBcast31, 0xC>(0.0f, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// DPP move of a double: both halves with the same control (0 where no
// source lane, or outside the row mask).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_d(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(u), CTRL, ROW_MASK, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(u >> 32), CTRL, ROW_MASK, 0xF, false);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                        static_cast<uint32_t>(lo));
}

__device__ __forceinline__ double wave_sum_d(double v) {
  v += dpp_d<kDppXor1>(v);
  v += dpp_d<kDppXor2>(v);
  v += dpp_d<kDppRowHalfMirror>(v);
  v += dpp_d<kDppRowMirror>(v);
  v += dpp_d<kDppRowBcast15, 0xA>(v);
  v += dpp_d<kDppRowBcast31, 0xC>(v);
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u), 63));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), 63));
  return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

// A float and a double summed over the wavefront, the two reductions
// interleaved; every lane gets both totals.
__device__ __forceinline__ void wave_sum_fd(float& f, double& d) {
  float a = f;
  double b = d;
  a += dpp<kDppXor1>(0.0f, a);
  b += dpp_d<kDppXor1>(b);
  a += dpp<kDppXor2>(0.0f, a);
  b += dpp_d<kDppXor2>(b);
  a += dpp<kDppRowHalfMirror>(0.0f, a);
  b += dpp_d<kDppRowHalfMirror>(b);
  a += dpp<kDppRowMirror>(0.0f, a);
  b += dpp_d<kDppRowMirror>(b);
  a += dpp<kDppRowBcast15, 0xA>(0.0f, a);
  b += dpp_d<kDppRowBcast15, 0xA>(b);
  a += dpp<kDppRowBcast31, 0xC>(0.0f, a);
  b += dpp_d<kDppRowBcast31, 0xC>(b);
  f = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 63));
  const uint64_t u = __builtin_bit_cast(uint64_t, b);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u), 63));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), 63));
  d = __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v, v));
  v = fmaxf(v, dpp<kDppXor2>(v, v));
  v = fmaxf(v, dpp<kDppRowHalfMirror>(v, v));
  v = fmaxf(v, dpp<kDppRowMirror>(v, v));
  v = fmaxf(v, dpp<kDppRowBcast15, 0xA>(v, v));
  v = fmaxf(v, dpp<kDppRowBcast31, 0xC>(v, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(old), static_cast<int>(v),
                                                           CTRL, ROW_MASK, 0xF, false));
}

// Unsigned max over the wavefront. 0 is the identity of the max, so each
// step can issue as a single v_max_u32 with a DPP source.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<kDppXor1>(0u, v));
  v = max(v, dpp_u32<kDppXor2>(0u, v));
  v = max(v, dpp_u32<kDppRowHalfMirror>(0u, v));
  v = max(v, dpp_u32<kDppRowMirror>(0u, v));
  v = max(v, dpp_u32<kDppRowBcast15, 0xA>(0u, v));
  v = max(v, dpp_u32<kDppRowBcast31, 0xC>(0u, v));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// Inclusive prefix sum over the 64 lanes in lane order. row_shr 1, 2 and 3
// (lanes without a source add 0) give each lane the sum of up to four lanes
// ending at it, row_shr 4 and 8 extend that to the start of its 16-lane row,
// and row_bcast 15 / 31 add the totals of the rows before it.
__device__ __forceinline__ float wave_incl_scan(float v) {
  float s = v + dpp<0x111>(0.0f, v);
  s += dpp<0x112>(0.0f, v);
  s += dpp<0x113>(0.0f, v);
  s += dpp<0x114>(0.0f, s);
  s += dpp<0x118>(0.0f, s);
  s += dpp<kDppRowBcast15, 0xA>(0.0f, s);
  s += dpp<kDppRowBcast31, 0xC>(0.0f, s);
  return s;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Float bits as an unsigned key that orders like the value (-0 below +0).
__device__ __forceinline__ uint32_t ordered_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float group_sum(float v, int width) {
  for (int m = width >> 1; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// ---- nibble dot products ---------------------------------------------------
// A nibble q masked into the low bits of a 16-bit lane is the f16 subnormal
// q * 2^-24, exactly. `w & 0x000F000F` therefore holds nibbles 0 and 4 of
// `w` as an f16 pair, `(w >> 4) & 0x000F000F` nibbles 1 and 5, and so on, and
// v_fma_mix_f32 multiplies either half by an fp32 x and accumulates in fp32.
// Every product and partial sum is the plain fp32 one times 2^-24 (a power of
// two, with fp32 and f16 denormals preserved), so scaling the sum by 2^24
// gives the same bits as converting each nibble to float whenever no product
// falls below 2^-102: about 14 VALU instructions per 8 nibbles instead of 21.
__device__ __forceinline__ float f16_lo(uint32_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v & 0xFFFFu)));
}
__device__ __forceinline__ float f16_hi(uint32_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v >> 16)));
}

// A zero the compiler cannot see through: seeding a chain with it keeps the
// first product a v_fma_mix_f32 instead of a convert and a multiply. The
// seeded chain differs from one started with the product only in the sign of
// an exactly-zero result.
__device__ __forceinline__ float opaque_zero() {
  float z = 0.0f;
  asm("" : "+v"(z));
  return z;
}

// z + 2^-24 * sum over the 8 nibbles of `w` (low nibble first) times
// x[0..7], accumulated in nibble order.
__device__ __forceinline__ float nib_dot8_s24(uint32_t w, const float* x, float z) {
  const uint32_t p0 = w & 0x000F000Fu;
  const uint32_t p1 = (w >> 4) & 0x000F000Fu;
  const uint32_t p2 = (w >> 8) & 0x000F000Fu;
  const uint32_t p3 = (w >> 12) & 0x000F000Fu;
  float d = fmaf(f16_lo(p0), x[0], z);
  d = fmaf(f16_lo(p1), x[1], d);
  d = fmaf(f16_lo(p2), x[2], d);
  d = fmaf(f16_lo(p3), x[3], d);
  d = fmaf(f16_hi(p0), x[4], d);
  d = fmaf(f16_hi(p1), x[5], d);
  d = fmaf(f16_hi(p2), x[6], d);
  d = fmaf(f16_hi(p3), x[7], d);
  return d;
}

constexpr float kTwo24 = 16777216.0f;

// Sum over the 8 nibbles of `w` times x[0..7].
__device__ __forceinline__ float nib_dot8(uint32_t w, const float* x) {
  return nib_dot8_s24(w, x, opaque_zero()) * kTwo24;
}

// 32 columns held by one 16-byte chunk, in two chains. Masking a word in
// place with 0x00F000F0 leaves nibbles 1 and 5 as the f16 subnormals q * 2^-20
// (bits 4-7 of each half), so with w and w >> 8 every nibble is one AND away
// from an f16: five instructions per word unpack eight nibbles, against seven
// when each nibble is shifted down first. Chain a holds the 2^-24 products
// (nibbles 0, 4, 2, 6 of each word), chain b the 2^-20 ones (1, 5, 3, 7);
// each is the plain fp32 chain times its power of two, and the two are
// scaled back and added once.
constexpr float kTwo20 = 1048576.0f;

__device__ __forceinline__ float nib_dot32(uint4 q, const float* x) {
  float a = opaque_zero(), b = opaque_zero();
  const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = w4[i], t = w >> 8;
    const float* xi = x + 8 * i;
    const uint32_t p0 = w & 0x000F000Fu;  // nibbles 0, 4
    const uint32_t p1 = w & 0x00F000F0u;  // nibbles 1, 5 (times 16)
    const uint32_t p2 = t & 0x000F000Fu;  // nibbles 2, 6
    const uint32_t p3 = t & 0x00F000F0u;  // nibbles 3, 7 (times 16)
    a = fmaf(f16_lo(p0), xi[0], a);
    b = fmaf(f16_lo(p1), xi[1], b);
    a = fmaf(f16_lo(p2), xi[2], a);
    b = fmaf(f16_lo(p3), xi[3], b);
    a = fmaf(f16_hi(p0), xi[4], a);
    b = fmaf(f16_hi(p1), xi[5], b);
    a = fmaf(f16_hi(p2), xi[6], a);
    b = fmaf(f16_hi(p3), xi[7], b);
  }
  return fmaf(b, kTwo20, a * kTwo24);
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  // silu(g) = g * sigmoid(g), sigmoid(v) = 1 / (1 + exp(-v))
  // (reference_ops.cpp:214-220).
  const float sig = 1.0f / (1.0f + expf(-g));
  return g * sig * u;
}

// Loads through the global address space. Pointers read from memory (expert
// tables) are generic to the compiler, which would otherwise emit flat loads.
template <typename T>
__device__ __forceinline__ T ldg(const void* p) {
  return *reinterpret_cast<const __attribute__((address_space(1))) T*>(
      reinterpret_cast<uintptr_t>(p));
}
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldg16(const void* p) {
  const u32x4 v = ldg<u32x4>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 ldg8(const void* p) {
  const u32x2 v = ldg<u32x2>(p);
  return make_uint2(v.x, v.y);
}

// Raw metadata bits (bf16/f16 in the low 16 bits, or f32 bits) and their
// widening, split so a load can be issued long before its value is needed.
template <int META>
__device__ __forceinline__ uint32_t meta_bits(const void* p, size_t i) {
  if constexpr (META == OSM_META_F32) {
    return ldg<uint32_t>(static_cast<const uint32_t*>(p) + i);
  } else {
    return ldg<uint16_t>(static_cast<const uint16_t*>(p) + i);
  }
}
template <int META>
__device__ __forceinline__ float meta_widen(uint32_t bits) {
  if constexpr (META == OSM_META_F32) {
    return __uint_as_float(bits);
  } else if constexpr (META == OSM_META_BF16) {
    return bf16_to_f32(bits);
  } else {
    return f16_to_f32(bits);
  }
}

inline int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : static_cast<int>(e);
}

}  // namespace osmk
