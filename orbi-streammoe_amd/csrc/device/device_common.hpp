// device_common.hpp -- helpers shared by the gfx950 kernels of libosm_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "osm_device.h"

namespace osmk {

constexpr int kWave = 64;

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
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}
// Sum over aligned groups of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float group_sum(float v, int width) {
  for (int m = width >> 1; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// ---- nibble dot products ---------------------------------------------------
// Sum over the 8 nibbles of `w` (low nibble first) times x[0..7]. The even
// and odd nibbles are split into bytes so each value converts with one
// byte-to-float instruction.
__device__ __forceinline__ float nib_dot8(uint32_t w, const float* x) {
  const uint32_t lo = w & 0x0F0F0F0Fu;
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
  float d = static_cast<float>(lo & 0xFFu) * x[0];
  d = fmaf(static_cast<float>(hi & 0xFFu), x[1], d);
  d = fmaf(static_cast<float>((lo >> 8) & 0xFFu), x[2], d);
  d = fmaf(static_cast<float>((hi >> 8) & 0xFFu), x[3], d);
  d = fmaf(static_cast<float>((lo >> 16) & 0xFFu), x[4], d);
  d = fmaf(static_cast<float>((hi >> 16) & 0xFFu), x[5], d);
  d = fmaf(static_cast<float>(lo >> 24), x[6], d);
  d = fmaf(static_cast<float>(hi >> 24), x[7], d);
  return d;
}

// 32 columns held by one 16-byte chunk.
__device__ __forceinline__ float nib_dot32(uint4 q, const float* x) {
  float d = nib_dot8(q.x, x);
  d += nib_dot8(q.y, x + 8);
  d += nib_dot8(q.z, x + 16);
  d += nib_dot8(q.w, x + 24);
  return d;
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
