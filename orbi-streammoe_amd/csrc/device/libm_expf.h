/*
 * libm_expf.h -- exp of a float with the bits of the host C library's expf.
 *
 * The reference ranks experts by softmax probabilities whose numerators are
 * std::exp(fl(L - m)) of floats (src/cpu/reference_ops.cpp:141-145), i.e.
 * the host libm's expf. That function is not correctly rounded, so a device
 * exp that is (or that is merely accurate) can order two probabilities
 * differently in the last bit. This is a restatement of the host's method:
 * the table-driven expf of ARM's optimized-routines (Szabolcs Nagy, 2017),
 * which glibc has used since 2.27:
 *
 *   x * 32/ln2 = k + r, |r| <= 1/2, k rounded to nearest by the 1.5 * 2^52
 *   shift; exp(x) = 2^(k/32) * 2^(r/32); 2^(k/32) is a table entry of
 *   2^(i/32) (i = k mod 32, each rounded to the nearest double, stored minus
 *   i << 47 so that adding k << 47 puts k/32's integer part in the exponent);
 *   2^(r/32) ~= 1 + c2 r + c1 r^2 + c0 r^3, evaluated in double, then
 *   rounded once to float.
 *
 * x86-64 glibc dispatches to a build of that code with FMA contraction: the
 * reduction, the polynomial's two linear terms and its r^2 term are fused
 * multiply-adds. The fused form is written out here with explicit FMAs, so
 * the arithmetic is the same on the host compiler and on gfx950 (IEEE double
 * FMA, multiply and add, one double-to-float rounding). The table entries
 * are the correctly rounded doubles of 2^(i/32) (recomputed from the
 * definition when the table was written).
 *
 * Pinned against the host's expf over every float <= 0 (2^31 inputs): on the
 * CPU for this header compiled with g++, and on the GPU for the device's own
 * results (block checksums).
 */
#ifndef OSM_LIBM_EXPF_H
#define OSM_LIBM_EXPF_H

#include <stdint.h>

#if defined(__HIPCC__)
#define OSM_LIBM_HD __host__ __device__
#else
#define OSM_LIBM_HD
#endif

OSM_LIBM_HD inline float osm_libm_expf(float x) {
  constexpr uint64_t tab[32] = {
      0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
      0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
      0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
      0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
      0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
      0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
      0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
      0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
  };
  // 32/ln2, the rounding shift, and the cubic's coefficients for r in units
  // of 1/32 (the minimax coefficients of 2^t - 1 scaled by 32^-3, 32^-2, 32^-1).
  constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
  constexpr double kShift = 0x1.8p+52;
  constexpr double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
  constexpr double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
  constexpr double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;

  const uint32_t ux = __builtin_bit_cast(uint32_t, x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {                            // |x| >= 88 or NaN
    if (ux == 0xff800000u) return 0.0f;              // -inf
    if (abstop >= 0x7f8u) return x + x;              // NaN, +inf
    if (x > 0x1.62e42ep6f) return __builtin_inff();  // above log(2^128)
    if (x < -0x1.9fe368p6f) return 0.0f;             // below log(2^-150)
  }
  const double xd = static_cast<double>(x);
  double kd = __builtin_fma(kInvLn2N, xd, kShift);
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  const uint64_t t = tab[ki % 32u] + (ki << 47);
  const double s = __builtin_bit_cast(double, t);
  const double z = __builtin_fma(c0, r, c1);
  const double r2 = r * r;
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return static_cast<float>(y);
}

#endif /* OSM_LIBM_EXPF_H */
