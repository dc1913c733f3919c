/*
 * osm_layout.h -- byte layout of one expert in HBM, shared by host C++ and
 * HIP device code (plain C, no runtime dependencies).
 *
 * An expert is one contiguous blob in the qpack section order the reference
 * writes for a cache slot (tests/vulkan_resident_expert_cache_test.cpp:138-162,
 * docs/OSM-39B-QPACK-EXPERT-GEOMETRY.md:35-74):
 *
 *   gate.weight  u32  [inter,  hidden/8]   8 nibbles per word, low nibble first
 *   gate.scales  meta [inter,  hidden/group]
 *   gate.biases  meta [inter,  hidden/group]
 *   up.weight / up.scales / up.biases        (same shapes as gate)
 *   down.weight  u32  [hidden, inter/8]
 *   down.scales  meta [hidden, inter/group]
 *   down.biases  meta [hidden, inter/group]
 *
 * meta is bf16, f16 or f32. With hidden 2048, inter 512, group 64 and bf16
 * metadata one expert is 1,769,472 bytes; with f32 metadata it is 1,966,080
 * bytes, the reference converter's expertStride. Keeping the qpack order
 * means a cache fill is one straight copy of the blob, with no repacking.
 */
#ifndef OSM_LAYOUT_H
#define OSM_LAYOUT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Callable from host code and from HIP kernels. */
#if defined(__HIP__)
#define OSM_HD __attribute__((host, device))
#else
#define OSM_HD
#endif

enum osm_meta_dtype {
  OSM_META_F32 = 0,
  OSM_META_F16 = 1,
  OSM_META_BF16 = 2
};

/* Router and shared-gate storage beyond the dtypes above: MLX affine 8-bit
 * (4 values per u32, low byte first) with f32 scale and bias per group,
 * held as one buffer [packed rows x D/4 words][scales rows x D/g][biases]. */
#define OSM_ROUTER_AFFINE_Q8 3u

/* Host view of one affine-q8 matrix [rows, cols]: what the router and
 * shared-gate pointers of a layer point at when their dtype is
 * OSM_ROUTER_AFFINE_Q8 (the checkpoint's MlxAffineModule at 8 bits). */
typedef struct osm_affine_q8 {
  const uint32_t* packed; /* [rows, cols/4], low byte first */
  const float* scales;    /* [rows, cols/group] */
  const float* biases;    /* [rows, cols/group] */
  uint32_t group;         /* group size: a multiple of 4 dividing cols */
} osm_affine_q8;

typedef struct osm_expert_geometry {
  uint32_t hidden;       /* model width D (gate/up input, down output) */
  uint32_t inter;        /* expert intermediate width I */
  uint32_t group;        /* affine quantisation group size */
  uint32_t meta_dtype;   /* enum osm_meta_dtype */
} osm_expert_geometry;

typedef struct osm_expert_offsets {
  size_t gate_q, gate_s, gate_b;
  size_t up_q, up_s, up_b;
  size_t down_q, down_s, down_b;
  size_t total;
} osm_expert_offsets;

static inline OSM_HD size_t osm_meta_bytes(uint32_t meta_dtype) {
  return meta_dtype == OSM_META_F32 ? 4u : 2u;
}

static inline OSM_HD osm_expert_offsets osm_expert_layout(osm_expert_geometry g) {
  osm_expert_offsets o;
  const size_t ms = osm_meta_bytes(g.meta_dtype);
  const size_t gu_q = (size_t)g.inter * g.hidden / 2u;          /* nibbles -> bytes */
  const size_t gu_m = (size_t)g.inter * (g.hidden / g.group) * ms;
  const size_t dn_q = (size_t)g.hidden * g.inter / 2u;
  const size_t dn_m = (size_t)g.hidden * (g.inter / g.group) * ms;
  o.gate_q = 0;
  o.gate_s = o.gate_q + gu_q;
  o.gate_b = o.gate_s + gu_m;
  o.up_q = o.gate_b + gu_m;
  o.up_s = o.up_q + gu_q;
  o.up_b = o.up_s + gu_m;
  o.down_q = o.up_b + gu_m;
  o.down_s = o.down_q + dn_q;
  o.down_b = o.down_s + dn_m;
  o.total = o.down_b + dn_m;
  return o;
}

/* The fused MoE kernels read 16-byte packed chunks (32 columns) that never
 * straddle a quantisation group, and every section must stay 16-byte
 * aligned: hidden and inter multiples of 32, group a multiple of 32 that
 * divides both. */
static inline OSM_HD int osm_geometry_fused_ok(osm_expert_geometry g) {
  return g.hidden > 0 && g.inter > 0 && g.group > 0 && g.hidden % 32u == 0 &&
         g.inter % 32u == 0 && g.group % 32u == 0 && g.hidden % g.group == 0 &&
         g.inter % g.group == 0 && g.hidden <= 8192u && g.inter <= 4096u &&
         g.meta_dtype <= OSM_META_BF16;
}

#ifdef __cplusplus
}
#endif

#endif /* OSM_LAYOUT_H */
