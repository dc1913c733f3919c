/*
 * osm_device.h -- the thin C ABI between the C++ host code and the HIP
 * device code of libosm_hip.so.
 *
 * Host translation units (csrc/host, csrc/capi.cpp) are plain C++20 and never
 * include HIP headers: every device allocation, copy, stream, event and
 * kernel launch goes through the functions below, which are implemented in
 * the .hip translation units. All functions return 0 on success or a HIP
 * error code; osmd_error_string() names it. Streams and events are opaque.
 */
#ifndef OSM_DEVICE_H
#define OSM_DEVICE_H

#include <stddef.h>
#include <stdint.h>

#include "../osm_layout.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef void* osmd_stream;
typedef void* osmd_event;
typedef void* osmd_graph; /* an instantiated, replayable graph */

const char* osmd_error_string(int code);

/* ---- runtime ------------------------------------------------------------ */
int osmd_device_count(int* count);
int osmd_set_device(int device);
int osmd_device_name(int device, char* buf, size_t n);
int osmd_device_mem_info(size_t* free_bytes, size_t* total_bytes);
int osmd_malloc(void** ptr, size_t bytes);
int osmd_free(void* ptr);
int osmd_host_malloc(void** ptr, size_t bytes); /* pinned */
int osmd_host_free(void* ptr);
int osmd_memcpy_h2d(void* dst, const void* src, size_t bytes, osmd_stream s);
int osmd_memcpy_d2h(void* dst, const void* src, size_t bytes, osmd_stream s);
int osmd_memcpy_d2d(void* dst, const void* src, size_t bytes, osmd_stream s);
/* Device-to-device copy with a kernel when dst, src and bytes are 16-byte
 * aligned (a kernel node when captured), else hipMemcpyAsync. */
int osmd_copy_d2d(void* dst, const void* src, size_t bytes, osmd_stream s);
/* Host-to-device copy by a kernel that reads pinned host memory (from
 * osmd_host_malloc) over PCIe itself, on a grid of at most `blocks`
 * workgroups; hipMemcpyAsync when dst, src or bytes is not 16-byte aligned. */
int osmd_copy_from_pinned(void* dst, const void* src, size_t bytes, unsigned blocks, osmd_stream s);
/* Zero-fill with a kernel (safe inside captured graphs). */
int osmd_zero(void* dst, size_t bytes, osmd_stream s);
int osmd_stream_create(osmd_stream* s);
int osmd_stream_destroy(osmd_stream s);
int osmd_stream_synchronize(osmd_stream s);
/* The device a stream was created on. */
int osmd_stream_device(osmd_stream s, int* device);
int osmd_event_create(osmd_event* e);
int osmd_event_destroy(osmd_event e);
int osmd_event_record(osmd_event e, osmd_stream s);
int osmd_event_synchronize(osmd_event e);
int osmd_stream_wait_event(osmd_stream s, osmd_event e);
int osmd_event_elapsed_ms(osmd_event start, osmd_event stop, float* ms);
int osmd_device_synchronize(void);
/* Block checksums of osm_libm_expf (the selection's exp) over float bit
 * patterns first .. first + count - 1: sums[b] = sum over block b's inputs i
 * (i from 0) of bits(exp(x)) * (2 i + 1) mod 2^64, ceil(count / block)
 * blocks, in device memory. */
int osmd_libm_expf_checksums(uint32_t first, uint64_t count, uint32_t block, uint64_t* sums, osmd_stream s);
/* The fixed workspace of the decode entry point that allocates nothing: a
 * file-scope device array of OSMD_STATIC_SCRATCH_BYTES, one copy per GPU,
 * held until the process ends. _init looks its address up on `device`,
 * which must be current (done at context creation); osmd_static_scratch
 * returns it (looking it up then if _init did not run or failed). */
#define OSMD_STATIC_SCRATCH_BYTES (4u << 20)
int osmd_static_scratch_init(int device);
int osmd_static_scratch(int device, void** out);
/* Records what is enqueued on s between begin and end (nothing runs), then
 * instantiates it. A failed launch inside still needs the end call, which
 * then returns its error and no graph. Capture must not record memset nodes:
 * buffers are cleared with osmd_zero. */
int osmd_capture_begin(osmd_stream s);
int osmd_capture_end(osmd_stream s, osmd_graph* out);
int osmd_graph_launch(osmd_graph g, osmd_stream s);
int osmd_graph_destroy(osmd_graph g);

/* ---- elementwise / projection kernels ----------------------------------- */
typedef struct osmd_q4_proj {
  const uint32_t* packed; /* [out_dim, packed_cols] */
  const void* scales;     /* [out_dim, groups] meta */
  const void* biases;     /* [out_dim, groups] meta */
  uint32_t out_dim;
  uint32_t packed_cols;
  uint32_t group;
  uint32_t meta_dtype;
} osmd_q4_proj;

int osmd_q4_dequant(const osmd_q4_proj* p, float* out, osmd_stream s);
int osmd_q4_gemv(const osmd_q4_proj* p, const float* x, float* y, osmd_stream s);
int osmd_unpack_nibbles(const uint32_t* packed, size_t words, uint8_t* out,
                        osmd_stream s);
int osmd_swiglu(const float* gate, const float* up, float* out, size_t n,
                osmd_stream s);
int osmd_weighted_accumulate(const float* src, float weight, float* acc,
                             size_t n, osmd_stream s);
int osmd_rms_norm(const float* in, const float* weight, float* out,
                  uint32_t rows, uint32_t dim, float eps, osmd_stream s);
/* Affine q4 quantizer (single_expert_pilot.cpp:276-358) of values [rows,
 * cols]: packed [rows, cols/8], scales/biases/bounds [rows, cols/group],
 * per-block error maximum and sum ([osmd_q4_quantize_blocks()] each), and
 * flags (zero on entry; bit 0 non-finite weight, bit 1 error above bound).
 * Geometry is checked by the caller. */
unsigned osmd_q4_quantize_blocks(size_t rows, size_t cols);
int osmd_q4_quantize(const float* values, size_t rows, size_t cols, size_t group,
                     uint32_t* packed, float* scales, float* biases, float* bounds,
                     float* block_max, double* block_sum, uint32_t* flags,
                     osmd_stream s);
/* One expert MLP (gate/up GEMV with fused SwiGLU, then down GEMV) for one
 * token, used by the resident-expert operator. h is [inter] scratch. */
int osmd_expert_forward(const uint8_t* blob, osm_expert_geometry g,
                        const float* x, float* h, float* out, osmd_stream s);

/* ---- fused routed-MoE decode ------------------------------------------- */
enum {
  OSMD_MOE_RMSNORM = 1u,  /* x is the residual stream; normalise it first */
  OSMD_MOE_RESIDUAL = 2u, /* y = x + moe(norm(x)) */
  OSMD_MOE_SHARED = 4u    /* add the sigmoid-gated shared expert */
};

typedef struct osmd_moe_args {
  osm_expert_geometry geom;
  uint32_t expert_count;   /* E */
  uint32_t top_k;          /* k */
  uint32_t norm_topk_prob; /* renormalise the selected probabilities */
  uint32_t router_dtype;   /* OSM_META_F32 / F16 / BF16 or OSM_ROUTER_AFFINE_Q8 for router, w_sg */
  uint32_t router_group;   /* OSM_ROUTER_AFFINE_Q8: quantisation group (a multiple of 4 dividing D) */
  uint32_t flags;          /* OSMD_MOE_* */
  uint32_t tokens;         /* B */
  float rms_eps;
  const float* x;                     /* [B, D] */
  float* y;                           /* [B, D] */
  const void* router;                 /* [E, D] */
  const void* shared_gate_vec;        /* [D] */
  const float* norm_weight;           /* [D] */
  const uint8_t* shared_expert;       /* blob */
  const uint8_t* const* expert_table; /* [E] device pointers to blobs, or null */
  const uint8_t* fallback_blob;       /* any valid blob, read in place of a null pointer */
  float* logits;      /* [B, E]   out */
  uint32_t* ids;      /* [B, k]   out */
  float* weights;     /* [B, k]   out */
  float* shared_gate; /* [B]      out */
  float* mass;        /* [B]      out */
  float* x_norm;      /* [B, D]   scratch/out */
  float* h;           /* [B, k+1, I] scratch */
  const uint8_t** slot_ptrs; /* [B, k+1] scratch: blob of each pick, shared last */
  /* Router partial sums (the grouped router GEMM splits K): when logit_planes
   * is set, it holds logit_parts planes [B][E + 1] (column E: the shared-gate
   * dot) that the selection adds in plane order, writing logits and
   * shared_gate itself; when null, logits and shared_gate are final. */
  const float* logit_planes;
  uint32_t logit_parts;
  /* Routing exactness. logit_bounds [B, E]: the router writes, for every
   * logit, a bound on its distance from the reference's sequentially summed
   * fp32 logit; with logit_planes, bound_planes holds the router GEMM's
   * per-plane parts of it, [logit_parts][2][B][E + 1]. The selection ranks on
   * the device logits only where the bounds prove the reference's order, and
   * otherwise recomputes the candidates' logits in the reference's order from
   * x (fp32, or bf16 when x_bf16; RMS-normalised first in the sublayer form).
   * route_stats (null, or 4 counters, added to): selections, selections that
   * took the exact path, exact paths that ranked every expert, and adjacent
   * picks whose order rests on exp rounding within 5 ulps. */
  float* logit_bounds;
  const float* bound_planes;
  uint32_t* route_stats;
  uint32_t x_bf16;
} osmd_moe_args;

/* Largest top-k and expert count the fused decode kernels accept. */
#define OSMD_MAX_TOP_K 16u
#define OSMD_MAX_EXPERTS 1024u

/* decode (every expert resident, expert_table set): three kernels --
 *   route:   RMSNorm (optional) + router GEMV + shared-gate dot -> logits
 *   gate_up: top-k selection from the logits (recomputed by every routed
 *            workgroup; one publishes ids/weights/mass/slot_ptrs), then the
 *            gate/up GEMVs with fused SwiGLU -> h
 *   down:    down GEMVs + weighted accumulate (+ residual) -> y
 * Host-driven residency (expert_table null): osmd_moe_route runs route and a
 * one-workgroup-per-token select kernel, so the host can read ids and write
 * slot_ptrs before osmd_moe_experts (gate_up then reads slot_ptrs). */
int osmd_moe_route(const osmd_moe_args* a, osmd_stream s);
int osmd_moe_experts(const osmd_moe_args* a, osmd_stream s);
int osmd_moe_decode(const osmd_moe_args* a, osmd_stream s);
/* Single kernels, for per-kernel timing: the router GEMV alone, gate/up
 * (with its selection when expert_table is set), and down. */
int osmd_moe_router(const osmd_moe_args* a, osmd_stream s);
int osmd_moe_gate_up(const osmd_moe_args* a, osmd_stream s);
int osmd_moe_down(const osmd_moe_args* a, osmd_stream s);

/* The selection kernel alone: top-k of a->logits for a->tokens tokens into
 * ids / weights / mass (and slot_ptrs from expert_table when set). */
int osmd_moe_select(const osmd_moe_args* a, osmd_stream s);

/* Host-driven residency in rounds (a capped cache runs some slots before
 * others are resident: picks that are already resident while the rest are
 * filled, or a budget that cannot hold a token's picks at once):
 *   osmd_moe_experts_parts: gate/up and down of the listed slots only (every
 *     token), each slot's per-row partials written to parts;
 *   osmd_moe_combine: y from the partials of every slot (and the residual),
 *     accumulated exactly as osmd_moe_experts's down kernel accumulates, so
 *     the result has its bits however the slots were split.
 * parts holds osmd_moe_parts_bytes() bytes ([B][k+1][D][lanes per row]).
 * Slot list: count indices (< k + 1), 5 bits each, entries 0-11 in lo and
 * 12-16 in hi (osmd_slot_list_add). */
typedef struct osmd_slot_list {
  uint64_t lo, hi;
  uint32_t count;
} osmd_slot_list;
static inline void osmd_slot_list_add(osmd_slot_list* l, uint32_t slot) {
  const uint32_t i = l->count++;
  if (i < 12u) l->lo |= (uint64_t)(slot & 31u) << (5u * i);
  else l->hi |= (uint64_t)(slot & 31u) << (5u * (i - 12u));
}
size_t osmd_moe_parts_bytes(const osm_expert_geometry* g, uint32_t nslot, uint32_t tokens);
int osmd_moe_experts_parts(const osmd_moe_args* a, osmd_slot_list slots, float* parts, osmd_stream s);
int osmd_moe_combine(const osmd_moe_args* a, const float* parts, osmd_stream s);

/* ---- grouped (multi-token) MoE ------------------------------------------
 * The routed-MoE sublayer for moe.tokens tokens with every (token, slot)
 * pair bucketed by expert and each expert's gate/up/down run once as an
 * MFMA grouped GEMM for all its pairs. moe.expert_table must be set; moe.x
 * is fp32 [T, D], or bf16 [T, D] when x_bf16 (bf16 router, no RMSNorm form).
 * Workspace sizes for T tokens, P = T * (k + shared) pairs:
 *   x_terms  bf16 [T][3][D]    x_sums   f32 [T][D/G]
 *   pair_pos u32 [P]           pair_w   f32 [P]
 *   tiles    80 B [osmd_moe_grouped_max_tiles()]   tile_count u32 [1]
 *   gu_part  f32 [splits(D)][2][P][I]
 *   h_terms  bf16 [P][2][I]    h_sums   f32 [P][I/G]
 *   partial  f32 [splits(I)][P][D]
 *   logit_planes f32 [osmd_moe_grouped_router_parts(D)][T][E + 1] (router GEMM partials)
 * where splits(n) = osmd_moe_grouped_splits(&moe.geom, n) K ranges of the
 * n columns (hidden for gate/up, inter for down).
 * plus the decode workspace of moe (logits, ids, weights, mass, shared_gate,
 * x_norm). P must be below 2^24 (hipErrorInvalidValue otherwise). */
typedef struct osmd_moe_grouped_args {
  osmd_moe_args moe;
  uint32_t x_bf16;
  uint16_t* x_terms;
  float* x_sums;
  uint32_t* pair_pos;
  float* pair_w;
  void* tiles;
  uint32_t* tile_count;
  float* gu_part;
  uint16_t* h_terms;
  float* h_sums;
  float* partial;
  float* logit_planes;
  /* Error bounds of the router GEMM's logits (any null: no bounds, every
   * selection takes the exact path): the router's 32-column norms
   * [E + 1][D/32] (row E the shared-gate vector), the input's [T][D/32],
   * and the bound planes [router_parts][T][E + 1]. */
  const float* router_norms;
  float* x_norms;
  float* bound_planes;
} osmd_moe_grouped_args;
size_t osmd_moe_grouped_max_tiles(uint32_t tokens, uint32_t nslot, uint32_t experts);
uint32_t osmd_moe_grouped_splits(const osm_expert_geometry* g, uint32_t cols);
uint32_t osmd_moe_grouped_router_parts(uint32_t hidden);
int osmd_moe_grouped(const osmd_moe_grouped_args* a, osmd_stream s);

/* Bytes of LDS the down kernel stages for `nslot` slots of width `inter`
 * (the host rejects layers whose staging exceeds 64 KiB). */
size_t osmd_moe_down_lds_bytes(uint32_t inter, uint32_t nslot);
/* ---- seeded synthetic inputs (bit-identical to the host generator) ------ */
int osmd_synth_expert_blobs(uint64_t seed, uint32_t layer, uint32_t first_expert,
                            uint32_t count, osm_expert_geometry g, uint8_t* dst,
                            size_t stride, osmd_stream s);
int osmd_synth_router_bf16(uint64_t seed, uint32_t layer, uint32_t experts,
                           uint32_t hidden, uint16_t* dst, osmd_stream s);
int osmd_synth_shared_gate_bf16(uint64_t seed, uint32_t layer, uint32_t hidden,
                                uint16_t* dst, osmd_stream s);
int osmd_synth_norm_weight(uint64_t seed, uint32_t layer, uint32_t hidden,
                           float* dst, osmd_stream s);
int osmd_synth_tokens(uint64_t seed, uint32_t first_token, uint32_t count,
                      uint32_t hidden, float* dst, osmd_stream s);

#ifdef __cplusplus
}
#endif

#endif /* OSM_DEVICE_H */
