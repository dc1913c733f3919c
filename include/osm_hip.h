/*
 * osm_hip.h -- C ABI of libosm_hip.so, the MI355X (gfx950) implementation of
 * the q4 routed-MoE hot path of orbi-streammoe.
 *
 * This is the drop-in boundary: plain C types, opaque handles, explicit
 * sizes. Each entry point names the reference interface it replaces
 * (paths relative to the orbi-streammoe source tree). Every call returns an
 * osm_status; on failure osm_last_error() holds the diagnostic of the calling
 * thread, the counterpart of the reference's {executed, diagnostic} results.
 * No exception crosses this boundary, and invalid geometry is rejected before
 * any device work is enqueued, as in the reference.
 *
 * Expert weights use the MLX affine 4-bit format: uint32 words carrying 8
 * nibbles (low nibble first), one scale and one bias per group of columns
 * (src/cpu/reference_ops.cpp:48-63). An expert "blob" is the qpack cache-slot
 * layout: gate/up/down x {weight u32, scales, biases} in that order, each
 * section contiguous; osm_expert_blob_bytes() gives its size.
 */
#ifndef OSM_HIP_H
#define OSM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- common --------------------------------------------------------------- */
typedef enum osm_status {
  OSM_OK = 0,
  OSM_E_INVALID = 1, /* rejected arguments/geometry (reference: std::invalid_argument or a failed precondition) */
  OSM_E_RUNTIME = 2, /* runtime failure (reference: std::runtime_error / executed=false) */
  OSM_E_DEVICE = 3   /* HIP runtime error */
} osm_status;

enum osm_meta_dtype_c { OSM_F32 = 0, OSM_F16 = 1, OSM_BF16 = 2 };

/* Router / shared-gate dtype beyond the three above: MLX affine 8-bit, as
 * real checkpoints store mlp.gate and shared_expert_gate
 * (checkpoint_sparse_moe_test.cpp:455-460). The layer's router and
 * shared-gate pointers then point at an osm_affine_q8_c each. */
enum { OSM_AFFINE_Q8 = 3 };
typedef struct osm_affine_q8_c {
  const uint32_t* packed; /* [rows, cols/4], four values per word, low byte first */
  const float* scales;    /* [rows, cols/group] */
  const float* biases;    /* [rows, cols/group] */
  uint32_t group;         /* a multiple of 4 dividing hidden; the same for router and shared gate */
} osm_affine_q8_c;

typedef struct osm_expert_geometry_c {
  uint32_t hidden;     /* model width D: gate/up input, down output */
  uint32_t inter;      /* expert intermediate width I */
  uint32_t group;      /* quantisation group size */
  uint32_t meta_dtype; /* OSM_F32 / OSM_F16 / OSM_BF16 scales and biases */
} osm_expert_geometry_c;

typedef struct osm_context_s* osm_context;
typedef struct osm_buffer_s* osm_buffer;
typedef struct osm_q4_projection_s* osm_q4_projection;
typedef struct osm_expert_s* osm_expert;
typedef struct osm_shared_expert_s* osm_shared_expert;
typedef struct osm_expert_slab_s* osm_expert_slab;
typedef struct osm_expert_store_s* osm_expert_store;
typedef struct osm_host_cache_s* osm_host_cache;
typedef struct osm_expert_storage_s* osm_expert_storage;
typedef struct osm_expert_cache_s* osm_expert_cache;
typedef struct osm_cache_policy_s* osm_cache_policy;
typedef struct osm_moe_layer_s* osm_moe_layer;
typedef struct osm_event_s* osm_event;
typedef struct osm_graph_s* osm_graph;

/* Diagnostic of the last failed call on this thread (empty string if none). */
const char* osm_last_error(void);
int osm_device_count(int* count);

/* ---- context: VulkanComputeContext (include/orbi/streammoe/backend/vulkan_compute_context.hpp:19-49) */
/* A context with a compute stream of its own. */
int osm_context_create(int device, osm_context* out);
/* A context whose operators are all ordered on the caller's stream
 * (a hipStream_t of `device`; OSM_E_DEVICE if it belongs to another device,
 * OSM_E_INVALID if NULL). The caller keeps the stream alive until the
 * context is destroyed; destroying the context leaves it alone. The
 * reference's context owns its one queue (vulkan_compute_context.hpp:19-49);
 * here the caller may share a stream with its own kernels, so that their
 * order needs no events. Fills of the capped expert cache still run on side
 * streams the library owns, joined to this stream by events. */
int osm_context_create_on_stream(int device, void* hip_stream, osm_context* out);
void osm_context_destroy(osm_context ctx);
int osm_context_synchronize(osm_context ctx);
/* Device name, NUL-terminated into buf. */
int osm_context_device_name(osm_context ctx, char* buf, size_t n);
/* The hipStream_t all operators of this context are ordered on. */
void* osm_context_stream(osm_context ctx);

/* Events on the context's compute stream (timing; no reference counterpart). */
int osm_event_create(osm_context ctx, osm_event* out);
void osm_event_destroy(osm_event e);
int osm_event_record(osm_event e);
int osm_event_elapsed_ms(osm_event start, osm_event stop, float* ms);

/* Raw device memory for callers that pass device pointers. */
int osm_device_alloc(osm_context ctx, size_t bytes, void** out);
int osm_device_free(osm_context ctx, void* ptr);
/* Synchronous: they return once the copy is done. */
int osm_memcpy_h2d(osm_context ctx, void* dst, const void* src, size_t bytes);
int osm_memcpy_d2h(osm_context ctx, void* dst, const void* src, size_t bytes);
/* Enqueued on the context's stream, returning before the copy runs: the host
 * memory must stay valid (and, for an upload, unchanged) until the stream has
 * passed the copy (osm_context_synchronize, an event, or the caller's own
 * wait on its stream). Host memory from osm_host_alloc is pinned, so the copy
 * is a DMA that overlaps the host; pageable memory is staged by the HIP
 * runtime. No reference counterpart: the reference's staging copies block on
 * a fence (vulkan_float_buffer.hpp:23-58). */
int osm_memcpy_h2d_async(osm_context ctx, void* dst, const void* src, size_t bytes);
int osm_memcpy_d2h_async(osm_context ctx, void* dst, const void* src, size_t bytes);
/* Pinned (page-locked) host memory for asynchronous copies. */
int osm_host_alloc(osm_context ctx, size_t bytes, void** out);
int osm_host_free(osm_context ctx, void* ptr);
/* Device-to-device copy enqueued on the context's compute stream; returns
 * before it runs (no synchronisation), so it may be captured into a graph or
 * refresh a graph's input between launches. 16-byte aligned copies run as a
 * kernel (1 KB per wavefront load), others as an async memcpy. */
int osm_memcpy_d2d_async(osm_context ctx, void* dst, const void* src, size_t bytes);

/* ---- float buffer: VulkanFloatBuffer (vulkan_float_buffer.hpp:23-58) ------- */
int osm_buffer_create(osm_context ctx, size_t element_count, osm_buffer* out);
void osm_buffer_destroy(osm_buffer b);
size_t osm_buffer_size(osm_buffer b);
float* osm_buffer_device_ptr(osm_buffer b);
/* Synchronous, as the reference's upload/download. */
int osm_buffer_upload(osm_buffer b, const float* values, size_t count);
int osm_buffer_download(osm_buffer b, float* values, size_t count);
/* The same copies enqueued on the context's stream without waiting (the
 * rules of osm_memcpy_h2d_async); count must equal the buffer's size. */
int osm_buffer_upload_async(osm_buffer b, const float* values, size_t count);
int osm_buffer_download_async(osm_buffer b, float* values, size_t count);

/* ---- single operators over host arrays -------------------------------------
 * run_vulkan_q4_dequant (vulkan_q4_dequant.hpp:23-30): out has rows*packed_cols*8 floats. */
int osm_q4_dequant(osm_context ctx, const uint32_t* packed, size_t packed_len, size_t rows,
                   size_t packed_cols, const float* scales, const float* biases,
                   size_t meta_len, size_t group_size, float* out, size_t out_len);
/* run_vulkan_q4_gemv (vulkan_q4_gemv.hpp:25-33). */
int osm_q4_gemv(osm_context ctx, const uint32_t* packed, size_t packed_len, size_t out_dim,
                size_t packed_cols, const float* scales, const float* biases, size_t meta_len,
                size_t group_size, const float* x, size_t x_len, float* y, size_t y_len);
/* run_vulkan_swiglu (vulkan_swiglu.hpp:19-23). */
int osm_swiglu(osm_context ctx, const float* gate, size_t gate_len, const float* up,
               size_t up_len, float* out);
/* run_vulkan_rms_norm (vulkan_rmsnorm.hpp:25-31): out has rows*dim floats. */
int osm_rms_norm(osm_context ctx, const float* input, size_t input_len, size_t rows, size_t dim,
                 const float* weight, size_t weight_len, float eps, float* out);
/* quantize_affine_q4_rows (src/conversion/single_expert_pilot.cpp:276-358)
 * on the device: values [rows, cols] fp32 (host) -> packed [rows, cols/8],
 * scales and biases [rows, cols/group] (host), and the largest and mean
 * absolute reconstruction error. OSM_E_INVALID for bad geometry (the
 * reference's std::invalid_argument), OSM_E_RUNTIME for a non-finite weight
 * or an error above the group bound (its std::runtime_error). */
int osm_q4_quantize(osm_context ctx, const float* values, size_t rows, size_t cols, size_t group,
                    uint32_t* packed, float* scales, float* biases, float* max_abs_error,
                    double* mean_abs_error);
/* Integer-exact nibble unpack of the packed layout: out[8*w + j] = nibble j
 * (low first) of word w (the lane order of reference_ops.cpp:48-63). */
int osm_unpack_nibbles(osm_context ctx, const uint32_t* packed, size_t words, uint8_t* out);

/* ---- operators over device buffers ----------------------------------------
 * run_vulkan_q4_gemv_buffers (vulkan_q4_gemv.hpp:39-48). */
int osm_q4_gemv_buffers(osm_context ctx, const uint32_t* packed, size_t packed_len,
                        size_t out_dim, size_t packed_cols, const float* scales,
                        const float* biases, size_t meta_len, size_t group_size, osm_buffer x,
                        osm_buffer y);
/* VulkanQ4ProjectionWeights::create (vulkan_q4_weights.hpp:30-38); scales and
 * biases are meta_len entries of meta_dtype (the reference passes OSM_F32). */
int osm_q4_projection_create(osm_context ctx, const uint32_t* packed, size_t packed_len,
                             size_t out_dim, size_t packed_cols, const void* scales,
                             const void* biases, uint32_t meta_dtype, size_t group_size,
                             osm_q4_projection* out);
void osm_q4_projection_destroy(osm_q4_projection p);
/* run_vulkan_q4_gemv_preloaded (vulkan_q4_gemv.hpp:53-57). */
int osm_q4_gemv_preloaded(osm_context ctx, osm_q4_projection weights, osm_buffer x, osm_buffer y);
/* run_vulkan_swiglu_buffers (vulkan_swiglu.hpp:25-30). */
int osm_swiglu_buffers(osm_context ctx, osm_buffer gate, osm_buffer up, osm_buffer out);
/* run_vulkan_weighted_accumulate (vulkan_weighted_accumulate.hpp:12-16):
 * accumulator[i] += weight * source[i]. */
int osm_weighted_accumulate(osm_context ctx, osm_buffer source, float weight,
                            osm_buffer accumulator);

/* ---- experts ----------------------------------------------------------------
 * Blob size of one expert (docs/OSM-39B-QPACK-EXPERT-GEOMETRY.md:61-74 byte
 * arithmetic); 0 for a geometry the fused kernels do not support. */
size_t osm_expert_blob_bytes(const osm_expert_geometry_c* g);
/* VulkanResidentExpert::create (vulkan_resident_expert.hpp:41-45). */
int osm_expert_create(osm_context ctx, const void* blob, size_t bytes,
                      const osm_expert_geometry_c* g, osm_expert* out);
void osm_expert_destroy(osm_expert e);
/* VulkanResidentExpert::run (vulkan_resident_expert.hpp:57-59). */
int osm_expert_run(osm_context ctx, osm_expert e, const float* x, size_t x_len, float* out,
                   size_t out_len);
/* VulkanResidentExpert::run_from_buffer / output_buffer (vulkan_resident_expert.hpp:61-69). */
int osm_expert_run_from_buffer(osm_context ctx, osm_expert e, osm_buffer x);
int osm_expert_download_output(osm_expert e, float* out, size_t out_len);
size_t osm_expert_accounted_bytes(osm_expert e);

/* VulkanResidentSharedExpert (vulkan_resident_shared_expert.hpp:49-69). */
int osm_shared_expert_create(osm_context ctx, const void* blob, size_t bytes,
                             const osm_expert_geometry_c* g, const float* scalar_gate,
                             size_t scalar_len, osm_shared_expert* out);
void osm_shared_expert_destroy(osm_shared_expert s);
int osm_shared_expert_scalar_scale(osm_shared_expert s, const float* hidden, size_t len,
                                   float* out_scale);
int osm_shared_expert_run_from_buffer(osm_context ctx, osm_shared_expert s, osm_buffer hidden);
int osm_shared_expert_download_output(osm_shared_expert s, float* out, size_t out_len);

/* ---- HBM-resident expert stack (all experts of `layers` layers) ------------
 * The all-resident mode of the resident cache: every expert in one slab,
 * addressed through a device pointer table, no host round trip per token. */
int osm_expert_slab_create(osm_context ctx, const osm_expert_geometry_c* g, uint32_t layers,
                           uint32_t experts, osm_expert_slab* out);
void osm_expert_slab_destroy(osm_expert_slab s);
size_t osm_expert_slab_stride(osm_expert_slab s);
int osm_expert_slab_upload(osm_expert_slab s, uint32_t layer, uint32_t expert, const void* blob,
                           size_t bytes);
int osm_expert_slab_download(osm_expert_slab s, uint32_t layer, uint32_t expert, void* out,
                             size_t bytes);
/* Fills every expert from the seeded generator on the device. */
int osm_expert_slab_synthesize(osm_expert_slab s, uint64_t seed);

/* ---- routed-MoE layer -------------------------------------------------------
 * Layer state of QwenCheckpointSparseMoeLayer / QwenCheckpointMoeSublayer
 * (checkpoint_sparse_moe.hpp, checkpoint_moe_sublayer.hpp): router [E, D] and
 * shared-expert gate vector [D] in router_dtype, optional RMSNorm weight [D]
 * (fp32, NULL for none), the shared expert blob (NULL when has_shared == 0). */
typedef struct osm_moe_config {
  osm_expert_geometry_c geometry;
  uint32_t expert_count;   /* E (<= 1024) */
  uint32_t top_k;          /* k (<= 16) */
  uint32_t norm_topk_prob; /* renormalise selected probabilities (qwen_router.hpp:10-15) */
  uint32_t has_shared;     /* add sigmoid(w_sg . x) * shared(x) */
  float rms_eps;           /* RMSNorm epsilon of the sublayer form */
} osm_moe_config;

/* router: [E, D] in router_dtype (OSM_F32 / OSM_F16 / OSM_BF16), or an
 * osm_affine_q8_c of [E, D] for OSM_AFFINE_Q8; shared_gate_vec likewise
 * [D] or an osm_affine_q8_c of [1, D]. */
int osm_moe_layer_create(osm_context ctx, const osm_moe_config* cfg, const void* router,
                         uint32_t router_dtype, const void* shared_gate_vec,
                         const float* norm_weight, const void* shared_blob, size_t shared_bytes,
                         uint32_t max_tokens, osm_moe_layer* out);
void osm_moe_layer_destroy(osm_moe_layer l);

/* Outputs of one decode; any pointer may be NULL. */
typedef struct osm_moe_outputs {
  float* out;            /* [tokens, D] */
  float* normalized;     /* [tokens, D] RMSNorm output (sublayer form) */
  uint32_t* ids;         /* [tokens, k] picks by descending probability, ties to the lower id */
  float* weights;        /* [tokens, k] routing weights */
  float* mass;           /* [tokens] selected probability mass (QwenRouterResult) */
  float* shared_gate;    /* [tokens] sigmoid(w_sg . x) */
  float* logits;         /* [tokens, E] router logits */
} osm_moe_outputs;

/* run_qwen_sparse_moe_vulkan_accum (src/model/routed_moe.hpp:58-65) with every
 * expert of slab layer `slab_layer` resident; sublayer != 0 gives
 * QwenCheckpointMoeSublayer::run (checkpoint_moe_sublayer.hpp:55):
 * out = hidden + MoE(RMSNorm(hidden)). Host arrays in and out. */
int osm_moe_layer_run_slab(osm_context ctx, osm_moe_layer l, osm_expert_slab slab,
                           uint32_t slab_layer, const float* hidden, uint32_t tokens,
                           int sublayer, const osm_moe_outputs* outputs);
/* Same through the GPU resident cache: routing on the device, residency
 * decided on the host from the routed ids (one wait), misses filled on side
 * streams while the picks already resident run. A budget that cannot hold
 * the call's picks at once runs them in rounds, each ending just before a
 * get would evict one of its picks (the reference runs each pick right after
 * its get, routed_moe.cpp:320-366); any budget of at least one expert works,
 * and outputs have the bits of the all-resident decode. */
int osm_moe_layer_run_cached(osm_context ctx, osm_moe_layer l, osm_expert_cache cache,
                             uint32_t layer, const float* hidden, uint32_t tokens, int sublayer,
                             const osm_moe_outputs* outputs);
/* Same with caller-chosen routed experts: ids [tokens, k] (< expert_count)
 * and weights [tokens, k] (finite) replace the router's picks; the router
 * still gives the shared gate, logits and the normalised input (no selection
 * runs; the mass output is the given weights' sum). No
 * counterpart in the reference, whose routed MoE always routes itself
 * (routed_moe.cpp:13-92); it drives the cache with an external routing
 * trace, e.g. correlated routing across decode steps. */
int osm_moe_layer_run_cached_picks(osm_context ctx, osm_moe_layer l, osm_expert_cache cache,
                                   uint32_t layer, const float* hidden, uint32_t tokens, int sublayer,
                                   const uint32_t* ids, const float* weights,
                                   const osm_moe_outputs* outputs);
/* Device pointers in and out, stream-ordered, no synchronisation. */
int osm_moe_layer_decode_device(osm_context ctx, osm_moe_layer l, osm_expert_slab slab,
                                uint32_t slab_layer, const float* x_dev, float* y_dev,
                                uint32_t tokens, int sublayer);
/* osm_moe_layer_decode_device without any device allocation. No counterpart
 * in the reference; it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It runs the per-token kernels (same bits as
 * osm_moe_layer_decode_device on OSM_PATH_PER_TOKEN) with their routing
 * workspace in the library's fixed 4 MiB device array, one per GPU, held
 * until the process ends, instead of the layer's. tokens must be in
 * [1, osm_moe_layer_static_tokens_capacity(l)] (119 at the Qwen3-Next
 * shape), else OSM_E_INVALID. Every call on one GPU shares that array, and
 * the routing it leaves there is overwritten by the next call: calls that
 * overlap in time on one GPU (several streams or contexts) race. That
 * routing cannot be queried: osm_moe_layer_routing returns OSM_E_INVALID
 * until the layer's next other call. */
int osm_moe_layer_decode_device_static(osm_context ctx, osm_moe_layer l, osm_expert_slab slab,
                                       uint32_t slab_layer, const float* x_dev, float* y_dev,
                                       uint32_t tokens, int sublayer);
uint32_t osm_moe_layer_static_tokens_capacity(osm_moe_layer l);
/* How decodes run (no counterpart in the reference, which pushes tokens
 * through the sublayer one at a time with 56 dispatches each,
 * src/session/greedy_token_session.cpp:170-192, routed_moe.cpp:254-430):
 * OSM_PATH_AUTO runs the three per-token kernels below 40 tokens and the
 * grouped GEMMs from 40 tokens on (group 32/64/128, hidden and intermediate
 * multiples of 128, 16-byte aligned input); OSM_PATH_PER_TOKEN always runs
 * the per-token kernels; OSM_PATH_GROUPED always buckets (token, slot) pairs
 * by expert and reads each expert once. */
enum osm_moe_path { OSM_PATH_AUTO = 0, OSM_PATH_PER_TOKEN = 1, OSM_PATH_GROUPED = 2 };
int osm_moe_layer_set_path(osm_moe_layer l, int path);
/* A prefill chunk: bf16 x [tokens, D] (device, 16-byte aligned) through the
 * grouped path, MoE form, y fp32 [tokens, D]; needs a bf16 router. Routing
 * per token is that of run_qwen_sparse_moe_vulkan_accum on the widened x. */
int osm_moe_layer_prefill_device(osm_context ctx, osm_moe_layer l, osm_expert_slab slab,
                                 uint32_t slab_layer, const uint16_t* x_bf16_dev, float* y_dev,
                                 uint32_t tokens);
/* The routing of the layer's last call, for its first `tokens` rows: what
 * QwenSparseMoeResult.routing and .shared_gate hold per token
 * (include/orbi/streammoe/model/routed_moe.hpp:21-27) after the device-side
 * calls above (decode_device, prefill_device, decode_layers, graphs), which
 * return only y. ids, weights, mass, shared_gate, logits and normalized (the
 * RMSNorm output of a sublayer decode, the input of a per-token MoE decode)
 * are filled where non-NULL; out is ignored. Synchronises the context's
 * stream. tokens must be in [1, max_tokens]. After
 * osm_moe_layer_decode_device_static, whose routing lives in the shared
 * fixed workspace, it returns OSM_E_INVALID until the layer's next other
 * call. */
int osm_moe_layer_routing(osm_context ctx, osm_moe_layer l, uint32_t tokens,
                          const osm_moe_outputs* outputs);
/* Routing exactness counters of the layer since its creation or the last
 * reset (no counterpart in the reference, whose router always sums on the
 * host in one order, src/cpu/reference_ops.cpp:85-93). The device sums
 * logits in other orders and bounds each one's distance from the
 * reference's; a selection whose order the bounds do not prove recomputes
 * its candidates' logits in the reference's order. out[0] selections (one
 * per token per call), out[1] selections that took that exact path, out[2]
 * exact paths that recomputed every expert and ranked them by the
 * reference's own probabilities (picks near exp underflow, or a near tie),
 * out[3] the near ties that sent a selection there: adjacent candidates
 * whose exps (the host libm's bits) are close enough for their
 * probabilities to round to one value, with the higher id ranked first.
 * Synchronises the context's stream; reset != 0 zeroes them afterwards. */
int osm_moe_layer_routing_stats(osm_context ctx, osm_moe_layer l, uint32_t out[4], int reset);

/* Self-check of the selection's exp (no counterpart in the reference: its
 * probabilities use the host libm's expf, src/cpu/reference_ops.cpp:141-145,
 * whose bits the device reproduces). Evaluates the device's exp on the float
 * bit patterns first_bits .. first_bits + count - 1 and writes
 * ceil(count / block) host checksums: out[b] = sum over block b's inputs i
 * (i from 0) of bits(exp(x)) * (2 i + 1) mod 2^64. A caller compares them
 * with the same sums of its own expf. first_bits + count <= 2^32. */
int osm_libm_expf_checksums(osm_context ctx, uint32_t first_bits, uint64_t count, uint32_t block, uint64_t* out);
/* Enqueues n_layers decodes back to back, as the reference's decoder stack
 * runs its layers in order (src/model/checkpoint_decoder_stack.cpp:191-204).
 * chained != 0: sublayer form, layer i reads the output of layer i-1 (x_dev
 * [tokens, D] in, y_dev [tokens, D] out, scratch_dev [tokens, D] ping-pong).
 * chained == 0: layer i reads x_dev + i*tokens*D and writes y_dev +
 * i*tokens*D (MoE form). Layer i uses layers[i] and slab layer
 * slab_layers[i]. */
/* The decoder stack's MoE sublayers through the capped cache
 * (checkpoint_decoder_stack.cpp:191-204 with run_qwen_sparse_moe_vulkan_accum
 * per layer): layer i runs layers[i] on cache layer cache_layers[i] as a
 * sublayer (RMSNorm, MoE, residual), on the previous layer's output; x and
 * y are host [tokens, D]. pick_ids / pick_weights (both or neither):
 * [n_layers][tokens][k] routed picks given from outside, as
 * osm_moe_layer_run_cached_picks takes them; NULL routes on the device.
 * The activations stay on the device between layers, and each layer's fills
 * wait only for the kernels that last read the slots they overwrite. With
 * picks given the whole stack is enqueued without a host wait, so fills
 * overlap the layers before; with device routing each layer's ids come back
 * to the host (one wait per layer), and the picks already resident run while
 * the misses are copied. Any budget of at least one expert works: when a
 * layer's picks do not fit at once they run in rounds, as the reference runs
 * each pick right after fetching it (routed_moe.cpp:320-366). Outputs are the
 * bits of the layer-by-layer calls. */
int osm_moe_run_cached_layers(osm_context ctx, const osm_moe_layer* layers, const uint32_t* cache_layers,
                              uint32_t n_layers, osm_expert_cache cache, const float* x, uint32_t tokens,
                              const uint32_t* pick_ids, const float* pick_weights, float* y);
int osm_moe_decode_layers(osm_context ctx, const osm_moe_layer* layers,
                          const uint32_t* slab_layers, uint32_t n_layers, osm_expert_slab slab,
                          const float* x_dev, float* y_dev, float* scratch_dev, uint32_t tokens,
                          int chained);
/* ---- graphs (no counterpart in the reference, whose decoder stack
 * dispatches every operator from the host) ------------------------------------
 * A decode step, or any sequence of enqueue-only calls on the context,
 * recorded once into a HIP graph: each launch replays every kernel on the
 * same buffers with one submission. Callers refresh input contents between
 * launches; layers, slabs and buffers must outlive the graph. Between
 * capture_begin and capture_end only enqueue-only calls may be made on the
 * context (decode_layers, moe_layer_decode_device, moe_layer_launch_phase,
 * memcpy_d2d_async); capture_end always ends the capture. */
int osm_decode_graph_create(osm_context ctx, const osm_moe_layer* layers,
                            const uint32_t* slab_layers, uint32_t n_layers, osm_expert_slab slab,
                            const float* x_dev, float* y_dev, float* scratch_dev, uint32_t tokens,
                            int chained, osm_graph* out);
int osm_graph_capture_begin(osm_context ctx);
int osm_graph_capture_end(osm_context ctx, osm_graph* out);
int osm_graph_launch(osm_context ctx, osm_graph g);
void osm_graph_destroy(osm_graph g);
/* Launches one kernel of a decode (phase 0 router GEMV, 1 expert selection +
 * gate/up + SwiGLU, 2 down + weighted accumulate); phases 1 and 2 read what
 * the previous phases of this layer left in its workspace. For per-kernel
 * timing. */
int osm_moe_layer_launch_phase(osm_context ctx, osm_moe_layer l, osm_expert_slab slab,
                               uint32_t slab_layer, const float* x_dev, float* y_dev,
                               uint32_t tokens, int sublayer, int phase);

/* ---- expert sources and caches ---------------------------------------------
 * Whole model in pinned host memory: the fill source of the capped cache.
 * A miss is copied by a 32-workgroup kernel that reads these pages over PCIe
 * (a pinned host L1 cache is read the same way; a pageable one by
 * hipMemcpyAsync), on the cache's side streams. */
int osm_expert_store_create(const osm_expert_geometry_c* g, uint32_t layers, uint32_t experts,
                            osm_expert_store* out);
void osm_expert_store_destroy(osm_expert_store s);
void* osm_expert_store_blob(osm_expert_store s, uint32_t layer, uint32_t expert);
/* Generates every expert on the device and copies it down. */
int osm_expert_store_synthesize(osm_context ctx, osm_expert_store s, uint64_t seed);

/* Storage callback of the host L1 cache (storage/expert_storage.hpp:20-29):
 * fill count destinations of `stride` bytes each; non-zero means the read
 * failed (the reference's storage throws). */
typedef int (*osm_read_experts_fn)(void* user, const uint32_t* layers, const uint32_t* experts,
                                   void* const* destinations, size_t count, size_t stride);

/* PosixPreadExpertStorage (storage/posix_pread_expert_storage.hpp:13-30,
 * posix_pread_expert_storage.cpp:98-187): <container_dir>/packed_experts/
 * layer_LL.bin holds layer LL's `experts` blobs back to back at `stride`
 * (the counts come from the caller; the reference reads them from the
 * container's layout.json). */
int osm_pread_storage_create(const char* container_dir, uint32_t layers, uint32_t experts, size_t stride,
                             osm_expert_storage* out);
void osm_expert_storage_destroy(osm_expert_storage s);
size_t osm_expert_storage_stride(osm_expert_storage s);
/* ExpertStorage::read_experts: every destination (destination_bytes each, at
 * least the stride) is filled, or the call fails: OSM_E_INVALID for a layer
 * or expert out of range or a small destination (checked before any read),
 * OSM_E_RUNTIME for an open or read error or a short read. */
int osm_expert_storage_read(osm_expert_storage s, const uint32_t* layers, const uint32_t* experts,
                            void* const* destinations, size_t count, size_t destination_bytes);

/* An expert's qpack cache slot bound by section name: the entries of the
 * container's section table (container/qpack.hpp:15-21) for gate_proj,
 * up_proj and down_proj (.weight / .scales / .biases), offsets within the
 * slot. The checks are bind_qpack_q4_projection's
 * (vulkan_qpack_expert.cpp:149-239), plus scales/biases in the geometry's
 * metadata dtype. The nine sections are copied into `blob` (blob_bytes =
 * osm_expert_blob_bytes(g)) in the blob's order; *identity (optional) is 1
 * when the slot already is the blob, as in the official contiguous layout,
 * so its first blob_bytes bytes can be uploaded unchanged. slot and blob
 * may be NULL to validate only. OSM_E_RUNTIME for a section table that
 * fails a check, OSM_E_INVALID for bad arguments or a metadata dtype
 * other than the geometry's. */
typedef struct osm_qpack_section_c {
  const char* name;  /* e.g. "gate_proj.weight" */
  const char* dtype; /* "U32", "F32", "F16" or "BF16" */
  uint32_t rank;     /* 2 */
  uint64_t rows, cols, offset, size;
} osm_qpack_section_c;
int osm_qpack_expert_repack(const osm_expert_geometry_c* g, const osm_qpack_section_c* sections, size_t n,
                            uint64_t slot_stride, const void* slot, void* blob, size_t blob_bytes,
                            int* identity);

/* The qpack container (container/qpack.hpp:15-90, container/qpack.cpp:41-308):
 * <dir>/manifest.json, <dir>/packed_experts/layout.json and
 * <dir>/packed_experts/layer_LL.bin. osm_qpack_open parses both JSON files
 * and runs QpackReader's checks (qpack.cpp:170-255): magic "QPACK",
 * version 1, non-zero layerCount / expertCount / expertStride, a non-empty
 * section table whose entries lie within the stride, linearLayers of
 * layerCount entries, quantBits and quantGroupSize both or neither and in
 * agreement with the packed gate/up/down shapes, layout.json and every layer
 * file declared in the manifest with their sizes, each layer file
 * expertCount x expertStride bytes. Any failure is OSM_E_RUNTIME with the
 * reference's message ("qpack: malformed layout <path>: ...", "qpack: section
 * exceeds expertStride: <name>", ...). */
typedef struct osm_qpack_s* osm_qpack;
typedef struct osm_qpack_info {
  const char* magic;             /* valid until osm_qpack_close */
  const char* model_name;
  const char* source_checkpoint;
  uint32_t version;
  uint32_t expert_count, layer_count, section_count;
  uint64_t expert_stride;
  int32_t quant_bits, quant_group_size; /* -1 when the manifest has null */
} osm_qpack_info;
int osm_qpack_open(const char* container_dir, osm_qpack* out);
void osm_qpack_close(osm_qpack q);
int osm_qpack_get_info(osm_qpack q, osm_qpack_info* out);
/* Entry i of layout.json's sections[] in file order, in the form
 * osm_qpack_expert_repack takes (name/dtype valid until close; rank is the
 * shape's length, rows/cols its first two entries or 0).
 * osm_qpack_find_section is QpackLayout::find_section: OSM_E_INVALID when
 * no section has that name. osm_qpack_section_shape copies up to max_dims
 * entries of the full shape and returns its length in *dims. */
int osm_qpack_get_section(osm_qpack q, uint32_t i, osm_qpack_section_c* out);
int osm_qpack_find_section(osm_qpack q, const char* name, osm_qpack_section_c* out);
int osm_qpack_section_shape(osm_qpack q, uint32_t i, uint64_t* shape, uint32_t max_dims, uint32_t* dims);
/* linearLayers: out[l] = 1 for a linear-attention layer; n >= layerCount. */
int osm_qpack_linear_layers(osm_qpack q, uint8_t* out, size_t n);
/* manifest.files: the declared size of a file named relative to the
 * container; OSM_E_INVALID when it is not declared. */
int osm_qpack_file_size(osm_qpack q, const char* relative_path, uint64_t* out);
/* QpackReader::read_expert (qpack.cpp:257-291): one expertStride slot.
 * OSM_E_INVALID for a layer or expert out of range (std::out_of_range) or a
 * destination under the stride (std::invalid_argument); OSM_E_RUNTIME for
 * an open failure or short read. */
int osm_qpack_read_expert(osm_qpack q, uint32_t layer, uint32_t expert, void* destination,
                          size_t destination_bytes);
/* QpackExpertStorage (storage/qpack_expert_storage.cpp:8-33) over a
 * container opened and checked as osm_qpack_open does. g == NULL: the
 * reference's adapter, whole expertStride slots. With a geometry, each slot
 * is bound by section name (the osm_qpack_expert_repack checks, made once at
 * creation) and every read lands as the blob of that geometry, so the
 * storage feeds a host cache and the device caches directly; the stride is
 * then osm_expert_blob_bytes(g). Reads go through pread, in parallel. The
 * handle is destroyed with osm_expert_storage_destroy. */
int osm_qpack_storage_create(const char* container_dir, const osm_expert_geometry_c* g,
                             osm_expert_storage* out);

typedef struct osm_host_cache_stats {
  uint64_t hits, misses, allocated_slots, capacity_slots, logical_bytes, budget_bytes;
} osm_host_cache_stats;

/* ExpertCache (cache/expert_cache.hpp:30-87). pinned != 0 puts slots in
 * pinned memory (needs a device). */
int osm_host_cache_create(size_t stride, size_t budget_bytes, size_t minimum_slots, int pinned,
                          osm_read_experts_fn read, void* user, osm_host_cache* out);
/* The same cache over a storage handle, which must outlive the cache. */
int osm_host_cache_create_with_storage(osm_expert_storage storage, size_t budget_bytes, size_t minimum_slots,
                                       int pinned, osm_host_cache* out);
void osm_host_cache_destroy(osm_host_cache c);
/* ExpertCache::fetch: out_slots[i] is the slot of experts[i]; out_bytes[i]
 * (optional) points at its bytes until the next fetch. */
int osm_host_cache_fetch(osm_host_cache c, uint32_t layer, const uint32_t* experts, size_t n,
                         uint64_t* out_slots, const void** out_bytes);
/* ExpertCache::resident_slot: slot or -1. */
int64_t osm_host_cache_resident_slot(osm_host_cache c, uint32_t layer, uint32_t expert);
void osm_host_cache_stats_get(osm_host_cache c, osm_host_cache_stats* out);

typedef struct osm_expert_cache_stats {
  uint64_t hits, misses, loads, evictions, resident_entries, resident_bytes, budget_bytes;
} osm_expert_cache_stats;

/* VulkanResidentExpertCache (vulkan_resident_expert_cache.hpp:27-83) over a
 * pinned store, or over a host L1 cache (the reference's miss path). */
int osm_expert_cache_create_from_store(osm_context ctx, osm_expert_store store,
                                       size_t budget_bytes, osm_expert_cache* out);
int osm_expert_cache_create_from_host_cache(osm_context ctx, osm_host_cache host,
                                            const osm_expert_geometry_c* g, size_t budget_bytes,
                                            osm_expert_cache* out);
void osm_expert_cache_destroy(osm_expert_cache c);
/* VulkanResidentExpertCache::get: device blob pointer of the resident expert. */
int osm_expert_cache_get(osm_expert_cache c, uint32_t layer, uint32_t expert,
                         const void** out_device_blob);
/* VulkanResidentExpertCache::run. */
int osm_expert_cache_run(osm_expert_cache c, uint32_t layer, uint32_t expert, const float* x,
                         size_t x_len, float* out, size_t out_len);
int osm_expert_cache_contains(osm_expert_cache c, uint32_t layer, uint32_t expert);
void osm_expert_cache_stats_get(osm_expert_cache c, osm_expert_cache_stats* out);
uint64_t osm_expert_cache_bytes_filled(osm_expert_cache c);

/* The resident cache's LFU+recency policy alone (host only, no device):
 * vulkan_resident_expert_cache.cpp:44-188. Returns 1 on a hit, 0 on a miss
 * (the key is admitted; evicted keys (layer<<32)|expert go to `evicted`,
 * their count to *n_evicted), or an osm_status error as a negative value. */
int osm_cache_policy_create(size_t budget_bytes, osm_cache_policy* out);
void osm_cache_policy_destroy(osm_cache_policy p);
int osm_cache_policy_get(osm_cache_policy p, uint32_t layer, uint32_t expert,
                         size_t accounted_bytes, uint64_t* evicted, size_t cap,
                         size_t* n_evicted);
int osm_cache_policy_contains(osm_cache_policy p, uint32_t layer, uint32_t expert);
void osm_cache_policy_stats_get(osm_cache_policy p, osm_expert_cache_stats* out);

/* ---- seeded synthetic inputs, generated on the device ---------------------
 * Bit-identical to the host generator described in the repository docs. */
int osm_synth_expert_blob(osm_context ctx, uint64_t seed, uint32_t layer, uint32_t expert,
                          const osm_expert_geometry_c* g, void* host_out, size_t bytes);
int osm_synth_router_bf16(osm_context ctx, uint64_t seed, uint32_t layer, uint32_t experts,
                          uint32_t hidden, uint16_t* host_out);
int osm_synth_shared_gate_bf16(osm_context ctx, uint64_t seed, uint32_t layer, uint32_t hidden,
                               uint16_t* host_out);
int osm_synth_norm_weight(osm_context ctx, uint64_t seed, uint32_t layer, uint32_t hidden,
                          float* host_out);
int osm_synth_tokens(osm_context ctx, uint64_t seed, uint32_t first_token, uint32_t count,
                     uint32_t hidden, float* host_out);
int osm_synth_tokens_device(osm_context ctx, uint64_t seed, uint32_t first_token, uint32_t count,
                            uint32_t hidden, float* dev_out);

#ifdef __cplusplus
}
#endif

#endif /* OSM_HIP_H */
