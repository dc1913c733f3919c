/*
 * osm_oracle.h -- CPU oracle for the q4 routed-MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is a restatement of the reference
 * CPU path (orbi-streammoe src/cpu, src/model/{qwen_router,shared_expert},
 * src/cache) used as the checker for the HIP product library. Only tests/,
 * the smoke() check and the cpu_baseline leg of bench.py may load it. The
 * product (libosm_hip.so) never links, loads or calls it.
 *
 * Every function returns 0 on success and a non-zero code when the reference
 * would have thrown (std::invalid_argument -> 1, std::runtime_error -> 2).
 * The message of the last failure is available from oracle_last_error().
 */
#ifndef OSM_ORACLE_H
#define OSM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_META_F32 = 0, ORACLE_META_F16 = 1, ORACLE_META_BF16 = 2 };

const char* oracle_last_error(void);

/* ---- single_expert_pilot.cpp:276-358 restatement -------------------------
 * quantize_affine_q4_rows: per (row, group) scale = range/15 (1 when flat),
 * bias = min, q = clamp(round-half-away((v - bias) / scale), 0, 15), low
 * nibble first. Outputs packed [rows, cols/8], scales/biases [rows, cols/g],
 * the largest and mean reconstruction error. Returns 1 for bad geometry, 2
 * for a non-finite weight or an error above the group bound. */
int oracle_quantize_affine_q4_rows(const float* values, size_t values_len, size_t rows,
                                   size_t cols, size_t group, uint32_t* packed,
                                   float* scales, float* biases, float* max_abs_error,
                                   double* mean_abs_error);

/* ---- reference_ops.cpp restatement ------------------------------------ */
int oracle_dequantize_affine_rows(const uint32_t* packed, size_t packed_len,
                                  size_t rows, size_t packed_cols,
                                  const float* scales, size_t scales_len,
                                  const float* biases, size_t biases_len,
                                  uint32_t bits, uint32_t group_size,
                                  float* out);
int oracle_matvec_row_major(const float* weight, size_t weight_len,
                            size_t out_dim, size_t in_dim,
                            const float* x, size_t x_len, float* out);
int oracle_rms_norm_inplace(float* values, size_t values_len, size_t rows,
                            size_t dim, const float* weight,
                            size_t weight_len, float eps);
int oracle_softmax_inplace(float* values, size_t n);
int oracle_route_top_k(const float* logits, size_t n, size_t k,
                       int normalize_selected, uint32_t* out_ids,
                       float* out_probs);
float oracle_sigmoid(float v);
float oracle_silu(float v);
int oracle_swiglu_inplace(float* gate, size_t gate_len, const float* up,
                          size_t up_len);

/* ---- qwen_router.cpp / shared_expert.cpp restatement ------------------ */
int oracle_route_qwen_top_k(const float* hidden, size_t hidden_len,
                            const float* router_weight, size_t router_len,
                            size_t hidden_size, size_t expert_count,
                            size_t top_k, int norm_topk_prob,
                            float* out_logits, uint32_t* out_ids,
                            float* out_weights, float* out_mass);
int oracle_run_shared_expert(const float* hidden, size_t hidden_len,
                             const float* gate_proj, size_t gate_len,
                             const float* up_proj, size_t up_len,
                             const float* down_proj, size_t down_len,
                             const float* scalar_gate, size_t scalar_len,
                             size_t hidden_size, size_t intermediate_size,
                             float* out_values, float* out_scalar_gate);

/* ---- metadata widening (vulkan_qpack_expert.cpp:54-87) ---------------- */
float oracle_bf16_to_float(uint16_t bits);

/* ---- the softmax numerator's exp (reference_ops.cpp:141-145) ------------ */
/* Block checksums of std::exp(float) -- the host libm's expf, as the
 * reference's softmax calls it -- over float bit patterns first ..
 * first + count - 1: out[b] = sum over block b's inputs i (i from 0) of
 * bits(exp(x)) * (2 i + 1) mod 2^64. Runs on every hardware thread. */
int oracle_libm_expf_checksums(uint32_t first, uint64_t count, uint32_t block, uint64_t* out);
float oracle_f16_to_float(uint16_t bits);

/* ---- expert blob (qpack section order) -------------------------------- */
size_t oracle_expert_blob_bytes(uint32_t hidden, uint32_t inter,
                                uint32_t group, int meta_dtype);
/* One expert MLP: dequantize x3 -> matvec -> SwiGLU -> matvec. */
int oracle_expert_forward(const uint8_t* blob, uint32_t hidden,
                          uint32_t inter, uint32_t group, int meta_dtype,
                          const float* x, float* out);
/* Single q4 projection (dequantize + matvec), reference GEMV test oracle. */
int oracle_q4_gemv(const uint32_t* packed, size_t out_dim, size_t packed_cols,
                   const float* scales, const float* biases,
                   size_t group_size, const float* x, float* y);

/* Sparse MoE for one token: routed top-k weighted sum + sigmoid-gated
 * shared expert. experts[e] points at expert e's blob. */
int oracle_qwen_sparse_moe(const float* hidden, const float* router_f32,
                           uint32_t expert_count, uint32_t top_k,
                           int norm_topk_prob,
                           const uint8_t* const* experts,
                           const uint8_t* shared_blob,
                           const float* shared_scalar_gate,
                           uint32_t hidden_size, uint32_t inter,
                           uint32_t group, int meta_dtype, float* out,
                           uint32_t* out_ids, float* out_weights,
                           float* out_mass, float* out_shared_gate,
                           float* out_logits);
/* RMSNorm -> sparse MoE -> residual for one token. */
int oracle_moe_sublayer(const float* residual, const float* norm_weight,
                        float eps, const float* router_f32,
                        uint32_t expert_count, uint32_t top_k,
                        int norm_topk_prob, const uint8_t* const* experts,
                        const uint8_t* shared_blob,
                        const float* shared_scalar_gate,
                        uint32_t hidden_size, uint32_t inter, uint32_t group,
                        int meta_dtype, float* out_normalized, float* out,
                        uint32_t* out_ids, float* out_weights,
                        float* out_shared_gate);

/* ---- synthetic seeded generator (counter-based, bit-reproducible) ----- */
/* The sublayer with given routed experts: RMSNorm, pick i's expert
 * (pick_blobs[i]) accumulated with weights[i] in pick order
 * (routed_moe.cpp:31-62), the sigmoid-gated shared expert, the residual. */
int oracle_moe_sublayer_picks(const float* residual, const float* norm_weight, float eps, const float* weights,
                              uint32_t k, const uint8_t* const* pick_blobs, const uint8_t* shared_blob,
                              const float* shared_scalar_gate, uint32_t hidden_size, uint32_t inter, uint32_t group,
                              int meta_dtype, float* out);

uint64_t oracle_synth_stream(uint64_t seed, uint32_t a, uint32_t b,
                             uint32_t tensor);
float oracle_synth_normal(uint64_t stream, uint64_t index);
void oracle_synth_expert_blob(uint64_t seed, uint32_t layer, uint32_t expert,
                              uint32_t hidden, uint32_t inter, uint32_t group,
                              int meta_dtype, uint8_t* out);
void oracle_synth_router_bf16(uint64_t seed, uint32_t layer,
                              uint32_t expert_count, uint32_t hidden,
                              uint16_t* out);
void oracle_synth_shared_gate_bf16(uint64_t seed, uint32_t layer,
                                   uint32_t hidden, uint16_t* out);
void oracle_synth_norm_weight(uint64_t seed, uint32_t layer, uint32_t hidden,
                              float* out);
void oracle_synth_tokens(uint64_t seed, uint32_t first_token, uint32_t count,
                         uint32_t hidden, float* out);

/* ---- cache policies (expert_cache.cpp, vulkan_resident_expert_cache.cpp) */
typedef struct oracle_host_cache oracle_host_cache;
/* Host L1 cache over a fake storage that writes (layer*37+expert*11+i)&0xFF. */
oracle_host_cache* oracle_host_cache_create(size_t stride, size_t budget,
                                            size_t minimum_slots);
void oracle_host_cache_destroy(oracle_host_cache* c);
/* fail_read != 0 makes the fake storage throw on this batch. Returns 0, or
 * 2 when the reference would throw std::runtime_error. out_slots gets the
 * slot per requested expert; out_bytes_ok is 1 when every returned slot
 * holds the expected pattern bytes. */
int oracle_host_cache_fetch(oracle_host_cache* c, uint32_t layer,
                            const uint32_t* experts, size_t n, int fail_read,
                            uint64_t* out_slots, int* out_bytes_ok);
int64_t oracle_host_cache_resident_slot(oracle_host_cache* c, uint32_t layer,
                                        uint32_t expert);
void oracle_host_cache_stats(oracle_host_cache* c, uint64_t* out6);
uint64_t oracle_host_cache_storage_batches(oracle_host_cache* c);

typedef struct oracle_device_cache oracle_device_cache;
oracle_device_cache* oracle_device_cache_create(size_t budget_bytes);
void oracle_device_cache_destroy(oracle_device_cache* c);
/* Returns 1 on hit, 0 on miss (loaded), negative on failure. Evicted keys
 * ((layer<<32)|expert) are written to out_evicted (capacity cap) and
 * counted in *out_n_evicted. */
int oracle_device_cache_get(oracle_device_cache* c, uint32_t layer,
                            uint32_t expert, size_t accounted_bytes,
                            uint64_t* out_evicted, size_t cap,
                            size_t* out_n_evicted);
int oracle_device_cache_contains(oracle_device_cache* c, uint32_t layer,
                                 uint32_t expert);
void oracle_device_cache_stats(oracle_device_cache* c, uint64_t* out7);

#ifdef __cplusplus
}
#endif

#endif /* OSM_ORACLE_H */
