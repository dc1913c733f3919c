// capi.cpp -- the C ABI of include/osm_hip.h over the C++ facade.
#include "../../include/osm_hip.h"

#include <cstring>
#include <exception>
#include <memory>
#include <new>
#include <stdexcept>
#include <limits>
#include <string>
#include <vector>

#include "host/host_util.hpp"
#include "host/osm_hip.hpp"

static_assert(sizeof(osm_expert_geometry_c) == sizeof(osm_expert_geometry),
              "public and internal geometry layouts must match");

struct osm_context_s {
  osm::HipComputeContext ctx;
};
struct osm_buffer_s {
  osm::HipFloatBuffer buf;
};
struct osm_q4_projection_s {
  osm::HipQ4ProjectionWeights w;
};
struct osm_expert_s {
  osm::HipResidentExpert e;
};
struct osm_shared_expert_s {
  osm::HipResidentSharedExpert s;
};
struct osm_expert_slab_s {
  osm::HipExpertSlab slab;
  osm_context owner;
};
struct osm_expert_store_s {
  std::unique_ptr<osm::PinnedExpertStore> store;
};
struct osm_graph_s {
  osm::HipGraph graph;
};
struct osm_event_s {
  osmd_event ev = nullptr;
  osm_context ctx = nullptr;
};

namespace {

thread_local std::string g_error;

int fail(int code, std::string msg) {
  g_error = std::move(msg);
  return code;
}
int ok() {
  g_error.clear();
  return OSM_OK;
}
osm_expert_geometry geom_of(const osm_expert_geometry_c* g) {
  osm_expert_geometry out{};
  if (g) std::memcpy(&out, g, sizeof(out));
  return out;
}
// Storage adapter over the caller's read callback.
class CallbackStorage final : public osm::ExpertStorage {
 public:
  CallbackStorage(std::size_t stride, osm_read_experts_fn fn, void* user)
      : stride_(stride), fn_(fn), user_(user) {}
  std::size_t expert_stride_bytes() const noexcept override { return stride_; }
  void read_experts(std::span<osm::ExpertReadRequest> requests) override {
    std::vector<uint32_t> layers, experts;
    std::vector<void*> dst;
    for (auto& r : requests) {
      if (r.destination.size() < stride_) throw std::runtime_error("storage destination too small");
      layers.push_back(r.id.layer);
      experts.push_back(r.id.expert);
      dst.push_back(r.destination.data());
    }
    if (fn_ == nullptr) throw std::runtime_error("expert storage has no read callback");
    const int rc = fn_(user_, layers.data(), experts.data(), dst.data(), dst.size(), stride_);
    if (rc != 0) throw std::runtime_error("expert storage read failed (callback returned " + std::to_string(rc) + ")");
  }

 private:
  std::size_t stride_;
  osm_read_experts_fn fn_;
  void* user_;
};

#define OSM_GUARD_BEGIN try {
#define OSM_GUARD_END                                        \
  }                                                          \
  catch (const std::invalid_argument& e) {                   \
    return fail(OSM_E_INVALID, e.what());                    \
  }                                                          \
  catch (const std::bad_alloc&) {                            \
    return fail(OSM_E_RUNTIME, "host allocation failed");    \
  }                                                          \
  catch (const std::exception& e) {                          \
    return fail(OSM_E_RUNTIME, e.what());                    \
  }                                                          \
  catch (...) {                                              \
    return fail(OSM_E_RUNTIME, "unknown exception");         \
  }

int from_diag(bool executed, const std::string& d) {
  return executed ? ok() : fail(OSM_E_INVALID, d);
}

}  // namespace

struct osm_host_cache_s {
  std::unique_ptr<CallbackStorage> storage;
  std::unique_ptr<osm::HostExpertCache> cache;
};
struct osm_expert_storage_s {
  std::unique_ptr<osm::ExpertStorage> storage;
};
struct osm_qpack_s {
  osm::QpackReader reader;
};
struct osm_expert_cache_s {
  osm_context owner = nullptr;
  std::unique_ptr<osm::HostCacheSource> host_source;  // when built over an L1 cache
  std::unique_ptr<osm::HipResidentExpertCache> cache;
};
struct osm_cache_policy_s {
  osm::LfuRecencyPolicy policy;
  explicit osm_cache_policy_s(std::size_t b) : policy(b) {}
};
struct osm_moe_layer_s {
  osm::HipMoeLayer layer;
};

extern "C" {

const char* osm_last_error(void) { return g_error.c_str(); }

int osm_device_count(int* count) {
  if (!count) return fail(OSM_E_INVALID, "count is null");
  const int rc = osmd_device_count(count);
  if (rc != 0) {
    *count = 0;
    return fail(OSM_E_DEVICE, std::string("hipGetDeviceCount: ") + osmd_error_string(rc));
  }
  return ok();
}

// ---- context ----------------------------------------------------------------
int osm_context_create(int device, osm_context* out) {
  OSM_GUARD_BEGIN
  if (!out) return fail(OSM_E_INVALID, "out is null");
  *out = nullptr;
  std::string d;
  auto c = osm::HipComputeContext::create(device, &d);
  if (!c) return fail(OSM_E_DEVICE, d);
  *out = new osm_context_s{std::move(*c)};
  return ok();
  OSM_GUARD_END
}
int osm_context_create_on_stream(int device, void* stream, osm_context* out) {
  OSM_GUARD_BEGIN
  if (!out) return fail(OSM_E_INVALID, "out is null");
  *out = nullptr;
  if (!stream) return fail(OSM_E_INVALID, "stream is null (osm_context_create makes a context with its own stream)");
  std::string d;
  auto c = osm::HipComputeContext::create(device, &d, stream);
  if (!c) return fail(OSM_E_DEVICE, d);
  *out = new osm_context_s{std::move(*c)};
  return ok();
  OSM_GUARD_END
}
void osm_context_destroy(osm_context ctx) { delete ctx; }
int osm_context_synchronize(osm_context ctx) {
  if (!ctx) return fail(OSM_E_INVALID, "context is null");
  std::string d;
  return ctx->ctx.synchronize(&d) ? ok() : fail(OSM_E_DEVICE, d);
}
int osm_context_device_name(osm_context ctx, char* buf, size_t n) {
  if (!ctx || !buf || n == 0) return fail(OSM_E_INVALID, "invalid arguments");
  std::strncpy(buf, ctx->ctx.device_name().c_str(), n - 1);
  buf[n - 1] = '\0';
  return ok();
}
void* osm_context_stream(osm_context ctx) { return ctx ? ctx->ctx.stream() : nullptr; }

int osm_event_create(osm_context ctx, osm_event* out) {
  if (!ctx || !out) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  auto* e = new osm_event_s;
  e->ctx = ctx;
  const int rc = osmd_event_create(&e->ev);
  if (rc != 0) {
    delete e;
    return fail(OSM_E_DEVICE, osm::hip_error("hipEventCreate", rc));
  }
  *out = e;
  return ok();
}
void osm_event_destroy(osm_event e) {
  if (!e) return;
  if (e->ev) osmd_event_destroy(e->ev);
  delete e;
}
int osm_event_record(osm_event e) {
  if (!e) return fail(OSM_E_INVALID, "event is null");
  const int rc = osmd_event_record(e->ev, e->ctx->ctx.stream());
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("hipEventRecord", rc));
}
int osm_event_elapsed_ms(osm_event start, osm_event stop, float* ms) {
  if (!start || !stop || !ms) return fail(OSM_E_INVALID, "invalid arguments");
  int rc = osmd_event_synchronize(stop->ev);
  if (rc == 0) rc = osmd_event_elapsed_ms(start->ev, stop->ev, ms);
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("hipEventElapsedTime", rc));
}

int osm_device_alloc(osm_context ctx, size_t bytes, void** out) {
  if (!ctx || !out || bytes == 0) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  const int rc = osmd_malloc(out, bytes);
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("hipMalloc", rc));
}
int osm_device_free(osm_context ctx, void* ptr) {
  if (!ctx) return fail(OSM_E_INVALID, "context is null");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  const int rc = osmd_free(ptr);
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("hipFree", rc));
}
int osm_memcpy_h2d(osm_context ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  int rc = osmd_memcpy_h2d(dst, src, bytes, ctx->ctx.stream());
  if (rc == 0) rc = osmd_stream_synchronize(ctx->ctx.stream());
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("hipMemcpy H2D", rc));
}
int osm_memcpy_d2h(osm_context ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  int rc = osmd_memcpy_d2h(dst, src, bytes, ctx->ctx.stream());
  if (rc == 0) rc = osmd_stream_synchronize(ctx->ctx.stream());
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("hipMemcpy D2H", rc));
}

int osm_memcpy_h2d_async(osm_context ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  const int rc = osmd_memcpy_h2d(dst, src, bytes, ctx->ctx.stream());
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("hipMemcpyAsync H2D", rc));
}
int osm_memcpy_d2h_async(osm_context ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  const int rc = osmd_memcpy_d2h(dst, src, bytes, ctx->ctx.stream());
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("hipMemcpyAsync D2H", rc));
}
int osm_host_alloc(osm_context ctx, size_t bytes, void** out) {
  if (!ctx || !out || bytes == 0) return fail(OSM_E_INVALID, "invalid arguments");
  *out = nullptr;
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  const int rc = osmd_host_malloc(out, bytes);
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("hipHostMalloc", rc));
}
int osm_host_free(osm_context ctx, void* ptr) {
  if (!ctx) return fail(OSM_E_INVALID, "context is null");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  const int rc = osmd_host_free(ptr);
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("hipHostFree", rc));
}

int osm_memcpy_d2d_async(osm_context ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  const int rc = osmd_copy_d2d(dst, src, bytes, ctx->ctx.stream());
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("device copy", rc));
}

// ---- float buffer -----------------------------------------------------------
int osm_buffer_create(osm_context ctx, size_t element_count, osm_buffer* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !out) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  auto b = osm::HipFloatBuffer::create(ctx->ctx, element_count, &d);
  if (!b) return fail(OSM_E_INVALID, d);
  *out = new osm_buffer_s{std::move(*b)};
  return ok();
  OSM_GUARD_END
}
void osm_buffer_destroy(osm_buffer b) { delete b; }
size_t osm_buffer_size(osm_buffer b) { return b ? b->buf.size() : 0; }
float* osm_buffer_device_ptr(osm_buffer b) { return b ? b->buf.data() : nullptr; }
int osm_buffer_upload(osm_buffer b, const float* values, size_t count) {
  if (!b || (!values && count)) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  return b->buf.upload(std::span<const float>(values, count), &d) ? ok() : fail(OSM_E_INVALID, d);
}
int osm_buffer_upload_async(osm_buffer b, const float* values, size_t count) {
  if (!b || !values) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  return b->buf.upload_async(values, count, &d) ? ok() : fail(OSM_E_INVALID, d);
}
int osm_buffer_download_async(osm_buffer b, float* values, size_t count) {
  if (!b || !values) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  return b->buf.download_async(values, count, &d) ? ok() : fail(OSM_E_INVALID, d);
}
int osm_buffer_download(osm_buffer b, float* values, size_t count) {
  if (!b || !values) return fail(OSM_E_INVALID, "invalid arguments");
  if (count != b->buf.size()) return fail(OSM_E_INVALID, "float buffer download size mismatch");
  std::string d;
  auto v = b->buf.download(&d);
  if (!v) return fail(OSM_E_DEVICE, d);
  std::memcpy(values, v->data(), v->size() * sizeof(float));
  return ok();
}

// ---- single operators -------------------------------------------------------
int osm_q4_dequant(osm_context ctx, const uint32_t* packed, size_t packed_len, size_t rows,
                   size_t packed_cols, const float* scales, const float* biases, size_t meta_len,
                   size_t group_size, float* out, size_t out_len) {
  OSM_GUARD_BEGIN
  if (!ctx || !packed || !scales || !biases || !out) return fail(OSM_E_INVALID, "null argument");
  if (out_len != rows * packed_cols * 8U) return fail(OSM_E_INVALID, "Q4 dequant output size mismatch");
  auto r = osm::run_hip_q4_dequant(ctx->ctx, {packed, packed_len}, rows, packed_cols,
                                   {scales, meta_len}, {biases, meta_len}, group_size);
  if (!r.executed) return fail(OSM_E_INVALID, r.diagnostic);
  std::memcpy(out, r.values.data(), out_len * sizeof(float));
  return ok();
  OSM_GUARD_END
}

int osm_q4_gemv(osm_context ctx, const uint32_t* packed, size_t packed_len, size_t out_dim,
                size_t packed_cols, const float* scales, const float* biases, size_t meta_len,
                size_t group_size, const float* x, size_t x_len, float* y, size_t y_len) {
  OSM_GUARD_BEGIN
  if (!ctx || !packed || !scales || !biases || !x || !y) return fail(OSM_E_INVALID, "null argument");
  if (y_len != out_dim) return fail(OSM_E_INVALID, "Q4 GEMV output size mismatch");
  auto r = osm::run_hip_q4_gemv(ctx->ctx, {packed, packed_len}, out_dim, packed_cols,
                                {scales, meta_len}, {biases, meta_len}, group_size, {x, x_len});
  if (!r.executed) return fail(OSM_E_INVALID, r.diagnostic);
  std::memcpy(y, r.values.data(), y_len * sizeof(float));
  return ok();
  OSM_GUARD_END
}

int osm_swiglu(osm_context ctx, const float* gate, size_t gate_len, const float* up, size_t up_len,
               float* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !gate || !up || !out) return fail(OSM_E_INVALID, "null argument");
  auto r = osm::run_hip_swiglu(ctx->ctx, {gate, gate_len}, {up, up_len});
  if (!r.executed) return fail(OSM_E_INVALID, r.diagnostic);
  std::memcpy(out, r.values.data(), r.values.size() * sizeof(float));
  return ok();
  OSM_GUARD_END
}

int osm_rms_norm(osm_context ctx, const float* input, size_t input_len, size_t rows, size_t dim,
                 const float* weight, size_t weight_len, float eps, float* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !input || !weight || !out) return fail(OSM_E_INVALID, "null argument");
  auto r = osm::run_hip_rms_norm(ctx->ctx, {input, input_len}, rows, dim, {weight, weight_len}, eps);
  if (!r.executed) return fail(OSM_E_INVALID, r.diagnostic);
  std::memcpy(out, r.values.data(), r.values.size() * sizeof(float));
  return ok();
  OSM_GUARD_END
}

int osm_q4_quantize(osm_context ctx, const float* values, size_t rows, size_t cols, size_t group,
                    uint32_t* packed, float* scales, float* biases, float* max_abs_error,
                    double* mean_abs_error) {
  OSM_GUARD_BEGIN
  if (!ctx || !values || !packed || !scales || !biases || !max_abs_error || !mean_abs_error)
    return fail(OSM_E_INVALID, "null argument");
  if (rows != 0 && cols > std::numeric_limits<size_t>::max() / rows)
    return fail(OSM_E_INVALID, "affine q4 quantizer: invalid matrix geometry");
  auto r = osm::quantize_affine_q4_rows_hip(ctx->ctx, {values, rows * cols}, rows, cols, group);
  if (r.invalid_argument) return fail(OSM_E_INVALID, r.diagnostic);
  if (!r.executed) return fail(OSM_E_RUNTIME, r.diagnostic);
  const auto& q = r.projection;
  std::memcpy(packed, q.packed.data(), q.packed.size() * sizeof(uint32_t));
  std::memcpy(scales, q.scales.data(), q.scales.size() * sizeof(float));
  std::memcpy(biases, q.biases.data(), q.biases.size() * sizeof(float));
  *max_abs_error = q.max_abs_error;
  *mean_abs_error = q.mean_abs_error;
  return ok();
  OSM_GUARD_END
}

int osm_unpack_nibbles(osm_context ctx, const uint32_t* packed, size_t words, uint8_t* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !packed || !out) return fail(OSM_E_INVALID, "null argument");
  std::string d;
  return osm::run_hip_unpack_nibbles(ctx->ctx, {packed, words}, {out, words * 8U}, &d)
             ? ok()
             : fail(OSM_E_INVALID, d);
  OSM_GUARD_END
}

int osm_q4_gemv_buffers(osm_context ctx, const uint32_t* packed, size_t packed_len, size_t out_dim,
                        size_t packed_cols, const float* scales, const float* biases,
                        size_t meta_len, size_t group_size, osm_buffer x, osm_buffer y) {
  OSM_GUARD_BEGIN
  if (!ctx || !packed || !scales || !biases || !x || !y) return fail(OSM_E_INVALID, "null argument");
  auto r = osm::run_hip_q4_gemv_buffers(ctx->ctx, {packed, packed_len}, out_dim, packed_cols,
                                        {scales, meta_len}, {biases, meta_len}, group_size, x->buf,
                                        y->buf);
  return from_diag(r.executed, r.diagnostic);
  OSM_GUARD_END
}

int osm_q4_projection_create(osm_context ctx, const uint32_t* packed, size_t packed_len,
                             size_t out_dim, size_t packed_cols, const void* scales,
                             const void* biases, uint32_t meta_dtype, size_t group_size,
                             osm_q4_projection* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !packed || !out) return fail(OSM_E_INVALID, "null argument");
  std::string d;
  auto w = osm::HipQ4ProjectionWeights::create_raw(ctx->ctx, {packed, packed_len}, out_dim,
                                                   packed_cols, scales, biases, meta_dtype,
                                                   group_size, &d);
  if (!w) return fail(OSM_E_INVALID, d);
  *out = new osm_q4_projection_s{std::move(*w)};
  return ok();
  OSM_GUARD_END
}
void osm_q4_projection_destroy(osm_q4_projection p) { delete p; }

int osm_q4_gemv_preloaded(osm_context ctx, osm_q4_projection weights, osm_buffer x, osm_buffer y) {
  if (!ctx || !weights || !x || !y) return fail(OSM_E_INVALID, "null argument");
  auto r = osm::run_hip_q4_gemv_preloaded(ctx->ctx, weights->w, x->buf, y->buf);
  return from_diag(r.executed, r.diagnostic);
}
int osm_swiglu_buffers(osm_context ctx, osm_buffer gate, osm_buffer up, osm_buffer out) {
  if (!ctx || !gate || !up || !out) return fail(OSM_E_INVALID, "null argument");
  auto r = osm::run_hip_swiglu_buffers(ctx->ctx, gate->buf, up->buf, out->buf);
  return from_diag(r.executed, r.diagnostic);
}
int osm_weighted_accumulate(osm_context ctx, osm_buffer source, float weight, osm_buffer accumulator) {
  if (!ctx || !source || !accumulator) return fail(OSM_E_INVALID, "null argument");
  auto r = osm::run_hip_weighted_accumulate(ctx->ctx, source->buf, weight, accumulator->buf);
  return from_diag(r.executed, r.diagnostic);
}

// ---- experts ----------------------------------------------------------------
size_t osm_expert_blob_bytes(const osm_expert_geometry_c* g) {
  if (!g) return 0;
  const osm_expert_geometry gg = geom_of(g);
  return osm::check_expert_geometry(gg, nullptr) ? osm::expert_blob_bytes(gg) : 0;
}

int osm_expert_create(osm_context ctx, const void* blob, size_t bytes, const osm_expert_geometry_c* g,
                      osm_expert* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !blob || !g || !out) return fail(OSM_E_INVALID, "null argument");
  std::string d;
  auto e = osm::HipResidentExpert::create(ctx->ctx, {static_cast<const std::byte*>(blob), bytes},
                                          geom_of(g), &d);
  if (!e) return fail(OSM_E_INVALID, d);
  *out = new osm_expert_s{std::move(*e)};
  return ok();
  OSM_GUARD_END
}
void osm_expert_destroy(osm_expert e) { delete e; }

int osm_expert_run(osm_context ctx, osm_expert e, const float* x, size_t x_len, float* out,
                   size_t out_len) {
  OSM_GUARD_BEGIN
  if (!ctx || !e || !x || !out) return fail(OSM_E_INVALID, "null argument");
  if (out_len != e->e.output_dim()) return fail(OSM_E_INVALID, "resident expert output size mismatch");
  auto r = e->e.run(ctx->ctx, {x, x_len});
  if (!r.executed) return fail(OSM_E_INVALID, r.diagnostic);
  std::memcpy(out, r.values.data(), out_len * sizeof(float));
  return ok();
  OSM_GUARD_END
}
int osm_expert_run_from_buffer(osm_context ctx, osm_expert e, osm_buffer x) {
  if (!ctx || !e || !x) return fail(OSM_E_INVALID, "null argument");
  auto r = e->e.run_from_buffer(ctx->ctx, x->buf);
  return from_diag(r.executed, r.diagnostic);
}
int osm_expert_download_output(osm_expert e, float* out, size_t out_len) {
  if (!e || !out) return fail(OSM_E_INVALID, "null argument");
  const auto* b = e->e.output_buffer();
  if (!b) return fail(OSM_E_INVALID, "resident expert has not run yet");
  if (out_len != b->size()) return fail(OSM_E_INVALID, "resident expert output size mismatch");
  std::string d;
  auto v = b->download(&d);
  if (!v) return fail(OSM_E_DEVICE, d);
  std::memcpy(out, v->data(), out_len * sizeof(float));
  return ok();
}
size_t osm_expert_accounted_bytes(osm_expert e) { return e ? e->e.accounted_bytes() : 0; }

int osm_shared_expert_create(osm_context ctx, const void* blob, size_t bytes,
                             const osm_expert_geometry_c* g, const float* scalar_gate,
                             size_t scalar_len, osm_shared_expert* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !blob || !g || !scalar_gate || !out) return fail(OSM_E_INVALID, "null argument");
  std::string d;
  auto s = osm::HipResidentSharedExpert::create(ctx->ctx, {static_cast<const std::byte*>(blob), bytes},
                                                geom_of(g), {scalar_gate, scalar_len}, &d);
  if (!s) return fail(OSM_E_INVALID, d);
  *out = new osm_shared_expert_s{std::move(*s)};
  return ok();
  OSM_GUARD_END
}
void osm_shared_expert_destroy(osm_shared_expert s) { delete s; }
int osm_shared_expert_scalar_scale(osm_shared_expert s, const float* hidden, size_t len, float* out_scale) {
  if (!s || !hidden || !out_scale) return fail(OSM_E_INVALID, "null argument");
  std::string d;
  auto v = s->s.scalar_scale({hidden, len}, &d);
  if (!v) return fail(OSM_E_INVALID, d);
  *out_scale = *v;
  return ok();
}
int osm_shared_expert_run_from_buffer(osm_context ctx, osm_shared_expert s, osm_buffer hidden) {
  if (!ctx || !s || !hidden) return fail(OSM_E_INVALID, "null argument");
  auto r = s->s.run_from_buffer(ctx->ctx, hidden->buf);
  return from_diag(r.executed, r.diagnostic);
}
int osm_shared_expert_download_output(osm_shared_expert s, float* out, size_t out_len) {
  if (!s || !out) return fail(OSM_E_INVALID, "null argument");
  const auto* b = s->s.output_buffer();
  if (!b) return fail(OSM_E_INVALID, "shared expert has not run yet");
  if (out_len != b->size()) return fail(OSM_E_INVALID, "shared expert output size mismatch");
  std::string d;
  auto v = b->download(&d);
  if (!v) return fail(OSM_E_DEVICE, d);
  std::memcpy(out, v->data(), out_len * sizeof(float));
  return ok();
}

// ---- slab -------------------------------------------------------------------
int osm_expert_slab_create(osm_context ctx, const osm_expert_geometry_c* g, uint32_t layers,
                           uint32_t experts, osm_expert_slab* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !g || !out) return fail(OSM_E_INVALID, "null argument");
  std::string d;
  auto s = osm::HipExpertSlab::create(ctx->ctx, geom_of(g), layers, experts, &d);
  if (!s) return fail(OSM_E_INVALID, d);
  *out = new osm_expert_slab_s{std::move(*s), ctx};
  return ok();
  OSM_GUARD_END
}
void osm_expert_slab_destroy(osm_expert_slab s) { delete s; }
size_t osm_expert_slab_stride(osm_expert_slab s) { return s ? s->slab.stride() : 0; }
int osm_expert_slab_upload(osm_expert_slab s, uint32_t layer, uint32_t expert, const void* blob,
                           size_t bytes) {
  if (!s || !blob) return fail(OSM_E_INVALID, "null argument");
  std::string d;
  return s->slab.upload(layer, expert, {static_cast<const std::byte*>(blob), bytes}, &d)
             ? ok()
             : fail(OSM_E_INVALID, d);
}
int osm_expert_slab_download(osm_expert_slab s, uint32_t layer, uint32_t expert, void* out, size_t bytes) {
  if (!s || !out) return fail(OSM_E_INVALID, "null argument");
  const std::uint8_t* src = s->slab.blob(layer, expert);
  if (!src) return fail(OSM_E_INVALID, "expert slab index out of range");
  if (bytes != s->slab.stride()) return fail(OSM_E_INVALID, "expert blob size mismatch");
  return osm_memcpy_d2h(s->owner, out, src, bytes);
}
int osm_expert_slab_synthesize(osm_expert_slab s, uint64_t seed) {
  if (!s) return fail(OSM_E_INVALID, "null argument");
  std::string d;
  return s->slab.synthesize(seed, &d) ? ok() : fail(OSM_E_DEVICE, d);
}

// ---- MoE layer ----------------------------------------------------------------
static_assert(sizeof(osm_affine_q8_c) == sizeof(osm_affine_q8) &&
                  offsetof(osm_affine_q8_c, group) == offsetof(osm_affine_q8, group) &&
                  static_cast<uint32_t>(OSM_AFFINE_Q8) == OSM_ROUTER_AFFINE_Q8,
              "the public affine-q8 view is the internal one");
int osm_moe_layer_create(osm_context ctx, const osm_moe_config* cfg, const void* router,
                         uint32_t router_dtype, const void* shared_gate_vec, const float* norm_weight,
                         const void* shared_blob, size_t shared_bytes, uint32_t max_tokens,
                         osm_moe_layer* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !cfg || !router || !out) return fail(OSM_E_INVALID, "null argument");
  osm::HipMoeLayerConfig c;
  c.geometry = geom_of(&cfg->geometry);
  c.expert_count = cfg->expert_count;
  c.top_k = cfg->top_k;
  c.norm_topk_prob = cfg->norm_topk_prob != 0;
  c.has_shared_expert = cfg->has_shared != 0;
  c.rms_eps = cfg->rms_eps;
  std::span<const float> nw;
  if (norm_weight) nw = std::span<const float>(norm_weight, cfg->geometry.hidden);
  std::span<const std::byte> sb;
  if (shared_blob) sb = std::span<const std::byte>(static_cast<const std::byte*>(shared_blob), shared_bytes);
  std::string d;
  auto l = osm::HipMoeLayer::create(ctx->ctx, c, router, router_dtype, shared_gate_vec, nw, sb,
                                    max_tokens, &d);
  if (!l) return fail(OSM_E_INVALID, d);
  *out = new osm_moe_layer_s{std::move(*l)};
  return ok();
  OSM_GUARD_END
}
void osm_moe_layer_destroy(osm_moe_layer l) { delete l; }

static int write_outputs(const osm::HipMoeResult& r, const osm_moe_outputs* o, bool sublayer) {
  if (!o) return ok();
  if (o->out) std::memcpy(o->out, r.values.data(), r.values.size() * sizeof(float));
  if (o->normalized && sublayer)
    std::memcpy(o->normalized, r.normalized.data(), r.normalized.size() * sizeof(float));
  if (o->ids) std::memcpy(o->ids, r.routing.ids.data(), r.routing.ids.size() * sizeof(uint32_t));
  if (o->weights) std::memcpy(o->weights, r.routing.weights.data(), r.routing.weights.size() * sizeof(float));
  if (o->mass) std::memcpy(o->mass, r.routing.mass.data(), r.routing.mass.size() * sizeof(float));
  if (o->shared_gate)
    std::memcpy(o->shared_gate, r.routing.shared_gate.data(), r.routing.shared_gate.size() * sizeof(float));
  if (o->logits) std::memcpy(o->logits, r.routing.logits.data(), r.routing.logits.size() * sizeof(float));
  return ok();
}

int osm_moe_layer_run_slab(osm_context ctx, osm_moe_layer l, osm_expert_slab slab, uint32_t slab_layer,
                           const float* hidden, uint32_t tokens, int sublayer,
                           const osm_moe_outputs* outputs) {
  OSM_GUARD_BEGIN
  if (!ctx || !l || !slab || !hidden) return fail(OSM_E_INVALID, "null argument");
  const auto* table = slab->slab.device_table(slab_layer);
  if (!table) return fail(OSM_E_INVALID, "slab layer out of range");
  if (slab->slab.experts() != l->layer.config().expert_count)
    return fail(OSM_E_INVALID, "slab expert count does not match the layer's router");
  if (std::memcmp(&slab->slab.geometry(), &l->layer.config().geometry, sizeof(osm_expert_geometry)) != 0)
    return fail(OSM_E_INVALID, "slab expert geometry does not match the layer");
  const std::size_t D = l->layer.config().geometry.hidden;
  auto r = l->layer.run(ctx->ctx, {hidden, static_cast<std::size_t>(tokens) * D}, tokens, table, sublayer != 0);
  if (!r.executed) return fail(OSM_E_INVALID, r.diagnostic);
  return write_outputs(r, outputs, sublayer != 0);
  OSM_GUARD_END
}

int osm_moe_layer_run_cached(osm_context ctx, osm_moe_layer l, osm_expert_cache cache, uint32_t layer,
                             const float* hidden, uint32_t tokens, int sublayer,
                             const osm_moe_outputs* outputs) {
  OSM_GUARD_BEGIN
  if (!ctx || !l || !cache || !hidden) return fail(OSM_E_INVALID, "null argument");
  const std::size_t D = l->layer.config().geometry.hidden;
  auto r = osm::run_qwen_sparse_moe_hip(ctx->ctx, *cache->cache, l->layer, layer,
                                        {hidden, static_cast<std::size_t>(tokens) * D}, sublayer != 0);
  if (!r.executed) return fail(OSM_E_INVALID, r.diagnostic);
  return write_outputs(r, outputs, sublayer != 0);
  OSM_GUARD_END
}

int osm_moe_layer_run_cached_picks(osm_context ctx, osm_moe_layer l, osm_expert_cache cache, uint32_t layer,
                                   const float* hidden, uint32_t tokens, int sublayer, const uint32_t* ids,
                                   const float* weights, const osm_moe_outputs* outputs) {
  OSM_GUARD_BEGIN
  if (!ctx || !l || !cache || !hidden || !ids || !weights) return fail(OSM_E_INVALID, "null argument");
  const std::size_t D = l->layer.config().geometry.hidden;
  const osm::HipMoePicks picks{ids, weights};
  auto r = osm::run_qwen_sparse_moe_hip(ctx->ctx, *cache->cache, l->layer, layer,
                                        {hidden, static_cast<std::size_t>(tokens) * D}, sublayer != 0, &picks);
  if (!r.executed) return fail(OSM_E_INVALID, r.diagnostic);
  return write_outputs(r, outputs, sublayer != 0);
  OSM_GUARD_END
}

int osm_moe_run_cached_layers(osm_context ctx, const osm_moe_layer* layers, const uint32_t* cache_layers,
                              uint32_t n_layers, osm_expert_cache cache, const float* x, uint32_t tokens,
                              const uint32_t* pick_ids, const float* pick_weights, float* y) {
  OSM_GUARD_BEGIN
  if (!ctx || !layers || !cache_layers || !cache || !x || !y || n_layers == 0 || tokens == 0 ||
      (!pick_ids) != (!pick_weights))
    return fail(OSM_E_INVALID, "invalid arguments");
  // The whole stack in one native call: activations on the device, each
  // layer's fills waiting only for the kernels that last read their slots.
  const std::size_t D = layers[0] ? layers[0]->layer.config().geometry.hidden : 0;
  std::vector<osm::HipMoeLayer*> ls(n_layers);
  for (uint32_t i = 0; i < n_layers; ++i) {
    if (!layers[i]) return fail(OSM_E_INVALID, "null layer");
    ls[i] = &layers[i]->layer;
  }
  std::string d;
  if (!osm::run_cached_stack(ctx->ctx, *cache->cache, ls, cache_layers,
                             std::span<const float>(x, static_cast<std::size_t>(tokens) * D), pick_ids, pick_weights,
                             y, &d))
    return fail(OSM_E_INVALID, d);
  return ok();
  OSM_GUARD_END
}

int osm_moe_layer_decode_device(osm_context ctx, osm_moe_layer l, osm_expert_slab slab,
                                uint32_t slab_layer, const float* x_dev, float* y_dev,
                                uint32_t tokens, int sublayer) {
  if (!ctx || !l || !slab) return fail(OSM_E_INVALID, "null argument");
  const auto* table = slab->slab.device_table(slab_layer);
  if (!table) return fail(OSM_E_INVALID, "slab layer out of range");
  if (slab->slab.experts() != l->layer.config().expert_count)
    return fail(OSM_E_INVALID, "slab expert count does not match the layer's router");
  auto r = l->layer.decode_device(ctx->ctx, x_dev, y_dev, tokens, table, sublayer != 0);
  return from_diag(r.executed, r.diagnostic);
}

int osm_moe_layer_decode_device_static(osm_context ctx, osm_moe_layer l, osm_expert_slab slab,
                                       uint32_t slab_layer, const float* x_dev, float* y_dev,
                                       uint32_t tokens, int sublayer) {
  if (!ctx || !l || !slab) return fail(OSM_E_INVALID, "null argument");
  const auto* table = slab->slab.device_table(slab_layer);
  if (!table) return fail(OSM_E_INVALID, "slab layer out of range");
  if (slab->slab.experts() != l->layer.config().expert_count)
    return fail(OSM_E_INVALID, "slab expert count does not match the layer's router");
  const char* diag = "";
  const int rc = l->layer.decode_device_static(ctx->ctx, x_dev, y_dev, tokens, table, sublayer != 0, &diag);
  return rc == OSM_OK ? ok() : fail(rc, diag);
}

uint32_t osm_moe_layer_static_tokens_capacity(osm_moe_layer l) {
  return l ? l->layer.static_tokens_capacity() : 0U;
}


// Builds the facade's decode step from C handles, checking each layer
// against the slab.
static int decode_step_of(osm_context ctx, const osm_moe_layer* layers, const uint32_t* slab_layers,
                          uint32_t n_layers, osm_expert_slab slab, const float* x_dev, float* y_dev,
                          float* scratch_dev, uint32_t tokens, int chained, osm::HipDecodeStep& step) {
  if (!ctx || !layers || !slab_layers || !slab || !x_dev || !y_dev || n_layers == 0)
    return fail(OSM_E_INVALID, "invalid arguments");
  if (chained && !scratch_dev) return fail(OSM_E_INVALID, "chained decode needs a scratch buffer");
  for (uint32_t i = 0; i < n_layers; ++i) {
    if (!layers[i]) return fail(OSM_E_INVALID, "null layer");
    const auto* table = slab->slab.device_table(slab_layers[i]);
    if (!table) return fail(OSM_E_INVALID, "slab layer out of range");
    if (slab->slab.experts() != layers[i]->layer.config().expert_count)
      return fail(OSM_E_INVALID, "slab expert count does not match a layer's router");
    step.layers.push_back(&layers[i]->layer);
    step.tables.push_back(table);
  }
  step.x = x_dev;
  step.y = y_dev;
  step.scratch = scratch_dev;
  step.tokens = tokens;
  step.chained = chained != 0;
  return ok();
}

int osm_moe_decode_layers(osm_context ctx, const osm_moe_layer* layers, const uint32_t* slab_layers,
                          uint32_t n_layers, osm_expert_slab slab, const float* x_dev, float* y_dev,
                          float* scratch_dev, uint32_t tokens, int chained) {
  OSM_GUARD_BEGIN
  osm::HipDecodeStep step;
  const int rc = decode_step_of(ctx, layers, slab_layers, n_layers, slab, x_dev, y_dev, scratch_dev, tokens,
                                chained, step);
  if (rc != OSM_OK) return rc;
  auto r = osm::enqueue_decode_step(ctx->ctx, step);
  return from_diag(r.executed, r.diagnostic);
  OSM_GUARD_END
}

int osm_decode_graph_create(osm_context ctx, const osm_moe_layer* layers, const uint32_t* slab_layers,
                            uint32_t n_layers, osm_expert_slab slab, const float* x_dev, float* y_dev,
                            float* scratch_dev, uint32_t tokens, int chained, osm_graph* out) {
  OSM_GUARD_BEGIN
  if (!out) return fail(OSM_E_INVALID, "null output handle");
  *out = nullptr;
  osm::HipDecodeStep step;
  const int rc = decode_step_of(ctx, layers, slab_layers, n_layers, slab, x_dev, y_dev, scratch_dev, tokens,
                                chained, step);
  if (rc != OSM_OK) return rc;
  std::string diag;
  auto g = osm::HipGraph::capture_decode_step(ctx->ctx, step, &diag);
  if (!g) return fail(OSM_E_INVALID, diag);
  *out = new osm_graph_s{std::move(*g)};
  return ok();
  OSM_GUARD_END
}

int osm_graph_capture_begin(osm_context ctx) {
  OSM_GUARD_BEGIN
  if (!ctx) return fail(OSM_E_INVALID, "null context");
  std::string diag;
  if (!osm::HipGraph::begin_capture(ctx->ctx, &diag)) return fail(OSM_E_DEVICE, diag);
  return ok();
  OSM_GUARD_END
}

int osm_graph_capture_end(osm_context ctx, osm_graph* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !out) return fail(OSM_E_INVALID, "null argument");
  *out = nullptr;
  std::string diag;
  auto g = osm::HipGraph::end_capture(ctx->ctx, &diag);
  if (!g) return fail(OSM_E_DEVICE, diag);
  *out = new osm_graph_s{std::move(*g)};
  return ok();
  OSM_GUARD_END
}

int osm_graph_launch(osm_context ctx, osm_graph g) {
  OSM_GUARD_BEGIN
  if (!ctx || !g) return fail(OSM_E_INVALID, "null argument");
  auto r = g->graph.launch(ctx->ctx);
  return from_diag(r.executed, r.diagnostic);
  OSM_GUARD_END
}

void osm_graph_destroy(osm_graph g) { delete g; }

}  // extern "C"

extern "C" {

int osm_moe_layer_set_path(osm_moe_layer l, int path) {
  if (!l) return fail(OSM_E_INVALID, "null layer");
  if (path < OSM_PATH_AUTO || path > OSM_PATH_GROUPED) return fail(OSM_E_INVALID, "unknown MoE path");
  std::string d;
  return l->layer.set_path(static_cast<osm::HipMoePath>(path), &d) ? ok() : fail(OSM_E_INVALID, d);
}


int osm_moe_layer_prefill_device(osm_context ctx, osm_moe_layer l, osm_expert_slab slab, uint32_t slab_layer,
                                 const uint16_t* x_bf16_dev, float* y_dev, uint32_t tokens) {
  OSM_GUARD_BEGIN
  if (!ctx || !l || !slab) return fail(OSM_E_INVALID, "null argument");
  const auto* table = slab->slab.device_table(slab_layer);
  if (!table) return fail(OSM_E_INVALID, "slab layer out of range");
  if (slab->slab.experts() != l->layer.config().expert_count)
    return fail(OSM_E_INVALID, "slab expert count does not match the layer's router");
  auto r = l->layer.prefill_device_bf16(ctx->ctx, x_bf16_dev, y_dev, tokens, table);
  return from_diag(r.executed, r.diagnostic);
  OSM_GUARD_END
}

int osm_moe_layer_routing(osm_context ctx, osm_moe_layer l, uint32_t tokens, const osm_moe_outputs* outputs) {
  OSM_GUARD_BEGIN
  if (!ctx || !l || !outputs) return fail(OSM_E_INVALID, "null argument");
  if (tokens == 0 || tokens > l->layer.max_tokens())
    return fail(OSM_E_INVALID, "routing download: token count must be in [1, max_tokens]");
  if (!l->layer.routing_queryable())
    return fail(OSM_E_INVALID,
                "routing download: the layer's last decode ran without allocation (its routing is not kept)");
  if (!ctx->ctx.activate(nullptr)) return fail(OSM_E_DEVICE, "HIP compute context cannot be made current");
  osm::HipMoeResult r;
  std::string d;
  if (!l->layer.download_routing(ctx->ctx, tokens, r.routing, &d)) return fail(OSM_E_DEVICE, d);
  if (outputs->normalized && !l->layer.download_normalized(ctx->ctx, tokens, r.normalized, &d))
    return fail(OSM_E_DEVICE, d);
  osm_moe_outputs o = *outputs;
  o.out = nullptr;
  return write_outputs(r, &o, true);
  OSM_GUARD_END
}

int osm_moe_layer_routing_stats(osm_context ctx, osm_moe_layer l, uint32_t out[4], int reset) {
  if (!ctx || !l || !out) return fail(OSM_E_INVALID, "null argument");
  std::uint32_t v[4] = {0, 0, 0, 0};
  std::string d;
  if (!l->layer.routing_stats(ctx->ctx, v, reset != 0, &d)) return fail(OSM_E_DEVICE, d);
  std::memcpy(out, v, sizeof(v));
  return ok();
}

int osm_libm_expf_checksums(osm_context ctx, uint32_t first_bits, uint64_t count, uint32_t block, uint64_t* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !out || count == 0 || block == 0) return fail(OSM_E_INVALID, "invalid arguments");
  if (static_cast<uint64_t>(first_bits) + count > (1ULL << 32)) return fail(OSM_E_INVALID, "range past 2^32");
  const uint64_t nblocks = (count + block - 1) / block;
  if (nblocks > 0x7FFFFFFFULL) return fail(OSM_E_INVALID, "too many blocks");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  osm::DeviceBytes sums;
  int rc = sums.allocate(nblocks * sizeof(uint64_t));
  const osmd_stream st = ctx->ctx.stream();
  if (rc == 0) rc = osmd_libm_expf_checksums(first_bits, count, block, sums.as<uint64_t>(), st);
  if (rc == 0) rc = osmd_memcpy_d2h(out, sums.get(), nblocks * sizeof(uint64_t), st);
  if (rc == 0) rc = osmd_stream_synchronize(st);
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("exp checksums", rc));
  OSM_GUARD_END
}

int osm_moe_layer_launch_phase(osm_context ctx, osm_moe_layer l, osm_expert_slab slab,
                               uint32_t slab_layer, const float* x_dev, float* y_dev, uint32_t tokens,
                               int sublayer, int phase) {
  if (!ctx || !l || !slab) return fail(OSM_E_INVALID, "null argument");
  const auto* table = slab->slab.device_table(slab_layer);
  if (!table) return fail(OSM_E_INVALID, "slab layer out of range");
  if (slab->slab.experts() != l->layer.config().expert_count)
    return fail(OSM_E_INVALID, "slab expert count does not match the layer's router");
  auto r = l->layer.launch_phase(ctx->ctx, x_dev, y_dev, tokens, table, sublayer != 0, phase);
  return from_diag(r.executed, r.diagnostic);
}

// ---- expert store -------------------------------------------------------------
int osm_expert_store_create(const osm_expert_geometry_c* g, uint32_t layers, uint32_t experts,
                            osm_expert_store* out) {
  OSM_GUARD_BEGIN
  if (!g || !out) return fail(OSM_E_INVALID, "null argument");
  auto s = std::make_unique<osm::PinnedExpertStore>(geom_of(g), layers, experts);
  *out = new osm_expert_store_s{std::move(s)};
  return ok();
  OSM_GUARD_END
}
void osm_expert_store_destroy(osm_expert_store s) { delete s; }
void* osm_expert_store_blob(osm_expert_store s, uint32_t layer, uint32_t expert) {
  if (!s) return nullptr;
  try {
    return s->store->mutable_blob(layer, expert);
  } catch (...) {
    return nullptr;
  }
}
int osm_expert_store_synthesize(osm_context ctx, osm_expert_store s, uint64_t seed) {
  OSM_GUARD_BEGIN
  if (!ctx || !s) return fail(OSM_E_INVALID, "null argument");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  auto& st = *s->store;
  // One layer at a time through a device staging buffer.
  osm::DeviceBytes stage;
  const std::size_t layer_bytes = st.stride() * st.experts();
  int rc = stage.allocate(layer_bytes);
  for (uint32_t l = 0; rc == 0 && l < st.layers(); ++l) {
    rc = osmd_synth_expert_blobs(seed, l, 0, st.experts(), st.geometry(), stage.as<std::uint8_t>(),
                                 st.stride(), ctx->ctx.stream());
    if (rc == 0) rc = osmd_memcpy_d2h(st.mutable_blob(l, 0), stage.get(), layer_bytes, ctx->ctx.stream());
    if (rc == 0) rc = osmd_stream_synchronize(ctx->ctx.stream());
  }
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("expert store synthesis failed", rc));
  OSM_GUARD_END
}

// ---- storage ------------------------------------------------------------------
int osm_pread_storage_create(const char* container_dir, uint32_t layers, uint32_t experts, size_t stride,
                             osm_expert_storage* out) {
  OSM_GUARD_BEGIN
  if (!container_dir || !out) return fail(OSM_E_INVALID, "null argument");
  *out = new osm_expert_storage_s{
      std::make_unique<osm::PosixPreadExpertStorage>(container_dir, layers, experts, stride)};
  return ok();
  OSM_GUARD_END
}
void osm_expert_storage_destroy(osm_expert_storage s) { delete s; }
size_t osm_expert_storage_stride(osm_expert_storage s) { return s ? s->storage->expert_stride_bytes() : 0; }
int osm_expert_storage_read(osm_expert_storage s, const uint32_t* layers, const uint32_t* experts,
                            void* const* destinations, size_t count, size_t destination_bytes) {
  OSM_GUARD_BEGIN
  if (!s || (count && (!layers || !experts || !destinations))) return fail(OSM_E_INVALID, "null argument");
  std::vector<osm::ExpertReadRequest> req(count);
  for (size_t i = 0; i < count; ++i) {
    if (!destinations[i]) return fail(OSM_E_INVALID, "null destination");
    req[i] = {{layers[i], experts[i]}, {static_cast<std::byte*>(destinations[i]), destination_bytes}};
  }
  try {
    s->storage->read_experts(req);
  } catch (const std::out_of_range& e) {
    return fail(OSM_E_INVALID, e.what());
  }
  return ok();
  OSM_GUARD_END
}

// ---- qpack slot binding ---------------------------------------------------------
int osm_qpack_expert_repack(const osm_expert_geometry_c* g, const osm_qpack_section_c* sections, size_t n,
                            uint64_t slot_stride, const void* slot, void* blob, size_t blob_bytes,
                            int* identity) {
  OSM_GUARD_BEGIN
  if (!g || (!sections && n)) return fail(OSM_E_INVALID, "null argument");
  std::vector<osm::QpackSectionView> views(n);
  for (size_t i = 0; i < n; ++i) {
    if (!sections[i].name || !sections[i].dtype) return fail(OSM_E_INVALID, "qpack section without name or dtype");
    views[i] = {sections[i].name, sections[i].dtype, sections[i].rank, sections[i].rows, sections[i].cols,
                sections[i].offset, sections[i].size};
  }
  const auto plan = osm::plan_qpack_expert(views, slot_stride, geom_of(g));
  if (identity) *identity = plan.identity ? 1 : 0;
  if (slot || blob) {
    if (!slot || !blob || blob_bytes < plan.blob_bytes) return fail(OSM_E_INVALID, "qpack repack: slot and a blob of osm_expert_blob_bytes needed");
    osm::repack_qpack_expert(plan, static_cast<const std::byte*>(slot), static_cast<std::byte*>(blob));
  }
  return ok();
  OSM_GUARD_END
}

// ---- qpack container ------------------------------------------------------------
namespace {
osm_qpack_section_c section_c(const osm::QpackSection& s) {
  osm_qpack_section_c c{};
  c.name = s.name.c_str();
  c.dtype = s.dtype.c_str();
  c.rank = static_cast<uint32_t>(s.shape.size());
  c.rows = s.shape.size() > 0 ? s.shape[0] : 0U;
  c.cols = s.shape.size() > 1 ? s.shape[1] : 0U;
  c.offset = s.offset;
  c.size = s.size;
  return c;
}
}  // namespace

int osm_qpack_open(const char* container_dir, osm_qpack* out) {
  OSM_GUARD_BEGIN
  if (!container_dir || !out) return fail(OSM_E_INVALID, "null argument");
  *out = nullptr;
  *out = new osm_qpack_s{osm::QpackReader(container_dir)};
  return ok();
  OSM_GUARD_END
}
void osm_qpack_close(osm_qpack q) { delete q; }
int osm_qpack_get_info(osm_qpack q, osm_qpack_info* out) {
  if (!q || !out) return fail(OSM_E_INVALID, "null argument");
  const auto& m = q->reader.manifest();
  const auto& l = q->reader.layout();
  out->magic = m.magic.c_str();
  out->model_name = m.model_name.c_str();
  out->source_checkpoint = m.source_checkpoint.c_str();
  out->version = m.version;
  out->expert_count = l.expert_count;
  out->layer_count = l.layer_count;
  out->section_count = static_cast<uint32_t>(l.sections.size());
  out->expert_stride = l.expert_stride;
  out->quant_bits = m.quant_bits ? static_cast<int32_t>(*m.quant_bits) : -1;
  out->quant_group_size = m.quant_group_size ? static_cast<int32_t>(*m.quant_group_size) : -1;
  return ok();
}
int osm_qpack_get_section(osm_qpack q, uint32_t i, osm_qpack_section_c* out) {
  if (!q || !out) return fail(OSM_E_INVALID, "null argument");
  const auto& secs = q->reader.layout().sections;
  if (i >= secs.size()) return fail(OSM_E_INVALID, "qpack: section index out of range");
  *out = section_c(secs[i]);
  return ok();
}
int osm_qpack_find_section(osm_qpack q, const char* name, osm_qpack_section_c* out) {
  if (!q || !name || !out) return fail(OSM_E_INVALID, "null argument");
  const osm::QpackSection* s = q->reader.layout().find_section(name);
  if (s == nullptr) return fail(OSM_E_INVALID, std::string("qpack: no section named ") + name);
  *out = section_c(*s);
  return ok();
}
int osm_qpack_section_shape(osm_qpack q, uint32_t i, uint64_t* shape, uint32_t max_dims, uint32_t* dims) {
  if (!q || !dims || (max_dims && !shape)) return fail(OSM_E_INVALID, "null argument");
  const auto& secs = q->reader.layout().sections;
  if (i >= secs.size()) return fail(OSM_E_INVALID, "qpack: section index out of range");
  const auto& sh = secs[i].shape;
  *dims = static_cast<uint32_t>(sh.size());
  for (uint32_t d = 0; d < max_dims && d < sh.size(); ++d) shape[d] = sh[d];
  return ok();
}
int osm_qpack_linear_layers(osm_qpack q, uint8_t* out, size_t n) {
  if (!q || !out) return fail(OSM_E_INVALID, "null argument");
  const auto& lin = q->reader.layout().linear_layers;
  if (n < lin.size()) return fail(OSM_E_INVALID, "qpack: output shorter than layerCount");
  for (std::size_t l = 0; l < lin.size(); ++l) out[l] = lin[l] ? 1 : 0;
  return ok();
}
int osm_qpack_file_size(osm_qpack q, const char* relative_path, uint64_t* out) {
  if (!q || !relative_path || !out) return fail(OSM_E_INVALID, "null argument");
  const auto& files = q->reader.manifest().files;
  const auto it = files.find(relative_path);
  if (it == files.end()) return fail(OSM_E_INVALID, std::string("qpack: manifest does not declare ") + relative_path);
  *out = it->second;
  return ok();
}
int osm_qpack_read_expert(osm_qpack q, uint32_t layer, uint32_t expert, void* destination,
                          size_t destination_bytes) {
  OSM_GUARD_BEGIN
  if (!q || (!destination && destination_bytes)) return fail(OSM_E_INVALID, "null argument");
  try {
    q->reader.read_expert(layer, expert, {static_cast<std::byte*>(destination), destination_bytes});
  } catch (const std::out_of_range& e) {
    return fail(OSM_E_INVALID, e.what());
  }
  return ok();
  OSM_GUARD_END
}
int osm_qpack_storage_create(const char* container_dir, const osm_expert_geometry_c* g,
                             osm_expert_storage* out) {
  OSM_GUARD_BEGIN
  if (!container_dir || !out) return fail(OSM_E_INVALID, "null argument");
  *out = nullptr;
  std::unique_ptr<osm::QpackExpertStorage> st;
  if (g) {
    const osm_expert_geometry geom = geom_of(g);
    st = std::make_unique<osm::QpackExpertStorage>(container_dir, &geom);
  } else {
    st = std::make_unique<osm::QpackExpertStorage>(container_dir);
  }
  *out = new osm_expert_storage_s{std::move(st)};
  return ok();
  OSM_GUARD_END
}

// ---- host L1 cache --------------------------------------------------------------
int osm_host_cache_create(size_t stride, size_t budget_bytes, size_t minimum_slots, int pinned,
                          osm_read_experts_fn read, void* user, osm_host_cache* out) {
  OSM_GUARD_BEGIN
  if (!out) return fail(OSM_E_INVALID, "null argument");
  auto storage = std::make_unique<CallbackStorage>(stride, read, user);
  auto cache = std::make_unique<osm::HostExpertCache>(*storage, budget_bytes, minimum_slots, pinned != 0);
  *out = new osm_host_cache_s{std::move(storage), std::move(cache)};
  return ok();
  OSM_GUARD_END
}
int osm_host_cache_create_with_storage(osm_expert_storage storage, size_t budget_bytes, size_t minimum_slots,
                                       int pinned, osm_host_cache* out) {
  OSM_GUARD_BEGIN
  if (!storage || !out) return fail(OSM_E_INVALID, "null argument");
  auto cache = std::make_unique<osm::HostExpertCache>(*storage->storage, budget_bytes, minimum_slots, pinned != 0);
  *out = new osm_host_cache_s{nullptr, std::move(cache)};
  return ok();
  OSM_GUARD_END
}
void osm_host_cache_destroy(osm_host_cache c) { delete c; }
int osm_host_cache_fetch(osm_host_cache c, uint32_t layer, const uint32_t* experts, size_t n,
                         uint64_t* out_slots, const void** out_bytes) {
  OSM_GUARD_BEGIN
  if (!c || (!experts && n) || (!out_slots && n)) return fail(OSM_E_INVALID, "null argument");
  const auto entries = c->cache->fetch(layer, {experts, n});
  for (std::size_t i = 0; i < entries.size(); ++i) {
    out_slots[i] = entries[i].slot;
    if (out_bytes) out_bytes[i] = entries[i].bytes.data();
  }
  return ok();
  OSM_GUARD_END
}
int64_t osm_host_cache_resident_slot(osm_host_cache c, uint32_t layer, uint32_t expert) {
  if (!c) return -1;
  const auto s = c->cache->resident_slot(layer, expert);
  return s ? static_cast<int64_t>(*s) : -1;
}
void osm_host_cache_stats_get(osm_host_cache c, osm_host_cache_stats* out) {
  if (!c || !out) return;
  const auto s = c->cache->stats();
  *out = {s.hits, s.misses, s.allocated_slots, s.capacity_slots, s.logical_bytes, s.budget_bytes};
}

// ---- GPU resident cache -------------------------------------------------------
int osm_expert_cache_create_from_store(osm_context ctx, osm_expert_store store, size_t budget_bytes,
                                       osm_expert_cache* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !store || !out) return fail(OSM_E_INVALID, "null argument");
  auto* c = new osm_expert_cache_s;
  c->owner = ctx;
  try {
    c->cache = std::make_unique<osm::HipResidentExpertCache>(ctx->ctx, *store->store, budget_bytes);
  } catch (...) {
    delete c;
    throw;
  }
  *out = c;
  return ok();
  OSM_GUARD_END
}
int osm_expert_cache_create_from_host_cache(osm_context ctx, osm_host_cache host,
                                            const osm_expert_geometry_c* g, size_t budget_bytes,
                                            osm_expert_cache* out) {
  OSM_GUARD_BEGIN
  if (!ctx || !host || !g || !out) return fail(OSM_E_INVALID, "null argument");
  auto* c = new osm_expert_cache_s;
  c->owner = ctx;
  try {
    c->host_source = std::make_unique<osm::HostCacheSource>(*host->cache, geom_of(g));
    c->cache = std::make_unique<osm::HipResidentExpertCache>(ctx->ctx, *c->host_source, budget_bytes);
  } catch (...) {
    delete c;
    throw;
  }
  *out = c;
  return ok();
  OSM_GUARD_END
}
void osm_expert_cache_destroy(osm_expert_cache c) { delete c; }
int osm_expert_cache_get(osm_expert_cache c, uint32_t layer, uint32_t expert, const void** out_device_blob) {
  if (!c) return fail(OSM_E_INVALID, "null argument");
  std::string d;
  auto* e = c->cache->get(layer, expert, &d);
  if (!e) return fail(OSM_E_RUNTIME, d);
  if (out_device_blob) *out_device_blob = e->device_blob();
  return ok();
}
int osm_expert_cache_run(osm_expert_cache c, uint32_t layer, uint32_t expert, const float* x,
                         size_t x_len, float* out, size_t out_len) {
  OSM_GUARD_BEGIN
  if (!c || !x || !out) return fail(OSM_E_INVALID, "null argument");
  auto r = c->cache->run(layer, expert, {x, x_len});
  if (!r.executed) return fail(OSM_E_RUNTIME, r.diagnostic);
  if (out_len != r.values.size()) return fail(OSM_E_INVALID, "expert cache run output size mismatch");
  std::memcpy(out, r.values.data(), out_len * sizeof(float));
  return ok();
  OSM_GUARD_END
}
int osm_expert_cache_contains(osm_expert_cache c, uint32_t layer, uint32_t expert) {
  return (c && c->cache->contains(layer, expert)) ? 1 : 0;
}
void osm_expert_cache_stats_get(osm_expert_cache c, osm_expert_cache_stats* out) {
  if (!c || !out) return;
  const auto s = c->cache->stats();
  *out = {s.hits, s.misses, s.loads, s.evictions, s.resident_entries, s.resident_bytes, s.budget_bytes};
}
uint64_t osm_expert_cache_bytes_filled(osm_expert_cache c) { return c ? c->cache->bytes_filled() : 0; }

// ---- policy alone -------------------------------------------------------------
int osm_cache_policy_create(size_t budget_bytes, osm_cache_policy* out) {
  OSM_GUARD_BEGIN
  if (!out) return fail(OSM_E_INVALID, "null argument");
  *out = new osm_cache_policy_s(budget_bytes);
  return ok();
  OSM_GUARD_END
}
void osm_cache_policy_destroy(osm_cache_policy p) { delete p; }
int osm_cache_policy_get(osm_cache_policy p, uint32_t layer, uint32_t expert, size_t accounted_bytes,
                         uint64_t* evicted, size_t cap, size_t* n_evicted) {
  if (n_evicted) *n_evicted = 0;
  if (!p) return -fail(OSM_E_INVALID, "null argument");
  try {
    const auto o = p->policy.access(layer, expert, accounted_bytes);
    for (std::size_t i = 0; i < o.evicted.size() && i < cap && evicted; ++i) evicted[i] = o.evicted[i];
    if (n_evicted) *n_evicted = o.evicted.size();
    ok();
    return o.hit ? 1 : 0;
  } catch (const std::invalid_argument& e) {
    return -fail(OSM_E_INVALID, e.what());
  } catch (const std::exception& e) {
    return -fail(OSM_E_RUNTIME, e.what());
  }
}
int osm_cache_policy_contains(osm_cache_policy p, uint32_t layer, uint32_t expert) {
  return (p && p->policy.contains(layer, expert)) ? 1 : 0;
}
void osm_cache_policy_stats_get(osm_cache_policy p, osm_expert_cache_stats* out) {
  if (!p || !out) return;
  const auto& q = p->policy;
  *out = {q.hits, q.misses, q.loads, q.evictions, q.resident_entries(), q.resident_bytes(), q.budget_bytes()};
}

// ---- synthetic inputs -----------------------------------------------------------
}  // extern "C"

namespace {
template <typename F>
int synth_to_host(osm_context ctx, void* host_out, std::size_t bytes, F&& launch) {
  if (!ctx || !host_out || bytes == 0) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  osm::DeviceBytes tmp;
  int rc = tmp.allocate(bytes);
  if (rc == 0) rc = launch(tmp.get());
  if (rc == 0) rc = osmd_memcpy_d2h(host_out, tmp.get(), bytes, ctx->ctx.stream());
  if (rc == 0) rc = osmd_stream_synchronize(ctx->ctx.stream());
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("synthetic generation failed", rc));
}
}  // namespace

extern "C" {

int osm_synth_expert_blob(osm_context ctx, uint64_t seed, uint32_t layer, uint32_t expert,
                          const osm_expert_geometry_c* g, void* host_out, size_t bytes) {
  if (!g) return fail(OSM_E_INVALID, "null geometry");
  const osm_expert_geometry gg = geom_of(g);
  std::string d;
  if (!osm::check_expert_geometry(gg, &d)) return fail(OSM_E_INVALID, d);
  if (bytes != osm::expert_blob_bytes(gg)) return fail(OSM_E_INVALID, "expert blob size mismatch");
  return synth_to_host(ctx, host_out, bytes, [&](void* dev) {
    return osmd_synth_expert_blobs(seed, layer, expert, 1, gg, static_cast<uint8_t*>(dev), bytes,
                                   ctx->ctx.stream());
  });
}
int osm_synth_router_bf16(osm_context ctx, uint64_t seed, uint32_t layer, uint32_t experts, uint32_t hidden,
                          uint16_t* host_out) {
  return synth_to_host(ctx, host_out, static_cast<std::size_t>(experts) * hidden * 2, [&](void* dev) {
    return osmd_synth_router_bf16(seed, layer, experts, hidden, static_cast<uint16_t*>(dev), ctx->ctx.stream());
  });
}
int osm_synth_shared_gate_bf16(osm_context ctx, uint64_t seed, uint32_t layer, uint32_t hidden,
                               uint16_t* host_out) {
  return synth_to_host(ctx, host_out, static_cast<std::size_t>(hidden) * 2, [&](void* dev) {
    return osmd_synth_shared_gate_bf16(seed, layer, hidden, static_cast<uint16_t*>(dev), ctx->ctx.stream());
  });
}
int osm_synth_norm_weight(osm_context ctx, uint64_t seed, uint32_t layer, uint32_t hidden, float* host_out) {
  return synth_to_host(ctx, host_out, static_cast<std::size_t>(hidden) * 4, [&](void* dev) {
    return osmd_synth_norm_weight(seed, layer, hidden, static_cast<float*>(dev), ctx->ctx.stream());
  });
}
int osm_synth_tokens(osm_context ctx, uint64_t seed, uint32_t first_token, uint32_t count, uint32_t hidden,
                     float* host_out) {
  return synth_to_host(ctx, host_out, static_cast<std::size_t>(count) * hidden * 4, [&](void* dev) {
    return osmd_synth_tokens(seed, first_token, count, hidden, static_cast<float*>(dev), ctx->ctx.stream());
  });
}
int osm_synth_tokens_device(osm_context ctx, uint64_t seed, uint32_t first_token, uint32_t count,
                            uint32_t hidden, float* dev_out) {
  if (!ctx || !dev_out) return fail(OSM_E_INVALID, "invalid arguments");
  std::string d;
  if (!ctx->ctx.activate(&d)) return fail(OSM_E_DEVICE, d);
  const int rc = osmd_synth_tokens(seed, first_token, count, hidden, dev_out, ctx->ctx.stream());
  return rc == 0 ? ok() : fail(OSM_E_DEVICE, osm::hip_error("synthetic tokens failed", rc));
}

}  // extern "C"
