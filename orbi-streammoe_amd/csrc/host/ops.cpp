// ops.cpp -- q4 projection weights and the single operators (the HIP
// counterparts of vulkan_q4_weights.cpp, vulkan_q4_dequant.cpp,
// vulkan_q4_gemv.cpp, vulkan_swiglu.cpp, vulkan_weighted_accumulate.cpp and
// vulkan_rmsnorm.cpp). Geometry is validated before any allocation or launch,
// with the reference's checks.
#include <cstring>
#include <limits>
#include <string>
#include <utility>

#include "host_util.hpp"
#include "osm_hip.hpp"

namespace osm {
namespace {

// vulkan_q4_gemv.cpp:286-337 / vulkan_q4_weights.cpp:98-140 /
// vulkan_q4_dequant.cpp:280-330.
bool validate_q4(std::size_t out_dim, std::size_t packed_cols, std::size_t group,
                 std::size_t packed_len, std::size_t scales_len, std::size_t biases_len,
                 std::string* diagnostic) {
  if (out_dim == 0U || packed_cols == 0U || group == 0U)
    return set_diag(diagnostic, "Q4 out_dim, packed_cols, and group_size must be non-zero."), false;
  if (packed_cols > std::numeric_limits<std::size_t>::max() / 8U)
    return set_diag(diagnostic, "Q4 input dimension overflow."), false;
  const std::size_t in_dim = packed_cols * 8U;
  if (in_dim % group != 0U)
    return set_diag(diagnostic, "Q4 input dimension must be divisible by group_size."), false;
  std::size_t words = 0;
  if (!mul_ok(out_dim, packed_cols, words) || packed_len != words)
    return set_diag(diagnostic, "Q4 packed size does not match out_dim * packed_cols."), false;
  std::size_t groups = 0;
  if (!mul_ok(out_dim, in_dim / group, groups))
    return set_diag(diagnostic, "Q4 scale/bias shape overflow."), false;
  if (scales_len != groups || biases_len != groups)
    return set_diag(diagnostic, "Q4 scales/biases do not match out_dim * groups_per_row."), false;
  if (out_dim > std::numeric_limits<std::uint32_t>::max() ||
      packed_cols > std::numeric_limits<std::uint32_t>::max() ||
      in_dim > std::numeric_limits<std::uint32_t>::max() ||
      group > std::numeric_limits<std::uint32_t>::max())
    return set_diag(diagnostic, "Q4 shape exceeds 32-bit kernel indexing."), false;
  return true;
}

// Copies a host span into a new device allocation on the context's stream.
int upload_bytes(HipComputeContext& ctx, DeviceBytes& dst, const void* src, std::size_t bytes) {
  int rc = dst.allocate(bytes);
  if (rc == 0 && bytes) rc = osmd_memcpy_h2d(dst.get(), src, bytes, ctx.stream());
  return rc;
}

bool same_device(const HipComputeContext& ctx, int dev) { return ctx.valid() && ctx.device() == dev; }

}  // namespace

// ---- HipQ4ProjectionWeights ------------------------------------------------
struct HipQ4ProjectionWeights::Impl {
  DeviceBytes packed, scales, biases;
  std::size_t out_dim = 0, packed_cols = 0, group = 0;
  std::uint32_t meta_dtype = OSM_META_F32;
  int device = -1;
};

HipQ4ProjectionWeights::HipQ4ProjectionWeights() = default;
HipQ4ProjectionWeights::~HipQ4ProjectionWeights() = default;
HipQ4ProjectionWeights::HipQ4ProjectionWeights(HipQ4ProjectionWeights&&) noexcept = default;
HipQ4ProjectionWeights& HipQ4ProjectionWeights::operator=(HipQ4ProjectionWeights&&) noexcept = default;

std::optional<HipQ4ProjectionWeights> HipQ4ProjectionWeights::create(
    HipComputeContext& context, std::span<const std::uint32_t> packed, std::size_t out_dim,
    std::size_t packed_cols, std::span<const float> scales, std::span<const float> biases,
    std::size_t group_size, std::string* diagnostic) noexcept {
  if (!validate_q4(out_dim, packed_cols, group_size, packed.size(), scales.size(),
                   biases.size(), diagnostic))
    return std::nullopt;
  return create_raw(context, packed, out_dim, packed_cols, scales.data(), biases.data(),
                    OSM_META_F32, group_size, diagnostic);
}

std::optional<HipQ4ProjectionWeights> HipQ4ProjectionWeights::create_raw(
    HipComputeContext& context, std::span<const std::uint32_t> packed, std::size_t out_dim,
    std::size_t packed_cols, const void* scales, const void* biases, std::uint32_t meta_dtype,
    std::size_t group_size, std::string* diagnostic) noexcept {
  try {
    if (!context.activate(diagnostic)) return std::nullopt;
    if (meta_dtype > OSM_META_BF16) {
      set_diag(diagnostic, "Q4 projection metadata dtype must be F32, F16 or BF16.");
      return std::nullopt;
    }
    if (group_size == 0U || packed_cols == 0U || out_dim == 0U) {
      set_diag(diagnostic, "Q4 projection dimensions and group size must be non-zero.");
      return std::nullopt;
    }
    const std::size_t groups = out_dim * (packed_cols * 8U / group_size);
    if (!validate_q4(out_dim, packed_cols, group_size, packed.size(), groups, groups, diagnostic))
      return std::nullopt;
    if (scales == nullptr || biases == nullptr) {
      set_diag(diagnostic, "Q4 projection scales and biases must be provided.");
      return std::nullopt;
    }
    auto impl = std::make_unique<Impl>();
    const std::size_t mb = groups * osm_meta_bytes(meta_dtype);
    int rc = upload_bytes(context, impl->packed, packed.data(), packed.size_bytes());
    if (rc == 0) rc = upload_bytes(context, impl->scales, scales, mb);
    if (rc == 0) rc = upload_bytes(context, impl->biases, biases, mb);
    if (rc == 0) rc = osmd_stream_synchronize(context.stream());
    if (rc != 0) {
      set_diag(diagnostic, hip_error("Q4 projection upload failed", rc));
      return std::nullopt;
    }
    impl->out_dim = out_dim;
    impl->packed_cols = packed_cols;
    impl->group = group_size;
    impl->meta_dtype = meta_dtype;
    impl->device = context.device();
    HipQ4ProjectionWeights w;
    w.impl_ = std::move(impl);
    set_diag(diagnostic, "Q4 projection weights resident in HBM.");
    return w;
  } catch (const std::exception& e) {
    set_diag(diagnostic, std::string("Q4 projection exception: ") + e.what());
    return std::nullopt;
  }
}

bool HipQ4ProjectionWeights::valid() const noexcept { return impl_ && impl_->packed.get(); }
std::size_t HipQ4ProjectionWeights::out_dim() const noexcept { return impl_ ? impl_->out_dim : 0; }
std::size_t HipQ4ProjectionWeights::packed_cols() const noexcept { return impl_ ? impl_->packed_cols : 0; }
std::size_t HipQ4ProjectionWeights::in_dim() const noexcept { return packed_cols() * 8U; }
std::size_t HipQ4ProjectionWeights::group_size() const noexcept { return impl_ ? impl_->group : 0; }
std::uint32_t HipQ4ProjectionWeights::meta_dtype() const noexcept { return impl_ ? impl_->meta_dtype : 0; }
std::size_t HipQ4ProjectionWeights::packed_size_bytes() const noexcept { return impl_ ? impl_->packed.size() : 0; }
std::size_t HipQ4ProjectionWeights::meta_size_bytes() const noexcept {
  return impl_ ? impl_->scales.size() + impl_->biases.size() : 0;
}
int HipQ4ProjectionWeights::device() const noexcept { return impl_ ? impl_->device : -1; }
osmd_q4_proj HipQ4ProjectionWeights::view() const noexcept {
  osmd_q4_proj p{};
  if (!impl_) return p;
  p.packed = impl_->packed.as<const std::uint32_t>();
  p.scales = impl_->scales.get();
  p.biases = impl_->biases.get();
  p.out_dim = static_cast<std::uint32_t>(impl_->out_dim);
  p.packed_cols = static_cast<std::uint32_t>(impl_->packed_cols);
  p.group = static_cast<std::uint32_t>(impl_->group);
  p.meta_dtype = impl_->meta_dtype;
  return p;
}

// ---- single operators ------------------------------------------------------
HipValuesResult run_hip_q4_dequant(HipComputeContext& context, std::span<const std::uint32_t> packed,
                                   std::size_t rows, std::size_t packed_cols,
                                   std::span<const float> scales, std::span<const float> biases,
                                   std::size_t group_size) noexcept {
  HipValuesResult r;
  try {
    if (!context.activate(&r.diagnostic)) return r;
    if (!validate_q4(rows, packed_cols, group_size, packed.size(), scales.size(), biases.size(),
                     &r.diagnostic))
      return r;
    auto w = HipQ4ProjectionWeights::create(context, packed, rows, packed_cols, scales, biases,
                                            group_size, &r.diagnostic);
    if (!w) return r;
    DeviceBytes out;
    const std::size_t n = rows * packed_cols * 8U;
    int rc = out.allocate(n * sizeof(float));
    const osmd_q4_proj view = w->view();
    if (rc == 0) rc = osmd_q4_dequant(&view, out.as<float>(), context.stream());
    r.values.resize(n);
    if (rc == 0) rc = osmd_memcpy_d2h(r.values.data(), out.get(), n * sizeof(float), context.stream());
    if (rc == 0) rc = osmd_stream_synchronize(context.stream());
    if (rc != 0) {
      r.values.clear();
      r.diagnostic = hip_error("Q4 dequant failed", rc);
      return r;
    }
    r.executed = true;
    r.diagnostic = "HIP Q4 dequant executed.";
  } catch (const std::exception& e) {
    r.values.clear();
    r.diagnostic = std::string("Q4 dequant exception: ") + e.what();
  }
  return r;
}

HipQuantizeResult quantize_affine_q4_rows_hip(HipComputeContext& context, std::span<const float> values,
                                              std::size_t rows, std::size_t cols,
                                              std::size_t group_size) noexcept {
  HipQuantizeResult r;
  try {
    if (rows == 0U || cols == 0U || group_size == 0U || cols % 8U != 0U || cols % group_size != 0U ||
        rows > std::numeric_limits<std::size_t>::max() / cols || values.size() != rows * cols) {
      r.invalid_argument = true;
      r.diagnostic = "affine q4 quantizer: invalid matrix geometry";
      return r;
    }
    if (!context.activate(&r.diagnostic)) return r;
    const std::size_t words = rows * (cols / 8U);
    const std::size_t groups = rows * (cols / group_size);
    const unsigned blocks = osmd_q4_quantize_blocks(rows, cols);
    DeviceBytes v, packed, scales, biases, bounds, bmax, bsum, flags;
    int rc = v.allocate(values.size_bytes());
    if (rc == 0) rc = packed.allocate(words * 4U);
    if (rc == 0) rc = scales.allocate(groups * 4U);
    if (rc == 0) rc = biases.allocate(groups * 4U);
    if (rc == 0) rc = bounds.allocate(groups * 4U);
    if (rc == 0) rc = bmax.allocate(blocks * sizeof(float));
    if (rc == 0) rc = bsum.allocate(blocks * sizeof(double));
    if (rc == 0) rc = flags.allocate(sizeof(std::uint32_t));
    const osmd_stream st = context.stream();
    if (rc == 0) rc = osmd_memcpy_h2d(v.get(), values.data(), values.size_bytes(), st);
    if (rc == 0) rc = osmd_zero(flags.get(), sizeof(std::uint32_t), st);
    if (rc == 0)
      rc = osmd_q4_quantize(v.as<const float>(), rows, cols, group_size, packed.as<std::uint32_t>(),
                            scales.as<float>(), biases.as<float>(), bounds.as<float>(), bmax.as<float>(),
                            bsum.as<double>(), flags.as<std::uint32_t>(), st);
    HipAffineQ4Projection& q = r.projection;
    q.rows = rows;
    q.cols = cols;
    q.packed_cols = cols / 8U;
    q.groups_per_row = cols / group_size;
    q.packed.resize(words);
    q.scales.resize(groups);
    q.biases.resize(groups);
    std::vector<float> hmax(blocks);
    std::vector<double> hsum(blocks);
    std::uint32_t hflags = 0;
    if (rc == 0) rc = osmd_memcpy_d2h(q.packed.data(), packed.get(), words * 4U, st);
    if (rc == 0) rc = osmd_memcpy_d2h(q.scales.data(), scales.get(), groups * 4U, st);
    if (rc == 0) rc = osmd_memcpy_d2h(q.biases.data(), biases.get(), groups * 4U, st);
    if (rc == 0) rc = osmd_memcpy_d2h(hmax.data(), bmax.get(), blocks * sizeof(float), st);
    if (rc == 0) rc = osmd_memcpy_d2h(hsum.data(), bsum.get(), blocks * sizeof(double), st);
    if (rc == 0) rc = osmd_memcpy_d2h(&hflags, flags.get(), sizeof(hflags), st);
    if (rc == 0) rc = osmd_stream_synchronize(st);
    if (rc != 0) {
      r.projection = {};
      r.diagnostic = hip_error("affine q4 quantizer failed", rc);
      return r;
    }
    if (hflags & 1U) {
      r.projection = {};
      r.diagnostic = "affine q4 quantizer: non-finite source weight";
      return r;
    }
    if (hflags & 2U) {
      r.projection = {};
      r.diagnostic = "affine q4 quantizer: error above the group bound";
      return r;
    }
    double total = 0.0;
    for (unsigned b = 0; b < blocks; ++b) {  // fixed order: deterministic
      q.max_abs_error = std::max(q.max_abs_error, hmax[b]);
      total += hsum[b];
    }
    q.mean_abs_error = total / static_cast<double>(rows * cols);
    r.executed = true;
    r.diagnostic = "HIP affine q4 quantizer executed.";
  } catch (const std::exception& e) {
    r.projection = {};
    r.diagnostic = std::string("affine q4 quantizer exception: ") + e.what();
  }
  return r;
}

HipValuesResult run_hip_q4_gemv(HipComputeContext& context, std::span<const std::uint32_t> packed,
                                std::size_t out_dim, std::size_t packed_cols,
                                std::span<const float> scales, std::span<const float> biases,
                                std::size_t group_size, std::span<const float> x) noexcept {
  HipValuesResult r;
  try {
    if (!context.activate(&r.diagnostic)) return r;
    if (!validate_q4(out_dim, packed_cols, group_size, packed.size(), scales.size(),
                     biases.size(), &r.diagnostic))
      return r;
    if (x.size() != packed_cols * 8U) {
      r.diagnostic = "Q4 GEMV input vector size does not match packed logical width.";
      return r;
    }
    auto w = HipQ4ProjectionWeights::create(context, packed, out_dim, packed_cols, scales, biases,
                                            group_size, &r.diagnostic);
    if (!w) return r;
    DeviceBytes xd, yd;
    int rc = upload_bytes(context, xd, x.data(), x.size_bytes());
    if (rc == 0) rc = yd.allocate(out_dim * sizeof(float));
    const osmd_q4_proj view = w->view();
    if (rc == 0) rc = osmd_q4_gemv(&view, xd.as<float>(), yd.as<float>(), context.stream());
    r.values.resize(out_dim);
    if (rc == 0) rc = osmd_memcpy_d2h(r.values.data(), yd.get(), out_dim * sizeof(float), context.stream());
    if (rc == 0) rc = osmd_stream_synchronize(context.stream());
    if (rc != 0) {
      r.values.clear();
      r.diagnostic = hip_error("Q4 GEMV failed", rc);
      return r;
    }
    r.executed = true;
    r.diagnostic = "HIP Q4 GEMV executed.";
  } catch (const std::exception& e) {
    r.values.clear();
    r.diagnostic = std::string("Q4 GEMV exception: ") + e.what();
  }
  return r;
}

HipDispatchResult run_hip_q4_gemv_buffers(HipComputeContext& context,
                                          std::span<const std::uint32_t> packed,
                                          std::size_t out_dim, std::size_t packed_cols,
                                          std::span<const float> scales,
                                          std::span<const float> biases, std::size_t group_size,
                                          const HipFloatBuffer& x, HipFloatBuffer& y) noexcept {
  HipDispatchResult r;
  if (!x.valid() || !y.valid() || !same_device(context, x.device()) || !same_device(context, y.device())) {
    r.diagnostic = "Q4 GEMV buffers are invalid or belong to another device.";
    return r;
  }
  if (x.size() != packed_cols * 8U || y.size() != out_dim) {
    r.diagnostic = "Q4 GEMV activation shapes do not match projection.";
    return r;
  }
  auto w = HipQ4ProjectionWeights::create(context, packed, out_dim, packed_cols, scales, biases,
                                          group_size, &r.diagnostic);
  if (!w) return r;
  r = run_hip_q4_gemv_preloaded(context, *w, x, y);
  if (r.executed) {
    // The staged weights are freed on return; wait for the kernel first.
    std::string d;
    if (!context.synchronize(&d)) {
      r.executed = false;
      r.diagnostic = d;
    }
  }
  return r;
}

HipDispatchResult run_hip_q4_gemv_preloaded(HipComputeContext& context,
                                            const HipQ4ProjectionWeights& weights,
                                            const HipFloatBuffer& x, HipFloatBuffer& y) noexcept {
  HipDispatchResult r;
  if (!context.activate(&r.diagnostic)) return r;
  if (!weights.valid() || !x.valid() || !y.valid()) {
    r.diagnostic = "Preloaded Q4 GEMV requires valid context, weights, and buffers.";
    return r;
  }
  if (x.size() != weights.in_dim() || y.size() != weights.out_dim()) {
    r.diagnostic = "Preloaded Q4 GEMV activation shapes do not match projection.";
    return r;
  }
  if (!same_device(context, weights.device()) || !same_device(context, x.device()) ||
      !same_device(context, y.device())) {
    r.diagnostic = "Preloaded Q4 GEMV resources belong to a different device.";
    return r;
  }
  const osmd_q4_proj view = weights.view();
  const int rc = osmd_q4_gemv(&view, x.data(), y.data(), context.stream());
  if (rc != 0) {
    r.diagnostic = hip_error("Preloaded Q4 GEMV launch failed", rc);
    return r;
  }
  r.executed = true;
  r.diagnostic = "HIP preloaded Q4 GEMV enqueued.";
  return r;
}

HipValuesResult run_hip_swiglu(HipComputeContext& context, std::span<const float> gate,
                               std::span<const float> up) noexcept {
  HipValuesResult r;
  try {
    if (!context.activate(&r.diagnostic)) return r;
    if (gate.empty() || up.empty()) {
      r.diagnostic = "SwiGLU inputs must not be empty.";
      return r;
    }
    if (gate.size() != up.size()) {
      r.diagnostic = "SwiGLU gate/up sizes must match.";
      return r;
    }
    DeviceBytes g, u, o;
    int rc = upload_bytes(context, g, gate.data(), gate.size_bytes());
    if (rc == 0) rc = upload_bytes(context, u, up.data(), up.size_bytes());
    if (rc == 0) rc = o.allocate(gate.size_bytes());
    if (rc == 0) rc = osmd_swiglu(g.as<float>(), u.as<float>(), o.as<float>(), gate.size(), context.stream());
    r.values.resize(gate.size());
    if (rc == 0) rc = osmd_memcpy_d2h(r.values.data(), o.get(), gate.size_bytes(), context.stream());
    if (rc == 0) rc = osmd_stream_synchronize(context.stream());
    if (rc != 0) {
      r.values.clear();
      r.diagnostic = hip_error("SwiGLU failed", rc);
      return r;
    }
    r.executed = true;
    r.diagnostic = "HIP SwiGLU executed.";
  } catch (const std::exception& e) {
    r.values.clear();
    r.diagnostic = std::string("SwiGLU exception: ") + e.what();
  }
  return r;
}

HipDispatchResult run_hip_swiglu_buffers(HipComputeContext& context, const HipFloatBuffer& gate,
                                         const HipFloatBuffer& up, HipFloatBuffer& output) noexcept {
  HipDispatchResult r;
  if (!context.activate(&r.diagnostic)) return r;
  if (!gate.valid() || !up.valid() || !output.valid()) {
    r.diagnostic = "SwiGLU requires valid buffers.";
    return r;
  }
  if (gate.size() == 0U || gate.size() != up.size() || gate.size() != output.size()) {
    r.diagnostic = "SwiGLU buffer sizes must be equal and non-zero.";
    return r;
  }
  if (!same_device(context, gate.device()) || !same_device(context, up.device()) ||
      !same_device(context, output.device())) {
    r.diagnostic = "SwiGLU buffers belong to a different device.";
    return r;
  }
  const int rc = osmd_swiglu(gate.data(), up.data(), output.data(), gate.size(), context.stream());
  if (rc != 0) {
    r.diagnostic = hip_error("SwiGLU launch failed", rc);
    return r;
  }
  r.executed = true;
  r.diagnostic = "HIP SwiGLU enqueued.";
  return r;
}

HipDispatchResult run_hip_weighted_accumulate(HipComputeContext& context,
                                              const HipFloatBuffer& source, float weight,
                                              HipFloatBuffer& accumulator) noexcept {
  HipDispatchResult r;
  if (!context.activate(&r.diagnostic)) return r;
  if (!source.valid() || !accumulator.valid()) {
    r.diagnostic = "weighted accumulate requires valid buffers.";
    return r;
  }
  if (source.size() == 0U || source.size() != accumulator.size()) {
    r.diagnostic = "weighted accumulate buffers must have equal non-zero sizes.";
    return r;
  }
  if (!std::isfinite(weight)) {
    r.diagnostic = "weighted accumulate routing weight must be finite.";
    return r;
  }
  if (!same_device(context, source.device()) || !same_device(context, accumulator.device())) {
    r.diagnostic = "weighted accumulate buffers belong to a different device.";
    return r;
  }
  const int rc = osmd_weighted_accumulate(source.data(), weight, accumulator.data(), source.size(),
                                          context.stream());
  if (rc != 0) {
    r.diagnostic = hip_error("weighted accumulate launch failed", rc);
    return r;
  }
  r.executed = true;
  r.diagnostic = "HIP weighted accumulate enqueued.";
  return r;
}

HipValuesResult run_hip_rms_norm(HipComputeContext& context, std::span<const float> input,
                                 std::size_t rows, std::size_t dim, std::span<const float> weight,
                                 float eps) noexcept {
  HipValuesResult r;
  try {
    if (!context.activate(&r.diagnostic)) return r;
    if (rows == 0 || dim == 0) {
      r.diagnostic = "RMSNorm rows and dim must be non-zero.";
      return r;
    }
    if (input.size() != rows * dim) {
      r.diagnostic = "RMSNorm input size does not match rows * dim.";
      return r;
    }
    if (weight.size() != dim) {
      r.diagnostic = "RMSNorm weight size does not match dim.";
      return r;
    }
    if (eps < 0.0F || !std::isfinite(eps)) {
      r.diagnostic = "RMSNorm eps must be finite and non-negative.";
      return r;
    }
    if (rows > std::numeric_limits<std::uint32_t>::max() ||
        dim > std::numeric_limits<std::uint32_t>::max()) {
      r.diagnostic = "RMSNorm shape exceeds 32-bit kernel indexing.";
      return r;
    }
    DeviceBytes in, w, out;
    int rc = upload_bytes(context, in, input.data(), input.size_bytes());
    if (rc == 0) rc = upload_bytes(context, w, weight.data(), weight.size_bytes());
    if (rc == 0) rc = out.allocate(input.size_bytes());
    if (rc == 0)
      rc = osmd_rms_norm(in.as<float>(), w.as<float>(), out.as<float>(),
                         static_cast<std::uint32_t>(rows), static_cast<std::uint32_t>(dim), eps,
                         context.stream());
    r.values.resize(input.size());
    if (rc == 0) rc = osmd_memcpy_d2h(r.values.data(), out.get(), input.size_bytes(), context.stream());
    if (rc == 0) rc = osmd_stream_synchronize(context.stream());
    if (rc != 0) {
      r.values.clear();
      r.diagnostic = hip_error("RMSNorm failed", rc);
      return r;
    }
    r.executed = true;
    r.diagnostic = "HIP RMSNorm executed.";
  } catch (const std::exception& e) {
    r.values.clear();
    r.diagnostic = std::string("RMSNorm exception: ") + e.what();
  }
  return r;
}

bool run_hip_unpack_nibbles(HipComputeContext& context, std::span<const std::uint32_t> packed,
                            std::span<std::uint8_t> out, std::string* diagnostic) noexcept {
  if (!context.activate(diagnostic)) return false;
  if (packed.empty() || out.size() != packed.size() * 8U)
    return set_diag(diagnostic, "unpack output must hold 8 bytes per packed word"), false;
  DeviceBytes in, o;
  int rc = upload_bytes(context, in, packed.data(), packed.size_bytes());
  if (rc == 0) rc = o.allocate(out.size());
  if (rc == 0) rc = osmd_unpack_nibbles(in.as<const std::uint32_t>(), packed.size(), o.as<std::uint8_t>(), context.stream());
  if (rc == 0) rc = osmd_memcpy_d2h(out.data(), o.get(), out.size(), context.stream());
  if (rc == 0) rc = osmd_stream_synchronize(context.stream());
  if (rc != 0) return set_diag(diagnostic, hip_error("nibble unpack failed", rc)), false;
  return true;
}

}  // namespace osm
