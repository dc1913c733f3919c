// experts.cpp -- resident expert, shared expert and the HBM expert slab (the
// HIP counterparts of vulkan_resident_expert.cpp and
// vulkan_resident_shared_expert.cpp).
#include <cmath>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "host_util.hpp"
#include "osm_hip.hpp"

namespace osm {

bool check_expert_geometry(const osm_expert_geometry& g, std::string* diagnostic) noexcept {
  if (g.hidden == 0 || g.inter == 0 || g.group == 0)
    return set_diag(diagnostic, "expert dimensions and group size must be non-zero"), false;
  if (g.meta_dtype > OSM_META_BF16)
    return set_diag(diagnostic, "expert metadata dtype must be F32, F16 or BF16"), false;
  if (!osm_geometry_fused_ok(g))
    return set_diag(diagnostic,
                    "expert geometry unsupported by the fused kernels: hidden and inter must be "
                    "multiples of 32 (hidden <= 8192, inter <= 4096) and the group a multiple of "
                    "32 dividing both"),
           false;
  return true;
}

std::size_t expert_blob_bytes(const osm_expert_geometry& g) noexcept {
  return osm_expert_layout(g).total;
}

// ---- HipResidentExpert -----------------------------------------------------
struct HipResidentExpert::Impl {
  osm_expert_geometry geom{};
  DeviceBytes owned;                 // empty for a view
  const std::uint8_t* blob = nullptr;
  int device = -1;
  std::optional<HipFloatBuffer> input, hidden, output;  // created on first run

  bool ensure_buffers(HipComputeContext& ctx, std::string* d) {
    if (!hidden) {
      hidden = HipFloatBuffer::create(ctx, geom.inter, d);
      if (!hidden) return false;
    }
    if (!output) {
      output = HipFloatBuffer::create(ctx, geom.hidden, d);
      if (!output) return false;
    }
    return true;
  }
};

HipResidentExpert::HipResidentExpert() = default;
HipResidentExpert::~HipResidentExpert() = default;
HipResidentExpert::HipResidentExpert(HipResidentExpert&&) noexcept = default;
HipResidentExpert& HipResidentExpert::operator=(HipResidentExpert&&) noexcept = default;

std::optional<HipResidentExpert> HipResidentExpert::create(HipComputeContext& context,
                                                           std::span<const std::byte> blob,
                                                           const osm_expert_geometry& geometry,
                                                           std::string* diagnostic) noexcept {
  try {
    if (!context.activate(diagnostic)) return std::nullopt;
    if (!check_expert_geometry(geometry, diagnostic)) return std::nullopt;
    const std::size_t bytes = expert_blob_bytes(geometry);
    if (blob.size() != bytes) {
      set_diag(diagnostic, "resident expert blob size does not match its geometry");
      return std::nullopt;
    }
    auto impl = std::make_unique<Impl>();
    int rc = impl->owned.allocate(bytes);
    if (rc == 0) rc = osmd_memcpy_h2d(impl->owned.get(), blob.data(), bytes, context.stream());
    if (rc == 0) rc = osmd_stream_synchronize(context.stream());
    if (rc != 0) {
      set_diag(diagnostic, hip_error("resident expert upload failed", rc));
      return std::nullopt;
    }
    impl->geom = geometry;
    impl->blob = impl->owned.as<const std::uint8_t>();
    impl->device = context.device();
    HipResidentExpert e;
    e.impl_ = std::move(impl);
    set_diag(diagnostic, "HIP resident expert created with gate/up/down weights in HBM.");
    return e;
  } catch (const std::exception& e) {
    set_diag(diagnostic, std::string("resident expert creation exception: ") + e.what());
    return std::nullopt;
  }
}

std::optional<HipResidentExpert> HipResidentExpert::view(HipComputeContext& context,
                                                         const std::uint8_t* device_blob,
                                                         const osm_expert_geometry& geometry,
                                                         std::string* diagnostic) noexcept {
  try {
    if (!context.valid()) {
      set_diag(diagnostic, "HIP compute context is not valid");
      return std::nullopt;
    }
    if (!check_expert_geometry(geometry, diagnostic)) return std::nullopt;
    if (device_blob == nullptr) {
      set_diag(diagnostic, "resident expert view needs a device blob");
      return std::nullopt;
    }
    auto impl = std::make_unique<Impl>();
    impl->geom = geometry;
    impl->blob = device_blob;
    impl->device = context.device();
    HipResidentExpert e;
    e.impl_ = std::move(impl);
    return e;
  } catch (const std::exception& e) {
    set_diag(diagnostic, std::string("resident expert view exception: ") + e.what());
    return std::nullopt;
  }
}

bool HipResidentExpert::valid() const noexcept { return impl_ && impl_->blob; }
std::size_t HipResidentExpert::input_dim() const noexcept { return impl_ ? impl_->geom.hidden : 0; }
std::size_t HipResidentExpert::intermediate_dim() const noexcept { return impl_ ? impl_->geom.inter : 0; }
std::size_t HipResidentExpert::output_dim() const noexcept { return impl_ ? impl_->geom.hidden : 0; }
std::size_t HipResidentExpert::packed_weight_bytes() const noexcept {
  if (!impl_) return 0;
  const auto o = osm_expert_layout(impl_->geom);
  return (o.gate_s - o.gate_q) + (o.up_s - o.up_q) + (o.down_s - o.down_q);
}
std::size_t HipResidentExpert::accounted_bytes() const noexcept {
  return impl_ ? expert_blob_bytes(impl_->geom) : 0;
}
const std::uint8_t* HipResidentExpert::device_blob() const noexcept { return impl_ ? impl_->blob : nullptr; }
const osm_expert_geometry& HipResidentExpert::geometry() const noexcept {
  static const osm_expert_geometry none{};
  return impl_ ? impl_->geom : none;
}

HipDispatchResult HipResidentExpert::run_from_buffer(HipComputeContext& context,
                                                     const HipFloatBuffer& x) noexcept {
  HipDispatchResult r;
  if (!valid()) {
    r.diagnostic = "resident expert is not valid";
    return r;
  }
  if (!context.activate(&r.diagnostic)) return r;
  if (context.device() != impl_->device) {
    r.diagnostic = "resident expert belongs to a different device";
    return r;
  }
  if (!x.valid() || x.device() != impl_->device || x.size() != impl_->geom.hidden) {
    r.diagnostic = "resident expert input buffer is invalid or has wrong shape/device";
    return r;
  }
  if (!impl_->ensure_buffers(context, &r.diagnostic)) return r;
  const int rc = osmd_expert_forward(impl_->blob, impl_->geom, x.data(), impl_->hidden->data(),
                                     impl_->output->data(), context.stream());
  if (rc != 0) {
    r.diagnostic = hip_error("resident expert launch failed", rc);
    return r;
  }
  r.executed = true;
  r.diagnostic = "HIP resident expert output remains in its device buffer.";
  return r;
}

const HipFloatBuffer* HipResidentExpert::output_buffer() const noexcept {
  return (impl_ && impl_->output) ? &*impl_->output : nullptr;
}

HipValuesResult HipResidentExpert::run(HipComputeContext& context, std::span<const float> x) noexcept {
  HipValuesResult r;
  if (!valid()) {
    r.diagnostic = "resident expert is not valid";
    return r;
  }
  if (x.size() != impl_->geom.hidden) {
    r.diagnostic = "resident expert input size mismatch";
    return r;
  }
  if (!impl_->input) {
    impl_->input = HipFloatBuffer::create(context, impl_->geom.hidden, &r.diagnostic);
    if (!impl_->input) return r;
  }
  if (!impl_->input->upload(x, &r.diagnostic)) return r;
  const auto d = run_from_buffer(context, *impl_->input);
  if (!d.executed) {
    r.diagnostic = d.diagnostic;
    return r;
  }
  auto v = impl_->output->download(&r.diagnostic);
  if (!v) return r;
  r.values = std::move(*v);
  r.executed = true;
  r.diagnostic = "HIP resident expert executed through the reusable buffer path.";
  return r;
}

// ---- HipResidentSharedExpert -----------------------------------------------
struct HipResidentSharedExpert::Impl {
  std::optional<HipResidentExpert> expert;
  std::vector<float> scalar_gate;
  DeviceBytes scalar_gate_dev;
};

HipResidentSharedExpert::HipResidentSharedExpert() = default;
HipResidentSharedExpert::~HipResidentSharedExpert() = default;
HipResidentSharedExpert::HipResidentSharedExpert(HipResidentSharedExpert&&) noexcept = default;
HipResidentSharedExpert& HipResidentSharedExpert::operator=(HipResidentSharedExpert&&) noexcept = default;

std::optional<HipResidentSharedExpert> HipResidentSharedExpert::create(
    HipComputeContext& context, std::span<const std::byte> blob, const osm_expert_geometry& geometry,
    std::span<const float> scalar_gate, std::string* diagnostic) noexcept {
  try {
    if (scalar_gate.size() != geometry.hidden) {
      set_diag(diagnostic, "shared expert gate/up/down/scalar geometry mismatch");
      return std::nullopt;
    }
    auto impl = std::make_unique<Impl>();
    impl->expert = HipResidentExpert::create(context, blob, geometry, diagnostic);
    if (!impl->expert) return std::nullopt;
    impl->scalar_gate.assign(scalar_gate.begin(), scalar_gate.end());
    int rc = impl->scalar_gate_dev.allocate(scalar_gate.size_bytes());
    if (rc == 0) rc = osmd_memcpy_h2d(impl->scalar_gate_dev.get(), scalar_gate.data(), scalar_gate.size_bytes(), context.stream());
    if (rc == 0) rc = osmd_stream_synchronize(context.stream());
    if (rc != 0) {
      set_diag(diagnostic, hip_error("shared expert scalar gate upload failed", rc));
      return std::nullopt;
    }
    HipResidentSharedExpert s;
    s.impl_ = std::move(impl);
    set_diag(diagnostic, "HIP shared expert resident in HBM.");
    return s;
  } catch (const std::exception& e) {
    set_diag(diagnostic, std::string("shared expert creation exception: ") + e.what());
    return std::nullopt;
  }
}

bool HipResidentSharedExpert::valid() const noexcept { return impl_ && impl_->expert && impl_->expert->valid(); }
std::size_t HipResidentSharedExpert::input_dim() const noexcept { return valid() ? impl_->expert->input_dim() : 0; }
std::size_t HipResidentSharedExpert::intermediate_dim() const noexcept { return valid() ? impl_->expert->intermediate_dim() : 0; }
std::size_t HipResidentSharedExpert::output_dim() const noexcept { return valid() ? impl_->expert->output_dim() : 0; }
std::size_t HipResidentSharedExpert::accounted_bytes() const noexcept {
  return valid() ? impl_->expert->accounted_bytes() + impl_->scalar_gate_dev.size() : 0;
}
const std::uint8_t* HipResidentSharedExpert::device_blob() const noexcept { return valid() ? impl_->expert->device_blob() : nullptr; }
const float* HipResidentSharedExpert::device_scalar_gate() const noexcept { return valid() ? impl_->scalar_gate_dev.as<const float>() : nullptr; }
std::span<const float> HipResidentSharedExpert::scalar_gate() const noexcept {
  return valid() ? std::span<const float>(impl_->scalar_gate) : std::span<const float>();
}

std::optional<float> HipResidentSharedExpert::scalar_scale(std::span<const float> hidden,
                                                           std::string* diagnostic) const noexcept {
  if (!valid()) {
    set_diag(diagnostic, "shared expert is not valid");
    return std::nullopt;
  }
  if (hidden.size() != impl_->scalar_gate.size()) {
    set_diag(diagnostic, "shared expert scalar gate input size mismatch");
    return std::nullopt;
  }
  float logit = 0.0F;
  for (std::size_t i = 0; i < hidden.size(); ++i) {
    const float prod = impl_->scalar_gate[i] * hidden[i];
    logit = logit + prod;
  }
  const float scale = 1.0F / (1.0F + std::exp(-logit));
  if (!std::isfinite(scale)) {
    set_diag(diagnostic, "shared expert scalar gate is non-finite");
    return std::nullopt;
  }
  set_diag(diagnostic, "shared expert scalar gate computed");
  return scale;
}

HipDispatchResult HipResidentSharedExpert::run_from_buffer(HipComputeContext& context,
                                                           const HipFloatBuffer& hidden) noexcept {
  if (!valid()) return HipDispatchResult{false, "shared expert is not valid"};
  return impl_->expert->run_from_buffer(context, hidden);
}

const HipFloatBuffer* HipResidentSharedExpert::output_buffer() const noexcept {
  return valid() ? impl_->expert->output_buffer() : nullptr;
}

// ---- HipExpertSlab ---------------------------------------------------------
struct HipExpertSlab::Impl {
  osm_expert_geometry geom{};
  std::uint32_t layers = 0, experts = 0;
  std::size_t stride = 0;
  DeviceBytes mem;
  DeviceBytes table;  // [layers][experts] pointers
  osmd_stream stream = nullptr;
  int device = -1;
};

HipExpertSlab::HipExpertSlab() = default;
HipExpertSlab::~HipExpertSlab() = default;
HipExpertSlab::HipExpertSlab(HipExpertSlab&&) noexcept = default;
HipExpertSlab& HipExpertSlab::operator=(HipExpertSlab&&) noexcept = default;

std::optional<HipExpertSlab> HipExpertSlab::create(HipComputeContext& context,
                                                   const osm_expert_geometry& geometry,
                                                   std::uint32_t layers, std::uint32_t experts,
                                                   std::string* diagnostic) noexcept {
  try {
    if (!context.activate(diagnostic)) return std::nullopt;
    if (!check_expert_geometry(geometry, diagnostic)) return std::nullopt;
    if (layers == 0 || experts == 0) {
      set_diag(diagnostic, "expert slab needs at least one layer and one expert");
      return std::nullopt;
    }
    auto impl = std::make_unique<Impl>();
    impl->geom = geometry;
    impl->layers = layers;
    impl->experts = experts;
    impl->stride = expert_blob_bytes(geometry);
    std::size_t n = 0, bytes = 0;
    if (!mul_ok(layers, experts, n) || !mul_ok(n, impl->stride, bytes)) {
      set_diag(diagnostic, "expert slab size overflows");
      return std::nullopt;
    }
    int rc = impl->mem.allocate(bytes);
    if (rc != 0) {
      set_diag(diagnostic, hip_error("expert slab allocation failed", rc));
      return std::nullopt;
    }
    std::vector<const std::uint8_t*> ptrs(n);
    for (std::size_t i = 0; i < n; ++i) ptrs[i] = impl->mem.as<const std::uint8_t>() + i * impl->stride;
    rc = impl->table.allocate(n * sizeof(void*));
    if (rc == 0) rc = osmd_memcpy_h2d(impl->table.get(), ptrs.data(), n * sizeof(void*), context.stream());
    if (rc == 0) rc = osmd_stream_synchronize(context.stream());
    if (rc != 0) {
      set_diag(diagnostic, hip_error("expert slab table upload failed", rc));
      return std::nullopt;
    }
    impl->stream = context.stream();
    impl->device = context.device();
    HipExpertSlab s;
    s.impl_ = std::move(impl);
    return s;
  } catch (const std::exception& e) {
    set_diag(diagnostic, std::string("expert slab exception: ") + e.what());
    return std::nullopt;
  }
}

bool HipExpertSlab::valid() const noexcept { return impl_ && impl_->mem.get(); }
std::uint32_t HipExpertSlab::layers() const noexcept { return impl_ ? impl_->layers : 0; }
std::uint32_t HipExpertSlab::experts() const noexcept { return impl_ ? impl_->experts : 0; }
std::size_t HipExpertSlab::stride() const noexcept { return impl_ ? impl_->stride : 0; }
std::size_t HipExpertSlab::bytes() const noexcept { return impl_ ? impl_->mem.size() : 0; }
const osm_expert_geometry& HipExpertSlab::geometry() const noexcept {
  static const osm_expert_geometry none{};
  return impl_ ? impl_->geom : none;
}
std::uint8_t* HipExpertSlab::blob(std::uint32_t layer, std::uint32_t expert) const noexcept {
  if (!valid() || layer >= impl_->layers || expert >= impl_->experts) return nullptr;
  return impl_->mem.as<std::uint8_t>() +
         (static_cast<std::size_t>(layer) * impl_->experts + expert) * impl_->stride;
}
const std::uint8_t* const* HipExpertSlab::device_table(std::uint32_t layer) const noexcept {
  if (!valid() || layer >= impl_->layers) return nullptr;
  return impl_->table.as<const std::uint8_t* const>() + static_cast<std::size_t>(layer) * impl_->experts;
}

bool HipExpertSlab::upload(std::uint32_t layer, std::uint32_t expert, std::span<const std::byte> blob,
                           std::string* diagnostic) noexcept {
  std::uint8_t* dst = this->blob(layer, expert);
  if (dst == nullptr) return set_diag(diagnostic, "expert slab index out of range"), false;
  if (blob.size() != impl_->stride) return set_diag(diagnostic, "expert blob size mismatch"), false;
  int rc = osmd_set_device(impl_->device);
  if (rc == 0) rc = osmd_memcpy_h2d(dst, blob.data(), blob.size(), impl_->stream);
  if (rc == 0) rc = osmd_stream_synchronize(impl_->stream);
  if (rc != 0) return set_diag(diagnostic, hip_error("expert slab upload failed", rc)), false;
  return true;
}

bool HipExpertSlab::synthesize(std::uint64_t seed, std::string* diagnostic) noexcept {
  if (!valid()) return set_diag(diagnostic, "expert slab is not valid"), false;
  int rc = osmd_set_device(impl_->device);
  for (std::uint32_t l = 0; rc == 0 && l < impl_->layers; ++l)
    rc = osmd_synth_expert_blobs(seed, l, 0, impl_->experts, impl_->geom, blob(l, 0), impl_->stride,
                                 impl_->stream);
  if (rc == 0) rc = osmd_stream_synchronize(impl_->stream);
  if (rc != 0) return set_diag(diagnostic, hip_error("expert slab synthesis failed", rc)), false;
  return true;
}

}  // namespace osm
