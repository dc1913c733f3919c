// runtime.cpp -- device/pinned memory, the compute context and float buffers
// (the HIP counterparts of vulkan_compute_context.cpp and
// vulkan_float_buffer.cpp).
#include <cstring>
#include <string>
#include <vector>
#include <utility>

#include "host_util.hpp"
#include "osm_hip.hpp"

namespace osm {

// ---- DeviceBytes / PinnedBytes ---------------------------------------------
DeviceBytes::~DeviceBytes() { reset(); }
DeviceBytes::DeviceBytes(DeviceBytes&& o) noexcept
    : ptr_(std::exchange(o.ptr_, nullptr)), bytes_(std::exchange(o.bytes_, 0)) {}
DeviceBytes& DeviceBytes::operator=(DeviceBytes&& o) noexcept {
  if (this != &o) {
    reset();
    ptr_ = std::exchange(o.ptr_, nullptr);
    bytes_ = std::exchange(o.bytes_, 0);
  }
  return *this;
}
int DeviceBytes::allocate(std::size_t bytes) {
  reset();
  if (bytes == 0) return 0;
  const int rc = osmd_malloc(&ptr_, bytes);
  if (rc != 0) {
    ptr_ = nullptr;
    return rc;
  }
  bytes_ = bytes;
  return 0;
}
void DeviceBytes::reset() noexcept {
  if (ptr_ != nullptr) osmd_free(ptr_);
  ptr_ = nullptr;
  bytes_ = 0;
}

PinnedBytes::~PinnedBytes() { reset(); }
PinnedBytes::PinnedBytes(PinnedBytes&& o) noexcept
    : ptr_(std::exchange(o.ptr_, nullptr)), bytes_(std::exchange(o.bytes_, 0)) {}
PinnedBytes& PinnedBytes::operator=(PinnedBytes&& o) noexcept {
  if (this != &o) {
    reset();
    ptr_ = std::exchange(o.ptr_, nullptr);
    bytes_ = std::exchange(o.bytes_, 0);
  }
  return *this;
}
int PinnedBytes::allocate(std::size_t bytes) {
  reset();
  if (bytes == 0) return 0;
  const int rc = osmd_host_malloc(&ptr_, bytes);
  if (rc != 0) {
    ptr_ = nullptr;
    return rc;
  }
  bytes_ = bytes;
  return 0;
}
void PinnedBytes::reset() noexcept {
  if (ptr_ != nullptr) osmd_host_free(ptr_);
  ptr_ = nullptr;
  bytes_ = 0;
}

// ---- HipComputeContext -----------------------------------------------------
struct HipComputeContext::Impl {
  int device = -1;
  std::string name;
  osmd_stream stream = nullptr;
  osmd_stream copy = nullptr;
  bool owns_stream = true;  // false: a caller's stream, left alive
  DeviceBytes workspace;
  std::vector<DeviceBytes> outgrown;  // kept for graphs captured over them
  ~Impl() {
    outgrown.clear();
    workspace.reset();
    if (device >= 0) osmd_set_device(device);
    if (copy) osmd_stream_destroy(copy);
    if (stream && owns_stream) osmd_stream_destroy(stream);
  }
};

void* HipComputeContext::shared_workspace(std::size_t bytes, int* rc) noexcept {
  if (rc) *rc = 0;
  if (!impl_) {
    if (rc) *rc = 1;
    return nullptr;
  }
  if (impl_->workspace.get() != nullptr && impl_->workspace.size() >= bytes) return impl_->workspace.get();
  try {
    DeviceBytes grown;
    const int r = grown.allocate(bytes);
    if (r != 0) {
      if (rc) *rc = r;
      return nullptr;
    }
    if (impl_->workspace.get() != nullptr) impl_->outgrown.push_back(std::move(impl_->workspace));
    impl_->workspace = std::move(grown);
    return impl_->workspace.get();
  } catch (...) {
    if (rc) *rc = 2;
    return nullptr;
  }
}

HipComputeContext::HipComputeContext() = default;
HipComputeContext::~HipComputeContext() = default;
HipComputeContext::HipComputeContext(HipComputeContext&&) noexcept = default;
HipComputeContext& HipComputeContext::operator=(HipComputeContext&&) noexcept = default;

std::optional<HipComputeContext> HipComputeContext::create(int device, std::string* diagnostic,
                                                           osmd_stream stream) noexcept {
  try {
    int count = 0;
    int rc = osmd_device_count(&count);
    if (rc != 0 || count <= 0) {
      set_diag(diagnostic, "no HIP device available" +
                               (rc != 0 ? std::string(": ") + osmd_error_string(rc) : std::string()));
      return std::nullopt;
    }
    if (device < 0 || device >= count) {
      set_diag(diagnostic, "HIP device index out of range");
      return std::nullopt;
    }
    if ((rc = osmd_set_device(device)) != 0) {
      set_diag(diagnostic, std::string("hipSetDevice failed: ") + osmd_error_string(rc));
      return std::nullopt;
    }
    if (stream != nullptr) {
      int on = -1;
      if ((rc = osmd_stream_device(stream, &on)) != 0) {
        set_diag(diagnostic, std::string("the caller's stream cannot be queried: ") + osmd_error_string(rc));
        return std::nullopt;
      }
      if (on != device) {
        set_diag(diagnostic, "the caller's stream belongs to device " + std::to_string(on) + ", not " +
                                 std::to_string(device));
        return std::nullopt;
      }
    }
    auto impl = std::make_unique<Impl>();
    impl->device = device;
    char name[256] = {0};
    if (osmd_device_name(device, name, sizeof(name)) == 0) impl->name = name;
    impl->owns_stream = stream == nullptr;
    impl->stream = stream;
    if ((stream == nullptr && (rc = osmd_stream_create(&impl->stream)) != 0) ||
        (rc = osmd_stream_create(&impl->copy)) != 0) {
      set_diag(diagnostic, std::string("stream creation failed: ") + osmd_error_string(rc));
      return std::nullopt;
    }
    // The no-allocation decode's fixed workspace: its address on this device,
    // looked up once with the device current. A failure here is not fatal;
    // that entry point looks it up again and reports the error itself.
    (void)osmd_static_scratch_init(device);
    HipComputeContext ctx;
    ctx.impl_ = std::move(impl);
    set_diag(diagnostic, "HIP compute context created");
    return ctx;
  } catch (const std::exception& e) {
    set_diag(diagnostic, std::string("context creation exception: ") + e.what());
    return std::nullopt;
  }
}

bool HipComputeContext::valid() const noexcept { return impl_ && impl_->stream && impl_->copy; }
int HipComputeContext::device() const noexcept { return impl_ ? impl_->device : -1; }
const std::string& HipComputeContext::device_name() const noexcept {
  static const std::string empty;
  return impl_ ? impl_->name : empty;
}
osmd_stream HipComputeContext::stream() const noexcept { return impl_ ? impl_->stream : nullptr; }
osmd_stream HipComputeContext::copy_stream() const noexcept { return impl_ ? impl_->copy : nullptr; }

bool HipComputeContext::activate(std::string* diagnostic) const noexcept {
  if (!valid()) return set_diag(diagnostic, "HIP compute context is not valid"), false;
  const int rc = osmd_set_device(impl_->device);
  if (rc != 0) return set_diag(diagnostic, std::string("hipSetDevice failed: ") + osmd_error_string(rc)), false;
  return true;
}

bool HipComputeContext::synchronize(std::string* diagnostic) const noexcept {
  if (!activate(diagnostic)) return false;
  int rc = osmd_stream_synchronize(impl_->copy);
  if (rc == 0) rc = osmd_stream_synchronize(impl_->stream);
  if (rc != 0) return set_diag(diagnostic, std::string("stream synchronize failed: ") + osmd_error_string(rc)), false;
  return true;
}

// ---- HipFloatBuffer --------------------------------------------------------
struct HipFloatBuffer::Impl {
  DeviceBytes mem;
  std::size_t count = 0;
  int device = -1;
  osmd_stream stream = nullptr;
};

HipFloatBuffer::HipFloatBuffer() = default;
HipFloatBuffer::~HipFloatBuffer() = default;
HipFloatBuffer::HipFloatBuffer(HipFloatBuffer&&) noexcept = default;
HipFloatBuffer& HipFloatBuffer::operator=(HipFloatBuffer&&) noexcept = default;

std::optional<HipFloatBuffer> HipFloatBuffer::create(HipComputeContext& context,
                                                     std::size_t element_count,
                                                     std::string* diagnostic) noexcept {
  try {
    if (!context.activate(diagnostic)) return std::nullopt;
    if (element_count == 0) {
      set_diag(diagnostic, "float buffer element count must be non-zero");
      return std::nullopt;
    }
    auto impl = std::make_unique<Impl>();
    const int rc = impl->mem.allocate(element_count * sizeof(float));
    if (rc != 0) {
      set_diag(diagnostic, std::string("float buffer allocation failed: ") + osmd_error_string(rc));
      return std::nullopt;
    }
    impl->count = element_count;
    impl->device = context.device();
    impl->stream = context.stream();
    HipFloatBuffer b;
    b.impl_ = std::move(impl);
    return b;
  } catch (const std::exception& e) {
    set_diag(diagnostic, std::string("float buffer exception: ") + e.what());
    return std::nullopt;
  }
}

bool HipFloatBuffer::valid() const noexcept { return impl_ && impl_->mem.get() != nullptr; }
std::size_t HipFloatBuffer::size() const noexcept { return impl_ ? impl_->count : 0; }
std::size_t HipFloatBuffer::size_bytes() const noexcept { return size() * sizeof(float); }
int HipFloatBuffer::device() const noexcept { return impl_ ? impl_->device : -1; }
float* HipFloatBuffer::data() const noexcept { return impl_ ? impl_->mem.as<float>() : nullptr; }

bool HipFloatBuffer::upload(std::span<const float> values, std::string* diagnostic) noexcept {
  if (!valid()) return set_diag(diagnostic, "float buffer is not valid"), false;
  if (values.size() != impl_->count)
    return set_diag(diagnostic, "float buffer upload size mismatch"), false;
  int rc = osmd_set_device(impl_->device);
  if (rc == 0) rc = osmd_memcpy_h2d(impl_->mem.get(), values.data(), values.size_bytes(), impl_->stream);
  if (rc == 0) rc = osmd_stream_synchronize(impl_->stream);
  if (rc != 0) return set_diag(diagnostic, std::string("float buffer upload failed: ") + osmd_error_string(rc)), false;
  return true;
}

bool HipFloatBuffer::upload_async(const float* values, std::size_t count, std::string* diagnostic) noexcept {
  if (!valid()) return set_diag(diagnostic, "float buffer is not valid"), false;
  if (count != impl_->count) return set_diag(diagnostic, "float buffer upload size mismatch"), false;
  int rc = osmd_set_device(impl_->device);
  if (rc == 0) rc = osmd_memcpy_h2d(impl_->mem.get(), values, size_bytes(), impl_->stream);
  if (rc != 0) return set_diag(diagnostic, std::string("float buffer upload failed: ") + osmd_error_string(rc)), false;
  return true;
}

bool HipFloatBuffer::download_async(float* values, std::size_t count, std::string* diagnostic) const noexcept {
  if (!valid()) return set_diag(diagnostic, "float buffer is not valid"), false;
  if (count != impl_->count) return set_diag(diagnostic, "float buffer download size mismatch"), false;
  int rc = osmd_set_device(impl_->device);
  if (rc == 0) rc = osmd_memcpy_d2h(values, impl_->mem.get(), size_bytes(), impl_->stream);
  if (rc != 0) return set_diag(diagnostic, std::string("float buffer download failed: ") + osmd_error_string(rc)), false;
  return true;
}

std::optional<std::vector<float>> HipFloatBuffer::download(std::string* diagnostic) const noexcept {
  try {
    if (!valid()) {
      set_diag(diagnostic, "float buffer is not valid");
      return std::nullopt;
    }
    std::vector<float> out(impl_->count);
    int rc = osmd_set_device(impl_->device);
    if (rc == 0) rc = osmd_memcpy_d2h(out.data(), impl_->mem.get(), size_bytes(), impl_->stream);
    if (rc == 0) rc = osmd_stream_synchronize(impl_->stream);
    if (rc != 0) {
      set_diag(diagnostic, std::string("float buffer download failed: ") + osmd_error_string(rc));
      return std::nullopt;
    }
    return out;
  } catch (const std::exception& e) {
    set_diag(diagnostic, std::string("float buffer download exception: ") + e.what());
    return std::nullopt;
  }
}

}  // namespace osm
