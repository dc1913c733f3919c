// osm_hip.hpp -- C++20 host facade of the MI355X q4 routed-MoE path.
//
// Mirrors the reference's backend operator surface (include/orbi/streammoe/
// backend/vulkan_*.hpp, model/routed_moe.hpp, cache/expert_cache.hpp) with
// HIP-backed classes of the same shape: factories return std::optional and
// fill a diagnostic, operations are noexcept and return {executed,
// diagnostic}, invalid geometry is rejected before any launch. Everything
// below talks to the device only through the thin C ABI in
// csrc/device/osm_device.h.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <functional>
#include <memory>
#include <mutex>
#include <optional>
#include <set>
#include <span>
#include <string>
#include <string_view>
#include <tuple>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../device/osm_device.h"

namespace osm {

// ---- results (vulkan_float_buffer.hpp:15-18, vulkan_q4_gemv.hpp:15-19) ----
struct HipDispatchResult {
  bool executed{};
  std::string diagnostic;
};

struct HipValuesResult {
  bool executed{};
  std::vector<float> values;
  std::string diagnostic;
};

// ---- device memory (RAII over osmd_malloc) ---------------------------------
class DeviceBytes {
 public:
  DeviceBytes() = default;
  ~DeviceBytes();
  DeviceBytes(const DeviceBytes&) = delete;
  DeviceBytes& operator=(const DeviceBytes&) = delete;
  DeviceBytes(DeviceBytes&& o) noexcept;
  DeviceBytes& operator=(DeviceBytes&& o) noexcept;
  // Returns a HIP error code (0 on success).
  int allocate(std::size_t bytes);
  void reset() noexcept;
  void* get() const noexcept { return ptr_; }
  std::size_t size() const noexcept { return bytes_; }
  template <typename T>
  T* as() const noexcept { return static_cast<T*>(ptr_); }

 private:
  void* ptr_ = nullptr;
  std::size_t bytes_ = 0;
};

class PinnedBytes {
 public:
  PinnedBytes() = default;
  ~PinnedBytes();
  PinnedBytes(const PinnedBytes&) = delete;
  PinnedBytes& operator=(const PinnedBytes&) = delete;
  PinnedBytes(PinnedBytes&& o) noexcept;
  PinnedBytes& operator=(PinnedBytes&& o) noexcept;
  int allocate(std::size_t bytes);
  void reset() noexcept;
  void* get() const noexcept { return ptr_; }
  std::size_t size() const noexcept { return bytes_; }

 private:
  void* ptr_ = nullptr;
  std::size_t bytes_ = 0;
};

// ---- context (vulkan_compute_context.hpp:19-49) ---------------------------
// One device, one compute stream and one side stream for cache fills.
class HipComputeContext {
 public:
  HipComputeContext();
  ~HipComputeContext();
  HipComputeContext(const HipComputeContext&) = delete;
  HipComputeContext& operator=(const HipComputeContext&) = delete;
  HipComputeContext(HipComputeContext&&) noexcept;
  HipComputeContext& operator=(HipComputeContext&&) noexcept;

  // stream: nullptr for a stream the context creates and owns, else a
  // caller's stream on `device`, which every operator of the context is then
  // ordered on and which the caller keeps alive until the context is gone.
  [[nodiscard]] static std::optional<HipComputeContext> create(
      int device = 0, std::string* diagnostic = nullptr, osmd_stream stream = nullptr) noexcept;

  [[nodiscard]] bool valid() const noexcept;
  [[nodiscard]] int device() const noexcept;
  [[nodiscard]] const std::string& device_name() const noexcept;
  [[nodiscard]] osmd_stream stream() const noexcept;
  [[nodiscard]] osmd_stream copy_stream() const noexcept;
  // Makes this context's device current on the calling thread.
  [[nodiscard]] bool activate(std::string* diagnostic = nullptr) const noexcept;
  [[nodiscard]] bool synchronize(std::string* diagnostic = nullptr) const noexcept;
  // Device workspace of at least `bytes`, shared by every layer that runs on
  // this context's stream (the grouped path's buffers): one layer's work
  // finishes on the stream before the next layer's starts, so they never
  // overlap. It grows and never shrinks; an outgrown buffer stays allocated
  // until the context ends, so that graphs captured over it stay valid.
  // Returns nullptr (and the HIP error in *rc) when the allocation fails.
  [[nodiscard]] void* shared_workspace(std::size_t bytes, int* rc) noexcept;

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

// ---- float buffer (vulkan_float_buffer.hpp:23-58) -------------------------
class HipFloatBuffer {
 public:
  HipFloatBuffer();
  ~HipFloatBuffer();
  HipFloatBuffer(const HipFloatBuffer&) = delete;
  HipFloatBuffer& operator=(const HipFloatBuffer&) = delete;
  HipFloatBuffer(HipFloatBuffer&&) noexcept;
  HipFloatBuffer& operator=(HipFloatBuffer&&) noexcept;

  [[nodiscard]] static std::optional<HipFloatBuffer> create(
      HipComputeContext& context, std::size_t element_count,
      std::string* diagnostic = nullptr) noexcept;

  [[nodiscard]] bool valid() const noexcept;
  [[nodiscard]] std::size_t size() const noexcept;
  [[nodiscard]] std::size_t size_bytes() const noexcept;
  [[nodiscard]] int device() const noexcept;
  [[nodiscard]] float* data() const noexcept;

  // Stream-ordered on the context's compute stream; both wait for completion.
  [[nodiscard]] bool upload(std::span<const float> values,
                            std::string* diagnostic = nullptr) noexcept;
  [[nodiscard]] std::optional<std::vector<float>> download(
      std::string* diagnostic = nullptr) const noexcept;
  // Enqueued on the context's compute stream, returning before the copy
  // runs: `values` must stay valid (and unchanged, for an upload) until the
  // stream has passed it. Pinned host memory makes the copy a DMA that
  // overlaps the host; pageable memory is staged by the runtime.
  [[nodiscard]] bool upload_async(const float* values, std::size_t count,
                                  std::string* diagnostic = nullptr) noexcept;
  [[nodiscard]] bool download_async(float* values, std::size_t count,
                                    std::string* diagnostic = nullptr) const noexcept;

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

// ---- q4 projection weights (vulkan_q4_weights.hpp:19-55) ------------------
class HipQ4ProjectionWeights {
 public:
  HipQ4ProjectionWeights();
  ~HipQ4ProjectionWeights();
  HipQ4ProjectionWeights(const HipQ4ProjectionWeights&) = delete;
  HipQ4ProjectionWeights& operator=(const HipQ4ProjectionWeights&) = delete;
  HipQ4ProjectionWeights(HipQ4ProjectionWeights&&) noexcept;
  HipQ4ProjectionWeights& operator=(HipQ4ProjectionWeights&&) noexcept;

  // The reference's signature: fp32 scales and biases.
  [[nodiscard]] static std::optional<HipQ4ProjectionWeights> create(
      HipComputeContext& context, std::span<const std::uint32_t> packed,
      std::size_t out_dim, std::size_t packed_cols,
      std::span<const float> scales, std::span<const float> biases,
      std::size_t group_size, std::string* diagnostic = nullptr) noexcept;

  // Metadata kept in its stored dtype (bf16/f16/f32); meta_count entries each.
  [[nodiscard]] static std::optional<HipQ4ProjectionWeights> create_raw(
      HipComputeContext& context, std::span<const std::uint32_t> packed,
      std::size_t out_dim, std::size_t packed_cols, const void* scales,
      const void* biases, std::uint32_t meta_dtype, std::size_t group_size,
      std::string* diagnostic = nullptr) noexcept;

  [[nodiscard]] bool valid() const noexcept;
  [[nodiscard]] std::size_t out_dim() const noexcept;
  [[nodiscard]] std::size_t packed_cols() const noexcept;
  [[nodiscard]] std::size_t in_dim() const noexcept;
  [[nodiscard]] std::size_t group_size() const noexcept;
  [[nodiscard]] std::uint32_t meta_dtype() const noexcept;
  [[nodiscard]] std::size_t packed_size_bytes() const noexcept;
  [[nodiscard]] std::size_t meta_size_bytes() const noexcept;  // scales + biases
  [[nodiscard]] int device() const noexcept;
  [[nodiscard]] osmd_q4_proj view() const noexcept;

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

// ---- single operators ------------------------------------------------------
// vulkan_q4_dequant.hpp:23-30
[[nodiscard]] HipValuesResult run_hip_q4_dequant(
    HipComputeContext& context, std::span<const std::uint32_t> packed,
    std::size_t rows, std::size_t packed_cols, std::span<const float> scales,
    std::span<const float> biases, std::size_t group_size) noexcept;
// AffineQ4Projection (conversion/single_expert_pilot.hpp:32-42).
struct HipAffineQ4Projection {
  std::size_t rows{}, cols{}, packed_cols{}, groups_per_row{};
  std::vector<std::uint32_t> packed;
  std::vector<float> scales, biases;
  float max_abs_error{};
  double mean_abs_error{};
};
struct HipQuantizeResult {
  bool executed{};
  bool invalid_argument{};  // where the reference throws std::invalid_argument
  HipAffineQ4Projection projection;
  std::string diagnostic;
};
// quantize_affine_q4_rows (single_expert_pilot.cpp:276-358) on the device:
// bad geometry -> invalid_argument; a non-finite weight or an error above the
// group bound -> executed = false (the reference's std::runtime_error).
[[nodiscard]] HipQuantizeResult quantize_affine_q4_rows_hip(HipComputeContext& context,
                                                            std::span<const float> values,
                                                            std::size_t rows, std::size_t cols,
                                                            std::size_t group_size) noexcept;
// vulkan_q4_gemv.hpp:25-33
[[nodiscard]] HipValuesResult run_hip_q4_gemv(
    HipComputeContext& context, std::span<const std::uint32_t> packed,
    std::size_t out_dim, std::size_t packed_cols, std::span<const float> scales,
    std::span<const float> biases, std::size_t group_size,
    std::span<const float> x) noexcept;
// vulkan_q4_gemv.hpp:39-48
[[nodiscard]] HipDispatchResult run_hip_q4_gemv_buffers(
    HipComputeContext& context, std::span<const std::uint32_t> packed,
    std::size_t out_dim, std::size_t packed_cols, std::span<const float> scales,
    std::span<const float> biases, std::size_t group_size,
    const HipFloatBuffer& x, HipFloatBuffer& y) noexcept;
// vulkan_q4_gemv.hpp:53-57
[[nodiscard]] HipDispatchResult run_hip_q4_gemv_preloaded(
    HipComputeContext& context, const HipQ4ProjectionWeights& weights,
    const HipFloatBuffer& x, HipFloatBuffer& y) noexcept;
// vulkan_swiglu.hpp:19-30
[[nodiscard]] HipValuesResult run_hip_swiglu(HipComputeContext& context,
                                             std::span<const float> gate,
                                             std::span<const float> up) noexcept;
[[nodiscard]] HipDispatchResult run_hip_swiglu_buffers(
    HipComputeContext& context, const HipFloatBuffer& gate,
    const HipFloatBuffer& up, HipFloatBuffer& output) noexcept;
// vulkan_weighted_accumulate.hpp:12-16
[[nodiscard]] HipDispatchResult run_hip_weighted_accumulate(
    HipComputeContext& context, const HipFloatBuffer& source, float weight,
    HipFloatBuffer& accumulator) noexcept;
// vulkan_rmsnorm.hpp:25-31
[[nodiscard]] HipValuesResult run_hip_rms_norm(
    HipComputeContext& context, std::span<const float> input, std::size_t rows,
    std::size_t dim, std::span<const float> weight, float eps) noexcept;
// Nibble unpack (integer-exact check of the packed layout): out[8*w + j] is
// nibble j (low first) of word w.
[[nodiscard]] bool run_hip_unpack_nibbles(HipComputeContext& context,
                                          std::span<const std::uint32_t> packed,
                                          std::span<std::uint8_t> out,
                                          std::string* diagnostic = nullptr) noexcept;

// ---- experts (vulkan_resident_expert.hpp:41-69) ----------------------------
// Validates an expert geometry for the fused kernels.
[[nodiscard]] bool check_expert_geometry(const osm_expert_geometry& g,
                                         std::string* diagnostic) noexcept;
[[nodiscard]] std::size_t expert_blob_bytes(const osm_expert_geometry& g) noexcept;

class HipResidentExpert {
 public:
  HipResidentExpert();
  ~HipResidentExpert();
  HipResidentExpert(const HipResidentExpert&) = delete;
  HipResidentExpert& operator=(const HipResidentExpert&) = delete;
  HipResidentExpert(HipResidentExpert&&) noexcept;
  HipResidentExpert& operator=(HipResidentExpert&&) noexcept;

  // Copies the blob (qpack section order) into its own device allocation.
  [[nodiscard]] static std::optional<HipResidentExpert> create(
      HipComputeContext& context, std::span<const std::byte> blob,
      const osm_expert_geometry& geometry, std::string* diagnostic = nullptr) noexcept;
  // Non-owning view of a blob already in device memory (a cache slot).
  [[nodiscard]] static std::optional<HipResidentExpert> view(
      HipComputeContext& context, const std::uint8_t* device_blob,
      const osm_expert_geometry& geometry, std::string* diagnostic = nullptr) noexcept;

  [[nodiscard]] bool valid() const noexcept;
  [[nodiscard]] std::size_t input_dim() const noexcept;
  [[nodiscard]] std::size_t intermediate_dim() const noexcept;
  [[nodiscard]] std::size_t output_dim() const noexcept;
  [[nodiscard]] std::size_t packed_weight_bytes() const noexcept;
  // Bytes of HBM the expert's weights occupy (the blob; one cache slot).
  [[nodiscard]] std::size_t accounted_bytes() const noexcept;
  [[nodiscard]] const std::uint8_t* device_blob() const noexcept;
  [[nodiscard]] const osm_expert_geometry& geometry() const noexcept;

  [[nodiscard]] HipValuesResult run(HipComputeContext& context,
                                    std::span<const float> x) noexcept;
  [[nodiscard]] HipDispatchResult run_from_buffer(HipComputeContext& context,
                                                  const HipFloatBuffer& x) noexcept;
  // Valid until this expert is moved/destroyed or run again.
  [[nodiscard]] const HipFloatBuffer* output_buffer() const noexcept;

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

// ---- shared expert (vulkan_resident_shared_expert.hpp:49-69) --------------
class HipResidentSharedExpert {
 public:
  HipResidentSharedExpert();
  ~HipResidentSharedExpert();
  HipResidentSharedExpert(const HipResidentSharedExpert&) = delete;
  HipResidentSharedExpert& operator=(const HipResidentSharedExpert&) = delete;
  HipResidentSharedExpert(HipResidentSharedExpert&&) noexcept;
  HipResidentSharedExpert& operator=(HipResidentSharedExpert&&) noexcept;

  [[nodiscard]] static std::optional<HipResidentSharedExpert> create(
      HipComputeContext& context, std::span<const std::byte> blob,
      const osm_expert_geometry& geometry, std::span<const float> scalar_gate,
      std::string* diagnostic = nullptr) noexcept;

  [[nodiscard]] bool valid() const noexcept;
  [[nodiscard]] std::size_t input_dim() const noexcept;
  [[nodiscard]] std::size_t intermediate_dim() const noexcept;
  [[nodiscard]] std::size_t output_dim() const noexcept;
  [[nodiscard]] std::size_t accounted_bytes() const noexcept;
  [[nodiscard]] const std::uint8_t* device_blob() const noexcept;
  [[nodiscard]] const float* device_scalar_gate() const noexcept;
  [[nodiscard]] std::span<const float> scalar_gate() const noexcept;

  // sigmoid(scalar_gate . hidden), summed in index order on the host like
  // vulkan_resident_shared_expert.cpp:292-317.
  [[nodiscard]] std::optional<float> scalar_scale(
      std::span<const float> hidden, std::string* diagnostic = nullptr) const noexcept;
  [[nodiscard]] HipDispatchResult run_from_buffer(HipComputeContext& context,
                                                  const HipFloatBuffer& hidden) noexcept;
  [[nodiscard]] const HipFloatBuffer* output_buffer() const noexcept;

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

// ---- host L1 expert cache (cache/expert_cache.hpp:30-87) ------------------
struct ExpertId {
  std::uint32_t layer{};
  std::uint32_t expert{};
};

struct ExpertReadRequest {
  ExpertId id{};
  std::span<std::byte> destination{};
};

// storage/expert_storage.hpp:20-29: every destination is fully populated or
// the call throws.
class ExpertStorage {
 public:
  virtual ~ExpertStorage() = default;
  [[nodiscard]] virtual std::size_t expert_stride_bytes() const noexcept = 0;
  virtual void read_experts(std::span<ExpertReadRequest> requests) = 0;
};

// PosixPreadExpertStorage (storage/posix_pread_expert_storage.hpp:13-30):
// <dir>/packed_experts/layer_LL.bin holds layer LL's `experts` blobs at
// `stride`. Reads run in parallel; any failure or short read throws.
class PosixPreadExpertStorage final : public ExpertStorage {
 public:
  PosixPreadExpertStorage(std::filesystem::path container_dir, std::uint32_t layers, std::uint32_t experts,
                          std::size_t stride);
  ~PosixPreadExpertStorage() override;
  PosixPreadExpertStorage(const PosixPreadExpertStorage&) = delete;
  PosixPreadExpertStorage& operator=(const PosixPreadExpertStorage&) = delete;

  [[nodiscard]] std::size_t expert_stride_bytes() const noexcept override { return stride_; }
  void read_experts(std::span<ExpertReadRequest> requests) override;
  [[nodiscard]] static std::filesystem::path layer_path(const std::filesystem::path& dir, std::uint32_t layer);

 private:
  int fd_for_layer(std::uint32_t layer);
  std::filesystem::path dir_;
  std::uint32_t layers_, experts_;
  std::size_t stride_;
  std::vector<int> fds_;
  std::mutex mutex_;
};

// One entry of a qpack container's section table (container/qpack.hpp:15-21),
// as it applies to one expert's cache slot.
struct QpackSectionView {
  std::string_view name, dtype;  // "gate_proj.weight", "U32" / "F32" / "F16" / "BF16"
  std::uint32_t rank = 2;
  std::uint64_t rows = 0, cols = 0;
  std::uint64_t offset = 0, size = 0;  // within the slot, bytes
};
// Where each of the blob's nine sections comes from in the slot, in blob
// order; identity when the slot already is the blob.
struct QpackExpertPlan {
  std::array<std::uint64_t, 9> src{};
  std::array<std::size_t, 9> dst{};
  std::array<std::size_t, 9> bytes{};
  std::size_t blob_bytes = 0;
  bool identity = false;
};
// bind_qpack_q4_projection's checks (vulkan_qpack_expert.cpp:149-239) for
// the three projections against `g`; throws std::runtime_error (or
// std::invalid_argument for a metadata dtype other than the geometry's).
[[nodiscard]] QpackExpertPlan plan_qpack_expert(std::span<const QpackSectionView> sections,
                                                std::uint64_t slot_stride, const osm_expert_geometry& g);
void repack_qpack_expert(const QpackExpertPlan& plan, const std::byte* slot, std::byte* blob);

// The qpack container (container/qpack.hpp:15-90): manifest.json,
// packed_experts/layout.json and packed_experts/layer_LL.bin, parsed and
// validated as QpackReader does (container/qpack.cpp:41-247).
struct QpackSection {
  std::string name, dtype;
  std::vector<std::uint64_t> shape;
  std::uint64_t offset{}, size{};
};
struct QpackLayout {
  std::uint32_t expert_count{}, layer_count{};
  std::uint64_t expert_stride{};
  std::vector<QpackSection> sections;
  std::vector<bool> linear_layers;
  [[nodiscard]] const QpackSection* find_section(std::string_view name) const noexcept;
};
struct QpackManifest {
  std::string magic;
  std::uint32_t version{};
  std::string model_name, source_checkpoint;
  std::optional<std::uint32_t> quant_bits, quant_group_size;
  std::unordered_map<std::string, std::uint64_t> files;
};
class QpackReader {
 public:
  static constexpr std::string_view kMagic = "QPACK";
  static constexpr std::uint32_t kManifestVersion = 1;
  // Throws std::runtime_error for a container that fails a check.
  explicit QpackReader(std::filesystem::path container_dir);
  [[nodiscard]] const std::filesystem::path& container_dir() const noexcept { return dir_; }
  [[nodiscard]] const QpackManifest& manifest() const noexcept { return manifest_; }
  [[nodiscard]] const QpackLayout& layout() const noexcept { return layout_; }
  [[nodiscard]] std::filesystem::path layer_path(std::uint32_t layer) const;
  // One fixed-stride slot: std::out_of_range for a bad layer or expert,
  // std::invalid_argument for a destination under the stride,
  // std::runtime_error for an I/O failure or short read.
  void read_expert(std::uint32_t layer, std::uint32_t expert, std::span<std::byte> destination) const;

 private:
  std::filesystem::path dir_;
  QpackManifest manifest_;
  QpackLayout layout_;
};

// Expert reads from a qpack container. Without a geometry it is the
// reference's QpackExpertStorage (storage/qpack_expert_storage.cpp:8-33):
// whole slots of expertStride bytes. With one, each slot is bound by
// section name (plan_qpack_expert) and repacked into the blob's order on
// admission; the stride is then the blob's size. Reads go through pread,
// in parallel.
class QpackExpertStorage final : public ExpertStorage {
 public:
  explicit QpackExpertStorage(std::filesystem::path container_dir, const osm_expert_geometry* g = nullptr);
  [[nodiscard]] std::size_t expert_stride_bytes() const noexcept override;
  void read_experts(std::span<ExpertReadRequest> requests) override;
  [[nodiscard]] const QpackReader& reader() const noexcept { return reader_; }
  [[nodiscard]] bool repacks() const noexcept { return plan_.has_value() && !plan_->identity; }

 private:
  QpackReader reader_;
  std::optional<QpackExpertPlan> plan_;
  std::unique_ptr<PosixPreadExpertStorage> pread_;
};

struct ExpertCacheEntry {
  ExpertId id{};
  std::size_t slot{};
  std::span<const std::byte> bytes{};
};

struct ExpertCacheStats {
  std::size_t hits{};
  std::size_t misses{};
  std::size_t allocated_slots{};
  std::size_t capacity_slots{};
  std::size_t logical_bytes{};
  std::size_t budget_bytes{};
};

// Fixed-stride slots in pinned host memory (so a GPU fill from a slot is an
// asynchronous DMA), lazily grown up to budget/stride; LFU+recency victims;
// members of the current batch protected; rollback when the storage throws.
class HostExpertCache {
 public:
  HostExpertCache(ExpertStorage& storage, std::size_t budget_bytes,
                  std::size_t minimum_slots = 1, bool pinned = true);
  ~HostExpertCache();
  HostExpertCache(const HostExpertCache&) = delete;
  HostExpertCache& operator=(const HostExpertCache&) = delete;

  [[nodiscard]] std::vector<ExpertCacheEntry> fetch(
      std::uint32_t layer, std::span<const std::uint32_t> experts);
  [[nodiscard]] std::optional<std::size_t> resident_slot(
      std::uint32_t layer, std::uint32_t expert) const noexcept;
  [[nodiscard]] ExpertCacheStats stats() const noexcept;
  [[nodiscard]] std::size_t stride_bytes() const noexcept { return stride_; }
  [[nodiscard]] bool pinned() const noexcept { return pinned_; }

 private:
  struct SlotMeta {
    std::optional<std::uint64_t> key{};
    std::size_t frequency{};
    std::uint64_t last_use{};
  };
  std::byte* slot_data(std::size_t slot) const noexcept;
  std::size_t pick_fill_slot(const std::unordered_set<std::size_t>& in_batch);

  ExpertStorage& storage_;
  std::size_t stride_{};
  std::size_t budget_bytes_{};
  std::size_t max_slots_{};
  bool pinned_{};
  std::vector<std::byte*> slots_;
  std::vector<PinnedBytes> pinned_slots_;
  std::vector<std::vector<std::byte>> pageable_slots_;
  std::vector<SlotMeta> meta_;
  std::unordered_map<std::uint64_t, std::size_t> key_to_slot_;
  std::unordered_map<std::uint64_t, std::size_t> frequency_;
  std::uint64_t tick_{};
  std::size_t hits_{};
  std::size_t misses_{};
};

// ---- GPU resident cache policy (vulkan_resident_expert_cache.cpp:44-188) --
// The LFU+recency decision logic alone, separable so host tests can drive it
// without a device: key (layer<<32)|expert, one tick per get, per-key
// frequency history that survives eviction, victims by min (frequency,
// last_use, key) while resident + incoming > budget.
class LfuRecencyPolicy {
 public:
  explicit LfuRecencyPolicy(std::size_t budget_bytes);

  struct Outcome {
    bool hit{};
    std::vector<std::uint64_t> evicted;  // keys, in eviction order
  };
  // First half of a get: one tick, frequency history, and on a hit the
  // entry's (frequency, last_use) refresh. Returns true on a hit.
  [[nodiscard]] bool touch(std::uint32_t layer, std::uint32_t expert);
  // Second half of a miss, once the expert's bytes are in hand: evict until
  // it fits, then insert. Throws std::invalid_argument for zero or
  // over-budget sizes (the reference's "accounting is zero" / "exceeds the
  // configured budget"). Returns the evicted keys in eviction order.
  [[nodiscard]] std::vector<std::uint64_t> admit(std::uint32_t layer, std::uint32_t expert,
                                                 std::size_t accounted_bytes);
  // touch + admit on a miss.
  [[nodiscard]] Outcome access(std::uint32_t layer, std::uint32_t expert,
                               std::size_t accounted_bytes);
  // Undo the insertion of a key whose fill failed.
  void forget(std::uint64_t key) noexcept;
  [[nodiscard]] bool contains(std::uint32_t layer, std::uint32_t expert) const noexcept;
  // The keys a get of (layer, expert) would evict, in eviction order, with
  // nothing changed: none on a hit or when it fits (a get's tick and
  // frequency update touch no resident entry on a miss, so the victims are
  // the same after it).
  [[nodiscard]] std::vector<std::uint64_t> victims_of(std::uint32_t layer, std::uint32_t expert,
                                                      std::size_t accounted_bytes) const;
  [[nodiscard]] static std::uint64_t make_key(std::uint32_t layer,
                                              std::uint32_t expert) noexcept {
    return (static_cast<std::uint64_t>(layer) << 32U) | expert;
  }

  std::size_t hits{};
  std::size_t misses{};
  std::size_t loads{};
  std::size_t evictions{};
  [[nodiscard]] std::size_t resident_entries() const noexcept { return entries_.size(); }
  [[nodiscard]] std::size_t resident_bytes() const noexcept { return resident_bytes_; }
  [[nodiscard]] std::size_t budget_bytes() const noexcept { return budget_bytes_; }

 private:
  struct Node {
    std::size_t bytes{};
    std::size_t frequency{};
    std::uint64_t last_use{};
  };
  // Resident keys ordered by (frequency, last_use, key): the victim is the
  // first (vulkan_resident_expert_cache.cpp's scan for the smallest triple).
  using Rank = std::tuple<std::size_t, std::uint64_t, std::uint64_t>;
  [[nodiscard]] std::uint64_t victim() const;
  std::size_t budget_bytes_{};
  std::size_t resident_bytes_{};
  std::unordered_map<std::uint64_t, Node> entries_;
  std::set<Rank> order_;
  std::unordered_map<std::uint64_t, std::size_t> history_;
  std::uint64_t tick_{};
};

// ---- expert sources for cache fills ---------------------------------------
// Where a resident-cache miss copies its blob from: a host pointer to the
// expert's bytes (pinned memory makes the copy an asynchronous DMA).
class ExpertBlobSource {
 public:
  virtual ~ExpertBlobSource() = default;
  [[nodiscard]] virtual const osm_expert_geometry& geometry() const noexcept = 0;
  // Throws on failure; the pointer stays valid until the next call.
  [[nodiscard]] virtual const std::byte* host_blob(std::uint32_t layer,
                                                   std::uint32_t expert) = 0;
  // True when returned pointers stay valid after later calls, so a fill
  // may still be in flight when the next one starts.
  [[nodiscard]] virtual bool stable_pointers() const noexcept { return false; }
  // True when the returned memory is pinned and mapped for the device, so a
  // fill may be a kernel that reads it over PCIe itself.
  [[nodiscard]] virtual bool device_readable() const noexcept { return false; }
};

// Whole model (layers x experts blobs) in one pinned host allocation.
class PinnedExpertStore final : public ExpertBlobSource {
 public:
  PinnedExpertStore(const osm_expert_geometry& geometry, std::uint32_t layers,
                    std::uint32_t experts);
  [[nodiscard]] const osm_expert_geometry& geometry() const noexcept override { return geom_; }
  [[nodiscard]] const std::byte* host_blob(std::uint32_t layer, std::uint32_t expert) override;
  [[nodiscard]] bool stable_pointers() const noexcept override { return true; }
  [[nodiscard]] bool device_readable() const noexcept override { return true; }
  [[nodiscard]] std::byte* mutable_blob(std::uint32_t layer, std::uint32_t expert);
  [[nodiscard]] std::size_t stride() const noexcept { return stride_; }
  [[nodiscard]] std::uint32_t layers() const noexcept { return layers_; }
  [[nodiscard]] std::uint32_t experts() const noexcept { return experts_; }
  [[nodiscard]] std::byte* data() const noexcept { return static_cast<std::byte*>(mem_.get()); }

 private:
  osm_expert_geometry geom_{};
  std::uint32_t layers_{}, experts_{};
  std::size_t stride_{};
  PinnedBytes mem_;
};

// The reference's miss path: host L1 cache over an ExpertStorage
// (vulkan_resident_expert_cache.cpp:98-107).
class HostCacheSource final : public ExpertBlobSource {
 public:
  HostCacheSource(HostExpertCache& cache, const osm_expert_geometry& geometry);
  [[nodiscard]] const osm_expert_geometry& geometry() const noexcept override { return geom_; }
  [[nodiscard]] const std::byte* host_blob(std::uint32_t layer, std::uint32_t expert) override;
  [[nodiscard]] bool device_readable() const noexcept override { return cache_.pinned(); }

 private:
  HostExpertCache& cache_;
  osm_expert_geometry geom_{};
};

// ---- GPU resident expert cache (vulkan_resident_expert_cache.hpp:27-83) ----
struct HipResidentExpertCacheStats {
  std::size_t hits{};
  std::size_t misses{};
  std::size_t loads{};
  std::size_t evictions{};
  std::size_t resident_entries{};
  std::size_t resident_bytes{};
  std::size_t budget_bytes{};
};

// One HBM slab of budget/stride slots. A miss copies the blob from the source
// into a free or evicted slot on the context's side stream; the compute
// stream waits for that copy, so work enqueued after get() sees the expert,
// and the side stream waits for work enqueued before get(), so a slot is
// never overwritten while an earlier kernel may still read it.
class HipResidentExpertCache {
 public:
  // Throws std::invalid_argument for an invalid context or a zero budget
  // (vulkan_resident_expert_cache.cpp:18-35).
  HipResidentExpertCache(HipComputeContext& context, ExpertBlobSource& source,
                         std::size_t budget_bytes);
  ~HipResidentExpertCache();
  HipResidentExpertCache(const HipResidentExpertCache&) = delete;
  HipResidentExpertCache& operator=(const HipResidentExpertCache&) = delete;

  [[nodiscard]] HipResidentExpert* get(std::uint32_t layer, std::uint32_t expert,
                                       std::string* diagnostic = nullptr) noexcept;
  [[nodiscard]] HipValuesResult run(std::uint32_t layer, std::uint32_t expert,
                                    std::span<const float> x) noexcept;
  [[nodiscard]] bool contains(std::uint32_t layer, std::uint32_t expert) const noexcept;
  // Keys ((layer << 32) | expert) that get(layer, expert) would evict, with
  // no tick and no policy update (empty on a hit or when it fits).
  [[nodiscard]] std::vector<std::uint64_t> victims_of(std::uint32_t layer, std::uint32_t expert) const;
  // Device blob of a resident expert, or null; no tick, no policy update.
  [[nodiscard]] const std::uint8_t* resident_blob(std::uint32_t layer, std::uint32_t expert) const noexcept;
  [[nodiscard]] HipResidentExpertCacheStats stats() const noexcept;
  // Fill batch: the misses of the gets between the two calls are copied
  // back to back on the side stream, which waits once (at the first miss)
  // for the compute stream's earlier work; the compute stream waits once for
  // the copies, in end_fills (which returns the HIP status of that wait).
  // Work enqueued on the compute stream between the two calls must not read
  // the cache's slots.
  void begin_fills() noexcept;
  [[nodiscard]] int end_fills() noexcept;
  // Pipelined use, for a stack of layers enqueued without host waits:
  // between begin_pipeline and end_pipeline, the refill of a slot waits only
  // for the work that last read it (the event given to mark_readers), not
  // for everything enqueued on the compute stream, so one layer's fills
  // overlap the kernels of the layers before. end_pipeline is called once
  // the compute stream has drained (the events may then be destroyed).
  void begin_pipeline() noexcept;
  void mark_readers(std::uint32_t layer, std::uint32_t expert, osmd_event done) noexcept;
  void end_pipeline() noexcept;

  [[nodiscard]] std::size_t slot_count() const noexcept;
  [[nodiscard]] std::size_t stride() const noexcept;
  [[nodiscard]] std::uint64_t bytes_filled() const noexcept;

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

// ---- HBM-resident expert stack (all experts of several layers) -------------
class HipExpertSlab {
 public:
  HipExpertSlab();
  ~HipExpertSlab();
  HipExpertSlab(const HipExpertSlab&) = delete;
  HipExpertSlab& operator=(const HipExpertSlab&) = delete;
  HipExpertSlab(HipExpertSlab&&) noexcept;
  HipExpertSlab& operator=(HipExpertSlab&&) noexcept;

  [[nodiscard]] static std::optional<HipExpertSlab> create(
      HipComputeContext& context, const osm_expert_geometry& geometry,
      std::uint32_t layers, std::uint32_t experts,
      std::string* diagnostic = nullptr) noexcept;

  [[nodiscard]] bool valid() const noexcept;
  [[nodiscard]] std::uint32_t layers() const noexcept;
  [[nodiscard]] std::uint32_t experts() const noexcept;
  [[nodiscard]] std::size_t stride() const noexcept;
  [[nodiscard]] std::size_t bytes() const noexcept;
  [[nodiscard]] const osm_expert_geometry& geometry() const noexcept;
  [[nodiscard]] std::uint8_t* blob(std::uint32_t layer, std::uint32_t expert) const noexcept;
  [[nodiscard]] const std::uint8_t* const* device_table(std::uint32_t layer) const noexcept;
  [[nodiscard]] bool upload(std::uint32_t layer, std::uint32_t expert,
                            std::span<const std::byte> blob,
                            std::string* diagnostic = nullptr) noexcept;
  // Fills every expert with the seeded synthetic generator, on the device.
  [[nodiscard]] bool synthesize(std::uint64_t seed, std::string* diagnostic = nullptr) noexcept;

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

// ---- routed-MoE layer (checkpoint_sparse_moe.hpp + checkpoint_moe_sublayer.hpp)
struct HipMoeLayerConfig {
  osm_expert_geometry geometry{};
  std::uint32_t expert_count{};
  std::uint32_t top_k{};
  bool norm_topk_prob{true};
  bool has_shared_expert{true};
  float rms_eps{1e-6F};
};

struct HipMoeRouting {
  std::vector<std::uint32_t> ids;   // [tokens, top_k], picks by descending probability
  std::vector<float> weights;       // [tokens, top_k]
  std::vector<float> mass;          // [tokens] selected probability mass
  std::vector<float> shared_gate;   // [tokens]
  std::vector<float> logits;        // [tokens, expert_count]
};

struct HipMoeResult {
  bool executed{};
  HipMoeRouting routing;
  std::vector<float> normalized;  // [tokens, hidden] RMSNorm output (sublayer only)
  std::vector<float> values;      // [tokens, hidden]
  std::string diagnostic;
};

// Per-layer state that stays resident: router [E, D] and shared-expert gate
// vector [D] (bf16 or f32), optional RMSNorm weight, the shared expert, and
// scratch for up to max_tokens tokens.
// How a decode runs: the per-token kernels (router, gate/up, down; every
// token reads its picks' weights) or grouped GEMMs (tokens bucketed by
// expert, each expert's weights read once for all its tokens). automatic takes the per-token kernels, and the grouped path from
// kGroupedMinTokens tokens on, between the batch sizes where it was
// measured to overtake the per-token kernels at the Qwen3-Next shape on
// MI355X (us per layer, per-token vs grouped: 32 tokens 148-177 vs 176-182;
// 40: 201-207 vs 198; 48: 213-218 vs 211; 64: 266-272 vs 239; 512: 2730 vs
// 387).
enum class HipMoePath { automatic = 0, per_token = 1, grouped = 2 };
inline constexpr std::uint32_t kGroupedMinTokens = 40;

class HipMoeLayer {
 public:
  HipMoeLayer();
  ~HipMoeLayer();
  HipMoeLayer(const HipMoeLayer&) = delete;
  HipMoeLayer& operator=(const HipMoeLayer&) = delete;
  HipMoeLayer(HipMoeLayer&&) noexcept;
  HipMoeLayer& operator=(HipMoeLayer&&) noexcept;

  // router / shared_gate_vec are in router_dtype (OSM_META_F32 or BF16/F16
  // bits); norm_weight may be empty (no RMSNorm); shared_blob may be empty
  // when config.has_shared_expert is false.
  [[nodiscard]] static std::optional<HipMoeLayer> create(
      HipComputeContext& context, const HipMoeLayerConfig& config,
      const void* router, std::uint32_t router_dtype, const void* shared_gate_vec,
      std::span<const float> norm_weight, std::span<const std::byte> shared_blob,
      std::uint32_t max_tokens, std::string* diagnostic = nullptr) noexcept;

  [[nodiscard]] bool valid() const noexcept;
  [[nodiscard]] const HipMoeLayerConfig& config() const noexcept;
  [[nodiscard]] std::uint32_t max_tokens() const noexcept;
  [[nodiscard]] const std::uint8_t* shared_blob() const noexcept;

  // Stream-ordered decode of `tokens` rows of device x into device y with
  // every routed expert resolved through `expert_table` (device, [E]).
  // sublayer=true: y = x + MoE(RMSNorm(x)); false: y = MoE(x).
  [[nodiscard]] HipDispatchResult decode_device(HipComputeContext& context,
                                                const float* x, float* y,
                                                std::uint32_t tokens,
                                                const std::uint8_t* const* expert_table,
                                                bool sublayer) noexcept;
  // decode_device through the per-token kernels with the routing workspace
  // (logits, picks, normalised input, h, slot pointers) in the library's
  // fixed per-device array instead of the layer's: no device memory is
  // allocated or freed. Returns 0 or an osm_status; *diagnostic (static
  // text) says why on failure, e.g. `tokens` beyond what the array holds
  // (static_tokens_capacity). Calls on one device share the array, so calls
  // that overlap in time on one device (two streams) race.
  [[nodiscard]] int decode_device_static(HipComputeContext& context, const float* x, float* y,
                                         std::uint32_t tokens, const std::uint8_t* const* expert_table,
                                         bool sublayer, const char** diagnostic) noexcept;
  [[nodiscard]] std::uint32_t static_tokens_capacity() const noexcept;
  // False (path unchanged) for a value that names no path.
  bool set_path(HipMoePath path, std::string* diagnostic = nullptr) noexcept;
  [[nodiscard]] HipMoePath path() const noexcept;
  // A prefill chunk in bf16 ([tokens, D], device) through the grouped path:
  // bf16 router, MoE form (no RMSNorm / residual), y fp32 [tokens, D].
  [[nodiscard]] HipDispatchResult prefill_device_bf16(HipComputeContext& context,
                                                      const std::uint16_t* x_bf16, float* y,
                                                      std::uint32_t tokens,
                                                      const std::uint8_t* const* expert_table) noexcept;
  // One kernel of a decode (0 router GEMV, 1 selection + gate/up + SwiGLU,
  // 2 down + weighted accumulate), for per-kernel timing; 1 and 2 read the
  // workspace the previous kernels of this layer left.
  [[nodiscard]] HipDispatchResult launch_phase(HipComputeContext& context, const float* x,
                                               float* y, std::uint32_t tokens,
                                               const std::uint8_t* const* expert_table,
                                               bool sublayer, int phase) noexcept;
  // Host in/out variant that also returns the routing of every token.
  [[nodiscard]] HipMoeResult run(HipComputeContext& context,
                                 std::span<const float> hidden, std::uint32_t tokens,
                                 const std::uint8_t* const* expert_table,
                                 bool sublayer) noexcept;
  // Routing outputs of the last decode (device pointers).
  [[nodiscard]] const std::uint32_t* device_ids() const noexcept;
  [[nodiscard]] bool download_routing(HipComputeContext& context, std::uint32_t tokens,
                                      HipMoeRouting& out,
                                      std::string* diagnostic = nullptr) const noexcept;
  // False after decode_device_static (its routing sits in the shared fixed
  // workspace, which later calls overwrite), true after any other decode.
  [[nodiscard]] bool routing_queryable() const noexcept;
  // The routing counters of every selection since creation or the last
  // reset: selections, selections that took the exact path, exact paths that
  // recomputed every expert, and unresolved adjacent picks. Synchronises the
  // context's stream; reset zeroes them afterwards.
  [[nodiscard]] bool routing_stats(HipComputeContext& context, std::uint32_t (&out)[4], bool reset,
                                   std::string* diagnostic = nullptr) noexcept;
  // The RMSNorm output (sublayer form) or the input (MoE form) of the last
  // per-token decode, or the normalised input of the last grouped sublayer.
  [[nodiscard]] bool download_normalized(HipComputeContext& context, std::uint32_t tokens,
                                         std::vector<float>& out,
                                         std::string* diagnostic = nullptr) const noexcept;

 private:
  friend struct MoeLayerAccess;
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

// One decode step through a stack of MoE layers, each with its device expert
// table (checkpoint_decoder_stack.cpp:191-204 runs the layers in order).
// chained: layer i + 1 reads what layer i wrote, each layer a sublayer
// y = x + MoE(RMSNorm(x)), ping-ponging through scratch so the last layer
// lands in y. Otherwise every layer decodes its own `tokens` rows:
// x + i * tokens * D into y + i * tokens * D.
struct HipDecodeStep {
  std::vector<HipMoeLayer*> layers;
  std::vector<const std::uint8_t* const*> tables;
  const float* x = nullptr;
  float* y = nullptr;
  float* scratch = nullptr;
  std::uint32_t tokens = 1;
  bool chained = false;
};

[[nodiscard]] HipDispatchResult enqueue_decode_step(HipComputeContext& context,
                                                    const HipDecodeStep& step) noexcept;

// Work recorded once from the context's compute stream into a HIP graph and
// replayed with one submission: the same kernels on the same buffers every
// launch, without the per-launch host and queue overhead. Only enqueue-only
// operations may run between begin_capture and end_capture (no
// synchronisation, no host copies, no memsets).
class HipGraph {
 public:
  HipGraph() = default;
  ~HipGraph();
  HipGraph(const HipGraph&) = delete;
  HipGraph& operator=(const HipGraph&) = delete;
  HipGraph(HipGraph&& o) noexcept;
  HipGraph& operator=(HipGraph&& o) noexcept;

  [[nodiscard]] static bool begin_capture(HipComputeContext& context,
                                          std::string* diagnostic = nullptr) noexcept;
  // Ends the capture begun on this context's stream (always) and
  // instantiates what was recorded.
  [[nodiscard]] static std::optional<HipGraph> end_capture(HipComputeContext& context,
                                                           std::string* diagnostic = nullptr) noexcept;
  // One decode step, captured.
  [[nodiscard]] static std::optional<HipGraph> capture_decode_step(HipComputeContext& context,
                                                                   const HipDecodeStep& step,
                                                                   std::string* diagnostic = nullptr) noexcept;
  [[nodiscard]] bool valid() const noexcept { return exec_ != nullptr; }
  [[nodiscard]] HipDispatchResult launch(HipComputeContext& context) noexcept;

 private:
  osmd_graph exec_ = nullptr;
  int device_ = -1;
};

// routed_moe.hpp:58-65 -- tokens through the resident cache: route on the
// device, make every pick resident in pick order (misses filled on the side
// streams), then the expert kernels. The cache decides residency on the host
// from the routed ids, as the reference's cache does. When the budget cannot
// hold a call's picks at once they run in rounds, each just before a get
// would evict one of its picks (the reference runs each pick right after its
// get, routed_moe.cpp:320-366); with device routing, picks already resident
// run while the misses are copied. Outputs have the bits of the fused
// kernels whatever the split.
// picks: null, or caller-chosen routed experts ([tokens, top_k] ids and
// weights) that replace the router's picks. The router alone then runs for
// the shared gate (and the logits and RMSNorm); routing returns the given
// ids and weights, and their sum as the mass. No counterpart in the
// reference, whose routed MoE always routes itself: it drives the cache with
// an external routing trace.
struct HipMoePicks {
  const std::uint32_t* ids = nullptr;
  const float* weights = nullptr;
};
[[nodiscard]] HipMoeResult run_qwen_sparse_moe_hip(
    HipComputeContext& context, HipResidentExpertCache& expert_cache,
    HipMoeLayer& layer_state, std::uint32_t layer, std::span<const float> hidden,
    bool sublayer, const HipMoePicks* picks = nullptr) noexcept;

// The decoder stack's layer loop (checkpoint_decoder_stack.cpp:191-204) as
// chained MoE sublayers over the capped cache. The activations stay on the
// device between layers and each layer's fills wait only for the kernels
// that last read the slots they overwrite. With every layer's picks given
// (ids and weights [n][tokens][k], both null otherwise) no layer waits for
// the host, so fills overlap earlier layers' kernels; with device routing
// each layer's ids come back to the host, which decides residency. Every
// output is the bits of run_qwen_sparse_moe_hip called layer by layer, in
// rounds or not. y = the last layer's output [tokens][D] (host). Returns
// false with a diagnostic.
[[nodiscard]] bool run_cached_stack(HipComputeContext& context, HipResidentExpertCache& expert_cache,
                                    std::span<HipMoeLayer* const> layers, const std::uint32_t* cache_layers,
                                    std::span<const float> x, const std::uint32_t* pick_ids,
                                    const float* pick_weights, float* y, std::string* diagnostic) noexcept;

}  // namespace osm
