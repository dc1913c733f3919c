// cache.cpp -- the two cache levels of the expert path:
//   HostExpertCache        host L1 slot cache over an ExpertStorage
//                          (policy of src/cache/expert_cache.cpp)
//   LfuRecencyPolicy       GPU-resident policy
//                          (src/backend/vulkan_resident_expert_cache.cpp:44-188)
//   HipResidentExpertCache one HBM slab of expert slots driven by that policy,
//                          filled from an ExpertBlobSource on a side stream.
#include <array>
#include <limits>
#include <stdexcept>
#include <string>
#include <tuple>
#include <utility>

#include "host_util.hpp"
#include "osm_hip.hpp"

namespace osm {
namespace {

std::uint64_t key_of(std::uint32_t layer, std::uint32_t expert) {
  return (static_cast<std::uint64_t>(layer) << 32U) | expert;
}

// Workgroups of a fill kernel that reads a pinned source over PCIe: 32 keep
// enough 16-byte reads in flight for the link (a 1.77 MB expert moved at
// 52 GB/s, against 44 GB/s for the DMA engine's per-expert copies); wider
// grids only contend (512 workgroups: 40 GB/s).
constexpr unsigned kFillBlocks = 32;

// Streams a fill batch's copies rotate over: the context's side stream and
// kFillStreams - 1 of the cache's own. Two fill kernels in flight keep the
// link busiest: with three or four, the capped 48-layer decode took 117.6 and
// 122.2 us per token-layer against 109.5.
constexpr std::uint32_t kFillStreams = 2;

}  // namespace

// ---- HostExpertCache -------------------------------------------------------
HostExpertCache::HostExpertCache(ExpertStorage& storage, std::size_t budget_bytes,
                                 std::size_t minimum_slots, bool pinned)
    : storage_(storage),
      stride_(storage.expert_stride_bytes()),
      budget_bytes_(budget_bytes),
      pinned_(pinned) {
  if (stride_ == 0) throw std::invalid_argument("expert cache: storage stride must be non-zero");
  max_slots_ = budget_bytes_ / stride_;
  if (max_slots_ < minimum_slots)
    throw std::invalid_argument("expert cache: budget cannot satisfy minimum slot count");
  slots_.reserve(max_slots_);
  meta_.reserve(max_slots_);
}

HostExpertCache::~HostExpertCache() = default;

std::byte* HostExpertCache::slot_data(std::size_t slot) const noexcept { return slots_[slot]; }

// A never-used slot first (lazy growth up to the budget), then the slot with
// the smallest (frequency, last_use, slot) outside the current batch
// (expert_cache.cpp:50-99).
std::size_t HostExpertCache::pick_fill_slot(const std::unordered_set<std::size_t>& in_batch) {
  if (slots_.size() < max_slots_) {
    std::byte* p = nullptr;
    if (pinned_) {
      PinnedBytes mem;
      const int rc = mem.allocate(stride_);
      if (rc != 0) throw std::runtime_error(hip_error("expert cache: pinned slot allocation failed", rc));
      p = static_cast<std::byte*>(mem.get());
      pinned_slots_.push_back(std::move(mem));
    } else {
      pageable_slots_.emplace_back(stride_);
      p = pageable_slots_.back().data();
    }
    slots_.push_back(p);
    meta_.push_back({});
    return slots_.size() - 1;
  }
  for (std::size_t s = 0; s < meta_.size(); ++s)
    if (!meta_[s].key.has_value()) return s;
  std::size_t best_slot = std::numeric_limits<std::size_t>::max();
  auto best = std::make_tuple(std::numeric_limits<std::size_t>::max(),
                              std::numeric_limits<std::uint64_t>::max(),
                              std::numeric_limits<std::size_t>::max());
  for (std::size_t s = 0; s < meta_.size(); ++s) {
    if (in_batch.count(s)) continue;
    const auto score = std::make_tuple(meta_[s].frequency, meta_[s].last_use, s);
    if (score < best) {
      best = score;
      best_slot = s;
    }
  }
  if (best_slot == std::numeric_limits<std::size_t>::max())
    throw std::runtime_error("expert cache: batch requires more simultaneous slots than budget allows");
  return best_slot;
}

std::vector<ExpertCacheEntry> HostExpertCache::fetch(std::uint32_t layer,
                                                     std::span<const std::uint32_t> experts) {
  if (experts.empty()) return {};
  {
    std::unordered_set<std::uint64_t> distinct;
    for (auto e : experts) distinct.insert(key_of(layer, e));
    if (distinct.size() > max_slots_)
      throw std::runtime_error("expert cache: request contains more distinct experts than cache slots");
  }
  ++tick_;
  std::unordered_set<std::size_t> in_batch;
  std::vector<std::size_t> chosen;
  chosen.reserve(experts.size());
  std::vector<std::pair<std::size_t, std::uint32_t>> fills;
  for (const auto e : experts) {
    const std::uint64_t key = key_of(layer, e);
    const std::size_t f = frequency_[key] + 1U;
    frequency_[key] = f;
    if (auto it = key_to_slot_.find(key); it != key_to_slot_.end()) {
      ++hits_;
      meta_[it->second].frequency = f;
      meta_[it->second].last_use = tick_;
      in_batch.insert(it->second);
      chosen.push_back(it->second);
      continue;
    }
    ++misses_;
    const std::size_t slot = pick_fill_slot(in_batch);
    if (meta_[slot].key.has_value()) key_to_slot_.erase(*meta_[slot].key);
    meta_[slot] = SlotMeta{key, f, tick_};
    key_to_slot_[key] = slot;
    in_batch.insert(slot);
    chosen.push_back(slot);
    fills.emplace_back(slot, e);
  }
  if (!fills.empty()) {
    std::vector<ExpertReadRequest> requests;
    requests.reserve(fills.size());
    for (const auto& [slot, e] : fills)
      requests.push_back({ExpertId{layer, e}, std::span<std::byte>(slot_data(slot), stride_)});
    try {
      storage_.read_experts(requests);
    } catch (...) {
      // New keys never become visible when their read fails (expert_cache.cpp:169-182).
      for (const auto& [slot, e] : fills) {
        (void)e;
        if (meta_[slot].key.has_value()) key_to_slot_.erase(*meta_[slot].key);
        meta_[slot] = SlotMeta{};
      }
      throw;
    }
  }
  std::vector<ExpertCacheEntry> out;
  out.reserve(experts.size());
  for (std::size_t i = 0; i < experts.size(); ++i)
    out.push_back({ExpertId{layer, experts[i]}, chosen[i],
                   std::span<const std::byte>(slot_data(chosen[i]), stride_)});
  return out;
}

std::optional<std::size_t> HostExpertCache::resident_slot(std::uint32_t layer,
                                                          std::uint32_t expert) const noexcept {
  const auto it = key_to_slot_.find(key_of(layer, expert));
  if (it == key_to_slot_.end()) return std::nullopt;
  return it->second;
}

ExpertCacheStats HostExpertCache::stats() const noexcept {
  return {hits_, misses_, slots_.size(), max_slots_, slots_.size() * stride_, budget_bytes_};
}

// ---- LfuRecencyPolicy ------------------------------------------------------
LfuRecencyPolicy::LfuRecencyPolicy(std::size_t budget_bytes) : budget_bytes_(budget_bytes) {
  if (budget_bytes_ == 0U)
    throw std::invalid_argument("resident expert cache: budget must be non-zero");
}

std::uint64_t LfuRecencyPolicy::victim() const {
  if (order_.empty()) throw std::runtime_error("resident expert cache: no eviction victim available");
  return std::get<2>(*order_.begin());
}

std::vector<std::uint64_t> LfuRecencyPolicy::victims_of(std::uint32_t layer, std::uint32_t expert,
                                                        std::size_t accounted_bytes) const {
  std::vector<std::uint64_t> out;
  if (entries_.count(make_key(layer, expert)) != 0 || accounted_bytes > budget_bytes_) return out;
  std::size_t resident = resident_bytes_;
  for (auto it = order_.begin(); it != order_.end() && resident + accounted_bytes > budget_bytes_; ++it) {
    out.push_back(std::get<2>(*it));
    resident -= entries_.at(std::get<2>(*it)).bytes;
  }
  return out;
}

bool LfuRecencyPolicy::touch(std::uint32_t layer, std::uint32_t expert) {
  ++tick_;
  const std::uint64_t key = make_key(layer, expert);
  const std::size_t f = history_[key] + 1U;
  history_[key] = f;
  if (auto it = entries_.find(key); it != entries_.end()) {
    ++hits;
    order_.erase(Rank{it->second.frequency, it->second.last_use, key});
    it->second.frequency = f;
    it->second.last_use = tick_;
    order_.insert(Rank{f, tick_, key});
    return true;
  }
  ++misses;
  return false;
}

std::vector<std::uint64_t> LfuRecencyPolicy::admit(std::uint32_t layer, std::uint32_t expert,
                                                   std::size_t accounted_bytes) {
  const std::uint64_t key = make_key(layer, expert);
  if (accounted_bytes == 0U)
    throw std::invalid_argument("resident expert cache: resident expert byte accounting is zero");
  if (accounted_bytes > budget_bytes_)
    throw std::invalid_argument("resident expert cache: one expert exceeds the configured budget");
  std::vector<std::uint64_t> evicted;
  while (!entries_.empty() && resident_bytes_ + accounted_bytes > budget_bytes_) {
    const std::uint64_t v = victim();
    auto it = entries_.find(v);
    resident_bytes_ -= it->second.bytes;
    order_.erase(Rank{it->second.frequency, it->second.last_use, v});
    entries_.erase(it);
    ++evictions;
    evicted.push_back(v);
  }
  if (!entries_.emplace(key, Node{accounted_bytes, history_[key], tick_}).second)
    throw std::runtime_error("resident expert cache: duplicate insertion");
  order_.insert(Rank{history_[key], tick_, key});
  resident_bytes_ += accounted_bytes;
  ++loads;
  return evicted;
}

LfuRecencyPolicy::Outcome LfuRecencyPolicy::access(std::uint32_t layer, std::uint32_t expert,
                                                   std::size_t accounted_bytes) {
  Outcome out;
  out.hit = touch(layer, expert);
  if (!out.hit) out.evicted = admit(layer, expert, accounted_bytes);
  return out;
}

void LfuRecencyPolicy::forget(std::uint64_t key) noexcept {
  auto it = entries_.find(key);
  if (it == entries_.end()) return;
  resident_bytes_ -= it->second.bytes;
  order_.erase(Rank{it->second.frequency, it->second.last_use, key});
  entries_.erase(it);
  if (loads > 0) --loads;
}

bool LfuRecencyPolicy::contains(std::uint32_t layer, std::uint32_t expert) const noexcept {
  return entries_.count(make_key(layer, expert)) != 0;
}

// ---- sources ---------------------------------------------------------------
PinnedExpertStore::PinnedExpertStore(const osm_expert_geometry& geometry, std::uint32_t layers,
                                     std::uint32_t experts)
    : geom_(geometry), layers_(layers), experts_(experts) {
  std::string d;
  if (!check_expert_geometry(geometry, &d)) throw std::invalid_argument(d);
  stride_ = expert_blob_bytes(geometry);
  std::size_t n = 0, bytes = 0;
  if (!mul_ok(layers, experts, n) || !mul_ok(n, stride_, bytes) || bytes == 0)
    throw std::invalid_argument("pinned expert store: invalid size");
  const int rc = mem_.allocate(bytes);
  if (rc != 0) throw std::runtime_error(hip_error("pinned expert store allocation failed", rc));
}

const std::byte* PinnedExpertStore::host_blob(std::uint32_t layer, std::uint32_t expert) {
  return mutable_blob(layer, expert);
}

std::byte* PinnedExpertStore::mutable_blob(std::uint32_t layer, std::uint32_t expert) {
  if (layer >= layers_ || expert >= experts_)
    throw std::out_of_range("pinned expert store: expert index out of range");
  return data() + (static_cast<std::size_t>(layer) * experts_ + expert) * stride_;
}

HostCacheSource::HostCacheSource(HostExpertCache& cache, const osm_expert_geometry& geometry)
    : cache_(cache), geom_(geometry) {
  if (cache.stride_bytes() != expert_blob_bytes(geometry))
    throw std::invalid_argument("host cache stride does not match the expert geometry");
}

const std::byte* HostCacheSource::host_blob(std::uint32_t layer, std::uint32_t expert) {
  const std::uint32_t request[1] = {expert};
  const auto entries = cache_.fetch(layer, request);
  if (entries.size() != 1U)
    throw std::runtime_error("resident expert cache: host cache returned unexpected entry count");
  return entries.front().bytes.data();
}

// ---- HipResidentExpertCache ------------------------------------------------
struct HipResidentExpertCache::Impl {
  HipComputeContext& ctx;
  ExpertBlobSource& source;
  osm_expert_geometry geom{};
  std::size_t stride = 0;
  std::size_t nslots = 0;
  LfuRecencyPolicy policy;
  DeviceBytes slab;
  std::vector<std::size_t> free_slots;
  std::unordered_map<std::uint64_t, std::size_t> key_slot;
  std::unordered_map<std::uint64_t, std::unique_ptr<HipResidentExpert>> views;
  osmd_event reuse_ev = nullptr, fill_ev = nullptr;
  std::uint64_t filled = 0;
  // Fill batch (begin_fills .. end_fills): one reuse wait before the first
  // copy and one fill wait per stream after the last, instead of two per
  // copy. Its copies rotate over the context's side stream and the cache's
  // own: several copies in flight keep PCIe busier than one.
  bool batching = false, batch_waited = false;
  std::uint32_t batch_fills = 0;
  std::array<osmd_stream, kFillStreams - 1> own{};     // the cache's fill streams
  std::array<osmd_event, kFillStreams - 1> own_ev{};   // their ends, for end_fills
  osmd_stream fill_stream(std::uint32_t i) const { return i == 0 ? ctx.copy_stream() : own[i - 1]; }
  // Slots written in this batch and the stream that wrote them: a slot
  // evicted and refilled within one batch is written again on the same
  // stream, so its two copies land in order.
  std::vector<std::pair<std::size_t, osmd_stream>> batch_slots;
  // Pipelined use: per slot, the event after its last readers (null: none
  // pending).
  bool pipelined = false;
  std::vector<osmd_event> slot_reader;

  Impl(HipComputeContext& c, ExpertBlobSource& s, std::size_t budget)
      : ctx(c), source(s), policy(budget) {}
  ~Impl() {
    (void)ctx.activate();
    if (ctx.valid() && (reuse_ev || fill_ev)) osmd_stream_synchronize(ctx.copy_stream());
    for (osmd_stream st : own)
      if (st) osmd_stream_synchronize(st);
    if (reuse_ev) osmd_event_destroy(reuse_ev);
    if (fill_ev) osmd_event_destroy(fill_ev);
    for (osmd_event ev : own_ev)
      if (ev) osmd_event_destroy(ev);
    for (osmd_stream st : own)
      if (st) osmd_stream_destroy(st);
  }
};

HipResidentExpertCache::HipResidentExpertCache(HipComputeContext& context, ExpertBlobSource& source,
                                               std::size_t budget_bytes) {
  std::string d;
  if (!context.valid() || !context.activate(&d))
    throw std::invalid_argument("resident expert cache: HIP context must be valid");
  impl_ = std::make_unique<Impl>(context, source, budget_bytes);
  impl_->geom = source.geometry();
  if (!check_expert_geometry(impl_->geom, &d)) throw std::invalid_argument(d);
  impl_->stride = expert_blob_bytes(impl_->geom);
  impl_->nslots = budget_bytes / impl_->stride;
  if (impl_->nslots > 0) {
    const int rc = impl_->slab.allocate(impl_->nslots * impl_->stride);
    if (rc != 0) throw std::runtime_error(hip_error("resident expert cache: slab allocation failed", rc));
  }
  impl_->free_slots.reserve(impl_->nslots);
  for (std::size_t s = impl_->nslots; s-- > 0;) impl_->free_slots.push_back(s);
  int rc = osmd_event_create(&impl_->reuse_ev);
  if (rc == 0) rc = osmd_event_create(&impl_->fill_ev);
  for (std::uint32_t i = 0; i + 1 < kFillStreams && rc == 0; ++i) {
    rc = osmd_event_create(&impl_->own_ev[i]);
    if (rc == 0) rc = osmd_stream_create(&impl_->own[i]);
  }
  if (rc != 0) throw std::runtime_error(hip_error("resident expert cache: event creation failed", rc));
}

HipResidentExpertCache::~HipResidentExpertCache() = default;

HipResidentExpert* HipResidentExpertCache::get(std::uint32_t layer, std::uint32_t expert,
                                               std::string* diagnostic) noexcept {
  Impl& m = *impl_;
  const std::uint64_t key = LfuRecencyPolicy::make_key(layer, expert);
  try {
    if (m.policy.touch(layer, expert)) {
      set_diag(diagnostic, "resident expert cache hit");
      return m.views.at(key).get();
    }
    // Miss: bytes first, then eviction and insertion (the reference's order,
    // vulkan_resident_expert_cache.cpp:98-171), so a failed fetch evicts nothing.
    const std::byte* src = m.source.host_blob(layer, expert);
    const auto evicted = m.policy.admit(layer, expert, m.stride);
    for (const std::uint64_t v : evicted) {
      m.free_slots.push_back(m.key_slot.at(v));
      m.key_slot.erase(v);
      m.views.erase(v);
    }
    if (m.free_slots.empty()) {
      m.policy.forget(key);
      throw std::runtime_error("resident expert cache: no free slot after eviction");
    }
    const std::size_t slot = m.free_slots.back();
    std::uint8_t* dst = m.slab.as<std::uint8_t>() + slot * m.stride;
    if (!m.ctx.activate(diagnostic)) {
      m.policy.forget(key);
      return nullptr;
    }
    // The side stream waits for everything enqueued so far on the compute
    // stream (earlier readers of this slot), copies, and the compute stream
    // waits for the copy. In a fill batch nothing is enqueued on the compute
    // stream between the gets, so the first copy's wait covers them all and
    // end_fills makes the compute stream wait once for the last copy.
    int rc = 0;
    if (!m.pipelined && (!m.batching || !m.batch_waited)) {
      rc = osmd_event_record(m.reuse_ev, m.ctx.stream());
      if (rc == 0) rc = osmd_stream_wait_event(m.ctx.copy_stream(), m.reuse_ev);
      for (std::uint32_t i = 0; m.batching && i + 1 < kFillStreams && rc == 0; ++i)
        rc = osmd_stream_wait_event(m.own[i], m.reuse_ev);
      m.batch_waited = m.batching && rc == 0;
    }
    osmd_stream cs = m.fill_stream(m.batching ? m.batch_fills % kFillStreams : 0U);
    if (m.batching) {
      for (const auto& [bs, bst] : m.batch_slots)
        if (bs == slot) cs = bst;
      m.batch_slots.emplace_back(slot, cs);
    }
    if (m.pipelined && rc == 0 && slot < m.slot_reader.size() && m.slot_reader[slot] != nullptr) {
      // Only the slot's last readers must be done before it is overwritten.
      rc = osmd_stream_wait_event(cs, m.slot_reader[slot]);
      m.slot_reader[slot] = nullptr;
    }
    if (rc == 0)
      rc = m.source.device_readable() ? osmd_copy_from_pinned(dst, src, m.stride, kFillBlocks, cs)
                                      : osmd_memcpy_h2d(dst, src, m.stride, cs);
    if (rc == 0 && !m.batching) {
      rc = osmd_event_record(m.fill_ev, m.ctx.copy_stream());
      if (rc == 0) rc = osmd_stream_wait_event(m.ctx.stream(), m.fill_ev);
    }
    if (rc == 0 && m.batching) ++m.batch_fills;
    if (rc == 0 && !m.source.stable_pointers()) rc = osmd_stream_synchronize(cs);
    if (rc != 0) {
      m.policy.forget(key);
      set_diag(diagnostic, hip_error("resident expert cache: fill failed", rc));
      return nullptr;
    }
    auto view = HipResidentExpert::view(m.ctx, dst, m.geom, diagnostic);
    if (!view) {
      m.policy.forget(key);
      return nullptr;
    }
    m.free_slots.pop_back();
    m.key_slot[key] = slot;
    auto owned = std::make_unique<HipResidentExpert>(std::move(*view));
    HipResidentExpert* out = owned.get();
    m.views[key] = std::move(owned);
    m.filled += m.stride;
    set_diag(diagnostic, "resident expert cache miss loaded into HBM");
    return out;
  } catch (const std::exception& e) {
    set_diag(diagnostic, std::string("resident expert cache exception: ") + e.what());
    return nullptr;
  }
}

void HipResidentExpertCache::begin_fills() noexcept {
  impl_->batching = true;
  impl_->batch_waited = false;
  impl_->batch_fills = 0;
  impl_->batch_slots.clear();
}

int HipResidentExpertCache::end_fills() noexcept {
  Impl& m = *impl_;
  int rc = 0;
  if (m.batching && m.batch_fills > 0) {
    rc = osmd_event_record(m.fill_ev, m.ctx.copy_stream());
    if (rc == 0) rc = osmd_stream_wait_event(m.ctx.stream(), m.fill_ev);
  }
  // The cache's own streams that took a copy in this batch.
  for (std::uint32_t i = 1; m.batching && i < kFillStreams && i < m.batch_fills && rc == 0; ++i) {
    rc = osmd_event_record(m.own_ev[i - 1], m.own[i - 1]);
    if (rc == 0) rc = osmd_stream_wait_event(m.ctx.stream(), m.own_ev[i - 1]);
  }
  m.batch_slots.clear();
  m.batching = false;
  m.batch_waited = false;
  m.batch_fills = 0;
  return rc;
}

void HipResidentExpertCache::begin_pipeline() noexcept {
  // Work enqueued before the pipeline may read any slot: every slot starts
  // with one event after it (a refill waits for it; once the stack's own
  // layers read the slot, for theirs instead).
  Impl& m = *impl_;
  osmd_event start = nullptr;
  if (m.ctx.activate() && osmd_event_record(m.reuse_ev, m.ctx.stream()) == 0) start = m.reuse_ev;
  m.pipelined = true;
  m.slot_reader.assign(m.nslots, start);
}

void HipResidentExpertCache::mark_readers(std::uint32_t layer, std::uint32_t expert, osmd_event done) noexcept {
  const auto it = impl_->key_slot.find(LfuRecencyPolicy::make_key(layer, expert));
  if (it != impl_->key_slot.end() && it->second < impl_->slot_reader.size()) impl_->slot_reader[it->second] = done;
}

void HipResidentExpertCache::end_pipeline() noexcept {
  impl_->pipelined = false;
  impl_->slot_reader.assign(impl_->slot_reader.size(), nullptr);
}

HipValuesResult HipResidentExpertCache::run(std::uint32_t layer, std::uint32_t expert,
                                            std::span<const float> x) noexcept {
  HipValuesResult r;
  std::string d;
  HipResidentExpert* e = get(layer, expert, &d);
  if (e == nullptr) {
    r.diagnostic = d;
    return r;
  }
  r = e->run(impl_->ctx, x);
  if (!r.executed && !d.empty()) r.diagnostic = d + "; execution: " + r.diagnostic;
  return r;
}

bool HipResidentExpertCache::contains(std::uint32_t layer, std::uint32_t expert) const noexcept {
  return impl_->policy.contains(layer, expert);
}

std::vector<std::uint64_t> HipResidentExpertCache::victims_of(std::uint32_t layer, std::uint32_t expert) const {
  return impl_->policy.victims_of(layer, expert, impl_->stride);
}

const std::uint8_t* HipResidentExpertCache::resident_blob(std::uint32_t layer, std::uint32_t expert) const noexcept {
  const auto it = impl_->key_slot.find(LfuRecencyPolicy::make_key(layer, expert));
  if (it == impl_->key_slot.end()) return nullptr;
  return impl_->slab.as<const std::uint8_t>() + it->second * impl_->stride;
}

HipResidentExpertCacheStats HipResidentExpertCache::stats() const noexcept {
  const auto& p = impl_->policy;
  return {p.hits, p.misses, p.loads, p.evictions, p.resident_entries(), p.resident_bytes(),
          p.budget_bytes()};
}

std::size_t HipResidentExpertCache::slot_count() const noexcept { return impl_->nslots; }
std::size_t HipResidentExpertCache::stride() const noexcept { return impl_->stride; }
std::uint64_t HipResidentExpertCache::bytes_filled() const noexcept { return impl_->filled; }

}  // namespace osm
