// moe.cpp -- routed-MoE layer state and decode (the HIP counterparts of
// src/model/checkpoint_sparse_moe.cpp, checkpoint_moe_sublayer.cpp and
// routed_moe.cpp:254-430).
#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <limits>
#include <string>
#include <unordered_set>
#include <utility>
#include <vector>

#include "host_util.hpp"
#include "osm_hip.h"
#include "osm_hip.hpp"

namespace osm {
namespace {

bool finite_weights(const void* p, std::size_t n, std::uint32_t dtype) {
  if (dtype == OSM_META_F32) return all_finite(std::span<const float>(static_cast<const float*>(p), n));
  const auto* h = static_cast<const std::uint16_t*>(p);
  const std::uint16_t exp_mask = dtype == OSM_META_BF16 ? 0x7F80U : 0x7C00U;
  for (std::size_t i = 0; i < n; ++i)
    if ((h[i] & exp_mask) == exp_mask) return false;
  return true;
}

// Every value scale * q + bias of an affine-q8 matrix is finite (the
// reference scans its dequantised router, qwen_router.cpp:54-59).
bool finite_q8(const osm_affine_q8& m, std::size_t rows, std::size_t cols) {
  const std::size_t gpr = cols / m.group;
  for (std::size_t r = 0; r < rows; ++r)
    for (std::size_t c = 0; c < cols; ++c) {
      const float q = static_cast<float>((m.packed[r * (cols / 4) + c / 4] >> (8 * (c % 4))) & 0xFFU);
      const volatile float prod = m.scales[r * gpr + c / m.group] * q;  // rounded before the add
      if (!std::isfinite(prod + m.biases[r * gpr + c / m.group])) return false;
    }
  return true;
}

// Slot-pointer tables of a call's expert launches. Each is written on the
// host into pinned memory that a copy kernel on the compute stream reads when
// it runs, so a table is filled once and never rewritten until the call has
// drained; the copy lands in the table's device mirror. Chunks are kept
// across calls (every call ends with its stream drained) and reused after
// reset().
class PtrTables {
 public:
  void reset() noexcept {
    for (Chunk& c : chunks_) c.used = 0;
    cur_ = 0;
  }
  // A fresh table of n pointers, 256-byte aligned and padded to 256 bytes.
  int take(std::size_t n, const std::uint8_t**& host, const std::uint8_t**& dev) {
    const std::size_t bytes = (n * sizeof(void*) + 255U) & ~static_cast<std::size_t>(255U);
    while (cur_ < chunks_.size() && chunks_[cur_].used + bytes > chunks_[cur_].cap) ++cur_;
    if (cur_ == chunks_.size()) {
      Chunk c;
      c.cap = std::max<std::size_t>(bytes, 64U << 10U);
      int rc = c.h.allocate(c.cap);
      if (rc == 0) rc = c.d.allocate(c.cap);
      if (rc != 0) return rc;
      chunks_.push_back(std::move(c));
    }
    Chunk& c = chunks_[cur_];
    host = reinterpret_cast<const std::uint8_t**>(static_cast<std::uint8_t*>(c.h.get()) + c.used);
    dev = reinterpret_cast<const std::uint8_t**>(c.d.as<std::uint8_t>() + c.used);
    c.used += bytes;
    return 0;
  }
  static std::size_t padded(std::size_t n) { return (n * sizeof(void*) + 255U) & ~static_cast<std::size_t>(255U); }

 private:
  struct Chunk {
    PinnedBytes h;
    DeviceBytes d;
    std::size_t cap = 0, used = 0;
  };
  std::vector<Chunk> chunks_;
  std::size_t cur_ = 0;
};

// Events that mark the slots a launch read (the capped cache's pipelined
// refills wait for them). Reused after reset(), once the call has drained.
class EventPool {
 public:
  EventPool() = default;
  EventPool(const EventPool&) = delete;
  EventPool& operator=(const EventPool&) = delete;
  ~EventPool() {
    for (osmd_event e : ev_) osmd_event_destroy(e);
  }
  void reset() noexcept { used_ = 0; }
  int next(osmd_event& out) {
    if (used_ == ev_.size()) {
      osmd_event e = nullptr;
      const int rc = osmd_event_create(&e);
      if (rc != 0) return rc;
      ev_.push_back(e);
    }
    out = ev_[used_++];
    return 0;
  }

 private:
  std::vector<osmd_event> ev_;
  std::size_t used_ = 0;
};

}  // namespace

struct HipMoeLayer::Impl {
  HipMoeLayerConfig cfg{};
  std::uint32_t router_dtype = OSM_META_BF16;
  std::uint32_t router_group = 0;  // OSM_ROUTER_AFFINE_Q8 only
  std::uint32_t max_tokens = 0;
  int device = -1;
  DeviceBytes router, shared_gate_vec, norm_weight, shared_blob;
  DeviceBytes zero_blob;  // fallback blob when there is no shared expert
  // workspace
  DeviceBytes x_in, y_out, logits, ids, weights, mass, shared_gate, x_norm, h, slot_ptrs;
  DeviceBytes logit_bounds;  // [T, E] bound of each logit's distance from the reference's
  DeviceBytes router_norms;  // bf16 router: [E + 1][D/32] norms of its 32-column chunks (row E: shared gate)
  DeviceBytes route_stats;   // 4 routing counters (osmd_moe_args::route_stats)
  PinnedBytes host_ptrs;  // staging for slot pointers chosen on the host
  PinnedBytes host_io;    // cache-driven path: pinned staging of inputs and outputs (grown on use)
  DeviceBytes dev_io;     // its device mirror: one copy in, one copy out per call
  // Cache-driven path: slot tables, events marking the slots each launch
  // read, and the per-slot partials of runs split into rounds (grown on use;
  // a buffer outgrown during a call is kept until the next call starts).
  PtrTables tables;
  EventPool events;
  DeviceBytes parts;
  std::vector<DeviceBytes> parts_retired;
  void begin_cached_call() noexcept {
    tables.reset();
    events.reset();
    parts_retired.clear();
  }
  float* ensure_parts(std::uint32_t tokens, int* rc) {
    const std::size_t need = osmd_moe_parts_bytes(&cfg.geometry, nslot(), tokens);
    if (parts.size() < need) {
      DeviceBytes fresh;
      *rc = fresh.allocate(need);
      if (*rc != 0) return nullptr;
      if (parts.get() != nullptr) parts_retired.push_back(std::move(parts));
      parts = std::move(fresh);
    }
    return parts.as<float>();
  }
  // grouped (multi-token) path: carved per call from the context's shared
  // workspace (every layer on one stream uses the same memory in turn)
  HipMoePath path = HipMoePath::automatic;
  enum GroupedBuf { kXTerms, kXSums, kPairPos, kPairW, kTiles, kTileCount, kGuPart, kHTerms, kHSums, kPartial,
                    kLogitPlanes, kXNorms, kBoundPlanes, kGroupedBufs };
  std::array<std::size_t, kGroupedBufs> g_off{};
  std::size_t g_bytes = 0;
  std::uint8_t* g_base = nullptr;

  void plan_grouped() {
    const osm_expert_geometry& g = cfg.geometry;
    const std::size_t T = max_tokens, D = g.hidden, I = g.inter, G = g.group;
    const std::size_t P = T * nslot();
    const std::size_t tiles = osmd_moe_grouped_max_tiles(max_tokens, nslot(), cfg.expert_count);
    const std::size_t parts = osmd_moe_grouped_router_parts(static_cast<std::uint32_t>(D));
    const std::array<std::size_t, kGroupedBufs> bytes = {
        T * 3U * D * 2U,                                                            // x terms
        T * (D / G) * 4U,                                                           // x group sums
        P * 4U, P * 4U,                                                             // pair positions, weights
        tiles * 80U, 4U,                                                            // tiles + rows, tile count
        osmd_moe_grouped_splits(&g, static_cast<std::uint32_t>(D)) * 2U * P * I * 4U,  // gate/up partials
        P * 2U * I * 2U, P * (I / G) * 4U,                                          // h terms, h sums
        osmd_moe_grouped_splits(&g, static_cast<std::uint32_t>(I)) * P * D * 4U,   // down partials
        parts * T * (cfg.expert_count + 1U) * 4U,                                   // logit planes
        T * (D / 32U) * 4U,                                                         // input chunk norms
        parts * T * (cfg.expert_count + 1U) * 4U};                                  // bound planes
    std::size_t off = 0;
    for (std::size_t i = 0; i < bytes.size(); ++i) {
      g_off[i] = off;
      off += (bytes[i] + 255U) & ~static_cast<std::size_t>(255U);
    }
    g_bytes = off;
  }

  int ensure_grouped(HipComputeContext& context) {
    if (g_bytes == 0) plan_grouped();
    int rc = 0;
    g_base = static_cast<std::uint8_t*>(context.shared_workspace(g_bytes, &rc));
    return g_base != nullptr ? 0 : (rc != 0 ? rc : 1);
  }
  template <typename T>
  T* gbuf(GroupedBuf b) const { return reinterpret_cast<T*>(g_base + g_off[b]); }

  // Whether a decode of `tokens` rows of x goes through the grouped GEMMs.
  bool grouped_ok(const void* x) const {
    const osm_expert_geometry& g = cfg.geometry;
    return (g.group == 32U || g.group == 64U || g.group == 128U) && g.hidden % 128U == 0U &&
           g.inter % 128U == 0U && reinterpret_cast<std::uintptr_t>(x) % 16U == 0U;
  }
  bool use_grouped(std::uint32_t tokens, const void* x) const {
    if (path == HipMoePath::per_token) return false;
    if (path == HipMoePath::grouped) return true;
    return tokens >= kGroupedMinTokens && grouped_ok(x);
  }

  osmd_moe_grouped_args grouped_args(const osmd_moe_args& a, bool x_bf16) {
    osmd_moe_grouped_args ga{};
    ga.moe = a;
    ga.x_bf16 = x_bf16 ? 1U : 0U;
    ga.x_terms = gbuf<std::uint16_t>(kXTerms);
    ga.x_sums = gbuf<float>(kXSums);
    ga.pair_pos = gbuf<std::uint32_t>(kPairPos);
    ga.pair_w = gbuf<float>(kPairW);
    ga.tiles = gbuf<void>(kTiles);
    ga.tile_count = gbuf<std::uint32_t>(kTileCount);
    ga.gu_part = gbuf<float>(kGuPart);
    ga.h_terms = gbuf<std::uint16_t>(kHTerms);
    ga.h_sums = gbuf<float>(kHSums);
    ga.partial = gbuf<float>(kPartial);
    ga.logit_planes = gbuf<float>(kLogitPlanes);
    ga.router_norms = router_norms.as<const float>();
    ga.x_norms = gbuf<float>(kXNorms);
    ga.bound_planes = gbuf<float>(kBoundPlanes);
    return ga;
  }

  std::uint32_t nslot() const { return cfg.top_k + (cfg.has_shared_expert ? 1U : 0U); }

  // Whether the last decode wrote its routing into the fixed workspace of
  // the allocation-free entry rather than into this layer's buffers. Every
  // other launch builds its arguments here, which clears it.
  mutable bool routing_in_static = false;
  osmd_moe_args args(const float* x, float* y, std::uint32_t tokens,
                     const std::uint8_t* const* table, bool sublayer) const {
    routing_in_static = false;
    osmd_moe_args a{};
    a.geom = cfg.geometry;
    a.expert_count = cfg.expert_count;
    a.top_k = cfg.top_k;
    a.norm_topk_prob = cfg.norm_topk_prob ? 1U : 0U;
    a.router_dtype = router_dtype;
    a.router_group = router_group;
    a.flags = (cfg.has_shared_expert ? static_cast<std::uint32_t>(OSMD_MOE_SHARED) : 0U) |
              (sublayer ? static_cast<std::uint32_t>(OSMD_MOE_RMSNORM | OSMD_MOE_RESIDUAL) : 0U);
    a.tokens = tokens;
    a.rms_eps = cfg.rms_eps;
    a.x = x;
    a.y = y;
    a.router = router.get();
    a.shared_gate_vec = shared_gate_vec.get();
    a.norm_weight = norm_weight.as<const float>();
    a.shared_expert = shared_blob.as<const std::uint8_t>();
    a.expert_table = table;
    a.fallback_blob = shared_blob.get() ? shared_blob.as<const std::uint8_t>() : zero_blob.as<const std::uint8_t>();
    a.logits = logits.as<float>();
    a.logit_bounds = logit_bounds.as<float>();
    a.route_stats = route_stats.as<std::uint32_t>();
    a.ids = ids.as<std::uint32_t>();
    a.weights = weights.as<float>();
    a.shared_gate = shared_gate.as<float>();
    a.mass = mass.as<float>();
    a.x_norm = x_norm.as<float>();
    a.h = h.as<float>();
    a.slot_ptrs = slot_ptrs.as<const std::uint8_t*>();
    return a;
  }
};

HipMoeLayer::HipMoeLayer() = default;
HipMoeLayer::~HipMoeLayer() = default;
HipMoeLayer::HipMoeLayer(HipMoeLayer&&) noexcept = default;
HipMoeLayer& HipMoeLayer::operator=(HipMoeLayer&&) noexcept = default;

std::optional<HipMoeLayer> HipMoeLayer::create(HipComputeContext& context, const HipMoeLayerConfig& config,
                                               const void* router, std::uint32_t router_dtype,
                                               const void* shared_gate_vec,
                                               std::span<const float> norm_weight,
                                               std::span<const std::byte> shared_blob,
                                               std::uint32_t max_tokens,
                                               std::string* diagnostic) noexcept {
  try {
    if (!context.activate(diagnostic)) return std::nullopt;
    const osm_expert_geometry& g = config.geometry;
    if (!check_expert_geometry(g, diagnostic)) return std::nullopt;
    if (config.expert_count == 0 || config.top_k == 0) {
      set_diag(diagnostic, "qwen router: dimensions and top_k must be non-zero");
      return std::nullopt;
    }
    if (config.top_k > config.expert_count) {
      set_diag(diagnostic, "qwen router: top_k cannot exceed expert_count");
      return std::nullopt;
    }
    if (config.top_k > OSMD_MAX_TOP_K || config.expert_count > OSMD_MAX_EXPERTS) {
      set_diag(diagnostic, "MoE layer: top_k <= 16 and expert_count <= 1024 are supported");
      return std::nullopt;
    }
    const std::size_t nslot = config.top_k + (config.has_shared_expert ? 1U : 0U);
    if (osmd_moe_down_lds_bytes(g.inter, static_cast<std::uint32_t>(nslot)) > 65536U) {
      set_diag(diagnostic, "MoE layer: (top_k + shared) * intermediate exceeds the 64 KiB LDS staging");
      return std::nullopt;
    }
    if ((router_dtype > OSM_META_BF16 && router_dtype != OSM_ROUTER_AFFINE_Q8) || router == nullptr) {
      set_diag(diagnostic, "MoE layer: router must be F32, F16, BF16 or affine Q8");
      return std::nullopt;
    }
    const bool q8 = router_dtype == OSM_ROUTER_AFFINE_Q8;
    const auto* rq = static_cast<const osm_affine_q8*>(router);
    const auto* sq = static_cast<const osm_affine_q8*>(shared_gate_vec);
    if (q8) {
      // checkpoint_sparse_moe.cpp:59-90 dequantises both modules at load; here
      // they stay 8-bit in HBM and the router kernel dequantises in registers.
      auto ok = [&](const osm_affine_q8* m) {
        return m && m->packed && m->scales && m->biases && m->group != 0 && m->group % 4U == 0 &&
               g.hidden % m->group == 0;
      };
      if (!ok(rq) || (config.has_shared_expert && (!ok(sq) || sq->group != rq->group))) {
        set_diag(diagnostic, "MoE layer: affine Q8 router and shared gate need one group size, a multiple of 4 dividing hidden");
        return std::nullopt;
      }
    }
    if (max_tokens == 0 || max_tokens > 65535U) {
      set_diag(diagnostic, "MoE layer: max_tokens must be in [1, 65535]");
      return std::nullopt;
    }
    if (!norm_weight.empty() && norm_weight.size() != g.hidden) {
      set_diag(diagnostic, "MoE sublayer: RMSNorm weight size does not match hidden");
      return std::nullopt;
    }
    if (config.has_shared_expert) {
      if (shared_blob.size() != expert_blob_bytes(g) || shared_gate_vec == nullptr) {
        set_diag(diagnostic, "Qwen sparse MoE shared expert geometry does not match hidden size");
        return std::nullopt;
      }
    }
    const std::size_t esz = q8 ? 0U : osm_meta_bytes(router_dtype);
    const std::size_t router_n = static_cast<std::size_t>(config.expert_count) * g.hidden;
    if (q8 ? !finite_q8(*rq, config.expert_count, g.hidden) : !finite_weights(router, router_n, router_dtype)) {
      set_diag(diagnostic, "qwen router: router weight contains non-finite value");
      return std::nullopt;
    }
    if (config.has_shared_expert &&
        (q8 ? !finite_q8(*sq, 1U, g.hidden) : !finite_weights(shared_gate_vec, g.hidden, router_dtype))) {
      set_diag(diagnostic, "shared expert scalar gate contains non-finite value");
      return std::nullopt;
    }
    auto impl = std::make_unique<Impl>();
    impl->cfg = config;
    impl->router_dtype = router_dtype;
    impl->router_group = q8 ? rq->group : 0U;
    impl->max_tokens = max_tokens;
    impl->device = context.device();
    const osmd_stream st = context.stream();
    auto up = [&](DeviceBytes& d, const void* src, std::size_t bytes) {
      int rc = d.allocate(bytes);
      if (rc == 0 && bytes) rc = osmd_memcpy_h2d(d.get(), src, bytes, st);
      return rc;
    };
    const std::size_t T = max_tokens, D = g.hidden, E = config.expert_count, K = config.top_k;
    // Affine q8: one buffer [packed rows x D/4][scales rows x D/g][biases].
    auto up_q8 = [&](DeviceBytes& d, const osm_affine_q8& m, std::size_t rows) {
      const std::size_t qb = rows * D, mb = rows * (D / m.group) * sizeof(float);
      int rc2 = d.allocate(qb + 2 * mb);
      if (rc2 == 0) rc2 = osmd_memcpy_h2d(d.get(), m.packed, qb, st);
      if (rc2 == 0) rc2 = osmd_memcpy_h2d(d.as<std::uint8_t>() + qb, m.scales, mb, st);
      if (rc2 == 0) rc2 = osmd_memcpy_h2d(d.as<std::uint8_t>() + qb + mb, m.biases, mb, st);
      return rc2;
    };
    int rc = q8 ? up_q8(impl->router, *rq, E) : up(impl->router, router, router_n * esz);
    if (rc == 0 && config.has_shared_expert)
      rc = q8 ? up_q8(impl->shared_gate_vec, *sq, 1U) : up(impl->shared_gate_vec, shared_gate_vec, D * esz);
    if (rc == 0 && !norm_weight.empty()) rc = up(impl->norm_weight, norm_weight.data(), norm_weight.size_bytes());
    if (rc == 0 && router_dtype == OSM_META_BF16) {
      // Norms of the bf16 router's 32-column chunks (and of the shared-gate
      // vector as row E), each rounded up, for the router GEMM's error bounds.
      const std::size_t chunks = D / 32U;
      std::vector<float> nrm((E + 1U) * chunks, 0.0F);
      auto widen = [](std::uint16_t b) {
        const std::uint32_t u = static_cast<std::uint32_t>(b) << 16;
        float f;
        std::memcpy(&f, &u, 4);
        return static_cast<double>(f);
      };
      for (std::size_t r = 0; r <= E; ++r) {
        const std::uint16_t* w = r < E ? static_cast<const std::uint16_t*>(router) + r * D
                                       : static_cast<const std::uint16_t*>(shared_gate_vec);
        if (w == nullptr) continue;
        for (std::size_t c = 0; c < chunks; ++c) {
          double ss = 0.0;
          for (std::size_t j = 0; j < 32U; ++j) ss += widen(w[c * 32U + j]) * widen(w[c * 32U + j]);
          nrm[r * chunks + c] = std::nextafter(static_cast<float>(std::sqrt(ss) * (1.0 + 1e-12)),
                                               std::numeric_limits<float>::infinity());
        }
      }
      rc = up(impl->router_norms, nrm.data(), nrm.size() * sizeof(float));
    }
    if (rc == 0 && config.has_shared_expert) rc = up(impl->shared_blob, shared_blob.data(), shared_blob.size());
    if (rc == 0 && !config.has_shared_expert) {
      rc = impl->zero_blob.allocate(expert_blob_bytes(g));
      if (rc == 0) rc = osmd_zero(impl->zero_blob.get(), impl->zero_blob.size(), st);
    }
    if (rc == 0) rc = impl->x_in.allocate(T * D * sizeof(float));
    if (rc == 0) rc = impl->y_out.allocate(T * D * sizeof(float));
    if (rc == 0) rc = impl->logits.allocate(T * E * sizeof(float));
    if (rc == 0) rc = impl->logit_bounds.allocate(T * E * sizeof(float));
    if (rc == 0) rc = impl->route_stats.allocate(4U * sizeof(std::uint32_t));
    if (rc == 0) rc = osmd_zero(impl->route_stats.get(), 4U * sizeof(std::uint32_t), st);
    if (rc == 0) rc = impl->ids.allocate(T * K * sizeof(std::uint32_t));
    if (rc == 0) rc = impl->weights.allocate(T * K * sizeof(float));
    if (rc == 0) rc = impl->mass.allocate(T * sizeof(float));
    if (rc == 0) rc = impl->shared_gate.allocate(T * sizeof(float));
    if (rc == 0) rc = impl->x_norm.allocate(T * D * sizeof(float));
    if (rc == 0) rc = impl->h.allocate(T * nslot * g.inter * sizeof(float));
    if (rc == 0) rc = impl->slot_ptrs.allocate(T * nslot * sizeof(void*));
    // Slot pointers start null (read as the fallback blob until a selection
    // writes them).
    if (rc == 0) rc = osmd_zero(impl->slot_ptrs.get(), impl->slot_ptrs.size(), st);
    if (rc == 0) rc = osmd_zero(impl->shared_gate.get(), T * sizeof(float), st);
    if (rc == 0) rc = impl->host_ptrs.allocate(T * nslot * sizeof(void*));
    if (rc == 0) rc = osmd_stream_synchronize(st);
    if (rc != 0) {
      set_diag(diagnostic, hip_error("MoE layer allocation/upload failed", rc));
      return std::nullopt;
    }
    HipMoeLayer layer;
    layer.impl_ = std::move(impl);
    set_diag(diagnostic, "HIP MoE layer state resident in HBM");
    return layer;
  } catch (const std::exception& e) {
    set_diag(diagnostic, std::string("MoE layer creation exception: ") + e.what());
    return std::nullopt;
  }
}

bool HipMoeLayer::valid() const noexcept { return impl_ && impl_->router.get(); }
const HipMoeLayerConfig& HipMoeLayer::config() const noexcept {
  static const HipMoeLayerConfig none{};
  return impl_ ? impl_->cfg : none;
}
std::uint32_t HipMoeLayer::max_tokens() const noexcept { return impl_ ? impl_->max_tokens : 0; }
const std::uint8_t* HipMoeLayer::shared_blob() const noexcept {
  return impl_ ? impl_->shared_blob.as<const std::uint8_t>() : nullptr;
}
const std::uint32_t* HipMoeLayer::device_ids() const noexcept {
  return impl_ ? impl_->ids.as<const std::uint32_t>() : nullptr;
}

HipDispatchResult HipMoeLayer::decode_device(HipComputeContext& context, const float* x, float* y,
                                             std::uint32_t tokens,
                                             const std::uint8_t* const* expert_table,
                                             bool sublayer) noexcept {
  HipDispatchResult r;
  if (!valid()) {
    r.diagnostic = "MoE layer is not valid";
    return r;
  }
  if (!context.activate(&r.diagnostic)) return r;
  if (context.device() != impl_->device) {
    r.diagnostic = "MoE layer belongs to a different device";
    return r;
  }
  if (tokens == 0 || tokens > impl_->max_tokens) {
    r.diagnostic = "MoE decode token count must be in [1, max_tokens]";
    return r;
  }
  if (x == nullptr || y == nullptr || expert_table == nullptr) {
    r.diagnostic = "MoE decode needs device input, output and expert table";
    return r;
  }
  if (sublayer && impl_->norm_weight.get() == nullptr) {
    r.diagnostic = "MoE sublayer decode needs an RMSNorm weight";
    return r;
  }
  const osmd_moe_args a = impl_->args(x, y, tokens, expert_table, sublayer);
  int rc;
  if (impl_->use_grouped(tokens, x)) {
    if (!impl_->grouped_ok(x)) {
      r.diagnostic = "grouped MoE needs group 32, 64 or 128, hidden and intermediate multiples of 128, and a 16-byte aligned input";
      return r;
    }
    rc = impl_->ensure_grouped(context);
    if (rc == 0) {
      const osmd_moe_grouped_args ga = impl_->grouped_args(a, false);
      rc = osmd_moe_grouped(&ga, context.stream());
    }
  } else {
    rc = osmd_moe_decode(&a, context.stream());
  }
  if (rc != 0) {
    r.diagnostic = hip_error("MoE decode launch failed", rc);
    return r;
  }
  r.executed = true;
  r.diagnostic = "HIP routed MoE decode enqueued";
  return r;
}

namespace {

// The routing workspace of `tokens` rows, carved from the fixed array in
// 256-byte aligned parts: logits, their bounds, ids, weights, mass, shared
// gate, normalised input, h, slot pointers.
std::size_t static_workspace_bytes(const HipMoeLayerConfig& c, std::size_t tokens) {
  auto al = [](std::size_t n) { return (n + 255U) & ~static_cast<std::size_t>(255U); };
  const std::size_t nslot = c.top_k + (c.has_shared_expert ? 1U : 0U);
  const std::size_t T = tokens;
  return 2U * al(T * c.expert_count * 4U) + 2U * al(T * c.top_k * 4U) + 2U * al(T * 4U) +
         al(T * c.geometry.hidden * 4U) + al(T * nslot * c.geometry.inter * 4U) + al(T * nslot * sizeof(void*));
}

}  // namespace

std::uint32_t HipMoeLayer::static_tokens_capacity() const noexcept {
  if (!valid()) return 0;
  // One token's parts each round up to 256 bytes, so budget / (one token's
  // bytes) is a lower bound; count up from it while the next one fits.
  std::size_t t = OSMD_STATIC_SCRATCH_BYTES / static_workspace_bytes(impl_->cfg, 1U);
  while (t < 65535U && static_workspace_bytes(impl_->cfg, t + 1U) <= OSMD_STATIC_SCRATCH_BYTES) ++t;
  return static_cast<std::uint32_t>(t < 65535U ? t : 65535U);
}

int HipMoeLayer::decode_device_static(HipComputeContext& context, const float* x, float* y, std::uint32_t tokens,
                                      const std::uint8_t* const* expert_table, bool sublayer,
                                      const char** diagnostic) noexcept {
  auto say = [&](const char* m) {
    if (diagnostic) *diagnostic = m;
  };
  if (!valid()) return say("MoE layer is not valid"), OSM_E_INVALID;
  if (!context.valid() || osmd_set_device(context.device()) != 0)
    return say("HIP compute context is not valid or its device cannot be made current"), OSM_E_DEVICE;
  if (context.device() != impl_->device) return say("MoE layer belongs to a different device"), OSM_E_INVALID;
  if (x == nullptr || y == nullptr || expert_table == nullptr)
    return say("MoE decode needs device input, output and expert table"), OSM_E_INVALID;
  if (sublayer && impl_->norm_weight.get() == nullptr)
    return say("MoE sublayer decode needs an RMSNorm weight"), OSM_E_INVALID;
  if (tokens == 0 || tokens > static_tokens_capacity())
    return say("MoE decode without allocation: token count must be in [1, static_tokens_capacity] "
               "(the fixed 4 MiB workspace)"),
           OSM_E_INVALID;
  void* base = nullptr;
  if (osmd_static_scratch(context.device(), &base) != 0 || base == nullptr)
    return say("MoE decode without allocation: the fixed workspace's device address is unavailable"), OSM_E_DEVICE;
  osmd_moe_args a = impl_->args(x, y, tokens, expert_table, sublayer);
  auto al = [](std::size_t n) { return (n + 255U) & ~static_cast<std::size_t>(255U); };
  const HipMoeLayerConfig& c = impl_->cfg;
  const std::size_t T = tokens, nslot = impl_->nslot();
  auto* p = static_cast<std::uint8_t*>(base);
  a.logits = reinterpret_cast<float*>(p);
  p += al(T * c.expert_count * 4U);
  a.logit_bounds = reinterpret_cast<float*>(p);
  p += al(T * c.expert_count * 4U);
  a.ids = reinterpret_cast<std::uint32_t*>(p);
  p += al(T * c.top_k * 4U);
  a.weights = reinterpret_cast<float*>(p);
  p += al(T * c.top_k * 4U);
  a.mass = reinterpret_cast<float*>(p);
  p += al(T * 4U);
  a.shared_gate = reinterpret_cast<float*>(p);
  p += al(T * 4U);
  a.x_norm = reinterpret_cast<float*>(p);
  p += al(T * c.geometry.hidden * 4U);
  a.h = reinterpret_cast<float*>(p);
  p += al(T * nslot * c.geometry.inter * 4U);
  a.slot_ptrs = reinterpret_cast<const std::uint8_t**>(p);
  // Nothing here is read before this call writes it: the router writes the
  // logits, their bounds, the shared gate and the normalised input, the
  // selection the picks and slot pointers, gate/up every slot's h. The
  // routing counters are the layer's own.
  if (osmd_moe_decode(&a, context.stream()) != 0) return say("MoE decode launch failed"), OSM_E_DEVICE;
  impl_->routing_in_static = true;
  say("");
  return OSM_OK;
}

bool HipMoeLayer::set_path(HipMoePath path, std::string* diagnostic) noexcept {
  if (!impl_) return set_diag(diagnostic, "MoE layer is not valid"), false;
  if (path != HipMoePath::automatic && path != HipMoePath::per_token && path != HipMoePath::grouped)
    return set_diag(diagnostic, "unknown MoE path"), false;
  impl_->path = path;
  return true;
}

HipMoePath HipMoeLayer::path() const noexcept { return impl_ ? impl_->path : HipMoePath::automatic; }

HipDispatchResult HipMoeLayer::prefill_device_bf16(HipComputeContext& context, const std::uint16_t* x_bf16,
                                                   float* y, std::uint32_t tokens,
                                                   const std::uint8_t* const* expert_table) noexcept {
  HipDispatchResult r;
  if (!valid()) {
    r.diagnostic = "MoE layer is not valid";
    return r;
  }
  if (!context.activate(&r.diagnostic)) return r;
  if (tokens == 0 || tokens > impl_->max_tokens || x_bf16 == nullptr || y == nullptr || expert_table == nullptr) {
    r.diagnostic = "MoE prefill: invalid arguments";
    return r;
  }
  if (!impl_->grouped_ok(x_bf16)) {
    r.diagnostic = "grouped MoE needs group 32, 64 or 128, hidden and intermediate multiples of 128, and a 16-byte aligned input";
    return r;
  }
  int rc = impl_->ensure_grouped(context);
  if (rc == 0) {
    osmd_moe_args a = impl_->args(nullptr, y, tokens, expert_table, false);
    a.x = reinterpret_cast<const float*>(x_bf16);  // read as bf16 (x_bf16 = 1)
    const osmd_moe_grouped_args ga = impl_->grouped_args(a, true);
    rc = osmd_moe_grouped(&ga, context.stream());
  }
  if (rc != 0) {
    r.diagnostic = hip_error("MoE prefill launch failed", rc);
    return r;
  }
  r.executed = true;
  r.diagnostic = "HIP grouped MoE prefill enqueued";
  return r;
}

HipDispatchResult HipMoeLayer::launch_phase(HipComputeContext& context, const float* x, float* y,
                                            std::uint32_t tokens,
                                            const std::uint8_t* const* expert_table, bool sublayer,
                                            int phase) noexcept {
  HipDispatchResult r;
  if (!valid() || !context.activate(&r.diagnostic)) {
    if (r.diagnostic.empty()) r.diagnostic = "MoE layer is not valid";
    return r;
  }
  if (tokens == 0 || tokens > impl_->max_tokens || x == nullptr || y == nullptr || expert_table == nullptr) {
    r.diagnostic = "MoE phase launch: invalid arguments";
    return r;
  }
  if (sublayer && impl_->norm_weight.get() == nullptr) {
    r.diagnostic = "MoE sublayer decode needs an RMSNorm weight";
    return r;
  }
  const osmd_moe_args a = impl_->args(x, y, tokens, expert_table, sublayer);
  int rc;
  switch (phase) {
    case 0: rc = osmd_moe_router(&a, context.stream()); break;
    case 1: rc = osmd_moe_gate_up(&a, context.stream()); break;
    case 2: rc = osmd_moe_down(&a, context.stream()); break;
    default:
      r.diagnostic = "MoE phase must be 0 (route), 1 (gate/up) or 2 (down)";
      return r;
  }
  if (rc != 0) {
    r.diagnostic = hip_error("MoE phase launch failed", rc);
    return r;
  }
  r.executed = true;
  return r;
}

bool HipMoeLayer::routing_queryable() const noexcept { return impl_ && !impl_->routing_in_static; }

bool HipMoeLayer::download_routing(HipComputeContext& context, std::uint32_t tokens, HipMoeRouting& out,
                                   std::string* diagnostic) const noexcept {
  try {
    if (!valid() || tokens == 0 || tokens > impl_->max_tokens)
      return set_diag(diagnostic, "routing download: invalid layer or token count"), false;
    if (!routing_queryable())
      return set_diag(diagnostic, "routing download: the last decode ran without allocation, so its routing "
                                  "lives in the shared fixed workspace and cannot be queried"),
             false;
    const std::size_t K = impl_->cfg.top_k, E = impl_->cfg.expert_count;
    out.ids.resize(tokens * K);
    out.weights.resize(tokens * K);
    out.mass.resize(tokens);
    out.shared_gate.resize(tokens);
    out.logits.resize(tokens * E);
    const osmd_stream st = context.stream();
    int rc = osmd_memcpy_d2h(out.ids.data(), impl_->ids.get(), tokens * K * 4, st);
    if (rc == 0) rc = osmd_memcpy_d2h(out.weights.data(), impl_->weights.get(), tokens * K * 4, st);
    if (rc == 0) rc = osmd_memcpy_d2h(out.mass.data(), impl_->mass.get(), tokens * 4, st);
    if (rc == 0) rc = osmd_memcpy_d2h(out.shared_gate.data(), impl_->shared_gate.get(), tokens * 4, st);
    if (rc == 0) rc = osmd_memcpy_d2h(out.logits.data(), impl_->logits.get(), tokens * E * 4, st);
    if (rc == 0) rc = osmd_stream_synchronize(st);
    if (rc != 0) return set_diag(diagnostic, hip_error("routing download failed", rc)), false;
    if (!impl_->cfg.has_shared_expert) std::fill(out.shared_gate.begin(), out.shared_gate.end(), 0.0F);
    return true;
  } catch (const std::exception& e) {
    return set_diag(diagnostic, std::string("routing download exception: ") + e.what()), false;
  }
}

bool HipMoeLayer::routing_stats(HipComputeContext& context, std::uint32_t (&out)[4], bool reset,
                                std::string* diagnostic) noexcept {
  if (!valid()) return set_diag(diagnostic, "MoE layer is not valid"), false;
  if (!context.activate(diagnostic)) return false;
  const osmd_stream st = context.stream();
  int rc = osmd_memcpy_d2h(out, impl_->route_stats.get(), sizeof(out), st);
  if (rc == 0 && reset) rc = osmd_zero(impl_->route_stats.get(), sizeof(out), st);
  if (rc == 0) rc = osmd_stream_synchronize(st);
  if (rc != 0) return set_diag(diagnostic, hip_error("routing counters download failed", rc)), false;
  return true;
}

bool HipMoeLayer::download_normalized(HipComputeContext& context, std::uint32_t tokens, std::vector<float>& out,
                                      std::string* diagnostic) const noexcept {
  try {
    if (!valid() || tokens == 0 || tokens > impl_->max_tokens)
      return set_diag(diagnostic, "normalised input download: invalid layer or token count"), false;
    out.resize(static_cast<std::size_t>(tokens) * impl_->cfg.geometry.hidden);
    const osmd_stream st = context.stream();
    int rc = osmd_memcpy_d2h(out.data(), impl_->x_norm.get(), out.size() * sizeof(float), st);
    if (rc == 0) rc = osmd_stream_synchronize(st);
    if (rc != 0) return set_diag(diagnostic, hip_error("normalised input download failed", rc)), false;
    return true;
  } catch (const std::exception& e) {
    return set_diag(diagnostic, std::string("normalised input download exception: ") + e.what()), false;
  }
}

HipMoeResult HipMoeLayer::run(HipComputeContext& context, std::span<const float> hidden,
                              std::uint32_t tokens, const std::uint8_t* const* expert_table,
                              bool sublayer) noexcept {
  HipMoeResult r;
  try {
    if (!valid()) {
      r.diagnostic = "MoE layer is not valid";
      return r;
    }
    const std::size_t D = impl_->cfg.geometry.hidden;
    if (tokens == 0 || hidden.size() != static_cast<std::size_t>(tokens) * D) {
      r.diagnostic = "qwen router: hidden vector size mismatch";
      return r;
    }
    if (!all_finite(hidden)) {
      r.diagnostic = "qwen router: hidden vector contains non-finite value";
      return r;
    }
    if (tokens > impl_->max_tokens) {
      r.diagnostic = "MoE decode token count exceeds max_tokens";
      return r;
    }
    if (!context.activate(&r.diagnostic)) return r;
    const osmd_stream st = context.stream();
    int rc = osmd_memcpy_h2d(impl_->x_in.get(), hidden.data(), hidden.size_bytes(), st);
    if (rc != 0) {
      r.diagnostic = hip_error("MoE input upload failed", rc);
      return r;
    }
    auto d = decode_device(context, impl_->x_in.as<const float>(), impl_->y_out.as<float>(), tokens,
                           expert_table, sublayer);
    if (!d.executed) {
      r.diagnostic = d.diagnostic;
      return r;
    }
    r.values.resize(hidden.size());
    rc = osmd_memcpy_d2h(r.values.data(), impl_->y_out.get(), hidden.size_bytes(), st);
    if (rc == 0 && sublayer) {
      r.normalized.resize(hidden.size());
      rc = osmd_memcpy_d2h(r.normalized.data(), impl_->x_norm.get(), hidden.size_bytes(), st);
    }
    if (rc != 0) {
      r.values.clear();
      r.diagnostic = hip_error("MoE output download failed", rc);
      return r;
    }
    if (!download_routing(context, tokens, r.routing, &r.diagnostic)) {
      r.values.clear();
      return r;
    }
    for (float v : r.values)
      if (!std::isfinite(v)) {
        r.values.clear();
        r.diagnostic = "routed MoE produced non-finite output";
        return r;
      }
    r.executed = true;
    r.diagnostic = "HIP routed MoE decode executed";
  } catch (const std::exception& e) {
    r.values.clear();
    r.diagnostic = std::string("MoE decode exception: ") + e.what();
  }
  return r;
}

// Internal access for the cache-driven path.
struct MoeLayerAccess {
  using Impl = HipMoeLayer::Impl;
  static Impl* impl(HipMoeLayer& l) { return l.impl_.get(); }
};

namespace {

std::size_t align256(std::size_t v) { return (v + 255U) & ~static_cast<std::size_t>(255U); }

// One layer's routed picks through the capped cache. The picks are made
// resident in pick order, token by token, as the reference fetches them
// (routed_moe.cpp:320-366), and their experts run:
//  - all at once, with the fused expert kernels, when every pick of the
//    call is resident together (the usual case);
//  - otherwise in rounds: a round ends just before a get that would evict
//    one of its own picks, and its experts then run while every one of them
//    is still resident -- so any budget of at least one expert works, as in
//    the reference, which runs each pick right after its get;
//  - with split_hits, a round's picks that were resident before it began run
//    before the compute stream waits for the round's fills, so they overlap
//    the copies.
// Rounds write per-slot partials and a combine launch adds them exactly as
// the fused down kernel adds them, so every split gives the fused bits.
struct CachedLayerRun {
  CachedLayerRun(HipComputeContext& c, HipResidentExpertCache& e, MoeLayerAccess::Impl& l) : ctx(c), cache(e), m(l) {}
  HipComputeContext& ctx;
  HipResidentExpertCache& cache;
  MoeLayerAccess::Impl& m;
  std::uint32_t cache_layer = 0;
  std::uint32_t tokens = 0;
  const std::uint32_t* ids = nullptr;  // host [tokens][k]
  osmd_moe_args ae{};                  // the experts' arguments (slot_ptrs is set per launch)
  bool pipelined = false;              // cache in pipelined mode: mark the slots each launch read
  bool split_hits = false;
  std::string* diag = nullptr;

  struct Pick {
    std::uint32_t t, j;
    bool ready;  // resident before this round's fills
  };
  std::vector<Pick> pend;
  std::unordered_set<std::uint64_t> pend_keys, filled;
  bool used_parts = false, shared_done = false;

  // A table of every token's slots: the given picks' blobs and the shared
  // expert's, copied to the device on the compute stream.
  int table(std::span<const Pick> picks, bool shared, const std::uint8_t**& dev) {
    const std::uint32_t nslot = m.nslot(), K = m.cfg.top_k;
    const std::uint8_t** host = nullptr;
    int rc = m.tables.take(static_cast<std::size_t>(tokens) * nslot, host, dev);
    if (rc != 0) return rc;
    std::fill(host, host + static_cast<std::size_t>(tokens) * nslot, nullptr);
    for (const Pick& p : picks)
      host[p.t * nslot + p.j] = cache.resident_blob(cache_layer, ids[p.t * K + p.j]);
    if (shared)
      for (std::uint32_t t = 0; t < tokens; ++t) host[t * nslot + K] = m.shared_blob.as<const std::uint8_t>();
    return osmd_copy_d2d(dev, host, PtrTables::padded(static_cast<std::size_t>(tokens) * nslot), ctx.stream());
  }

  // Marks the slots of `picks` as read by everything enqueued so far.
  int mark(std::span<const Pick> picks) {
    if (!pipelined) return 0;
    osmd_event ev = nullptr;
    int rc = m.events.next(ev);
    if (rc == 0) rc = osmd_event_record(ev, ctx.stream());
    if (rc != 0) return rc;
    for (const Pick& p : picks) cache.mark_readers(cache_layer, ids[p.t * m.cfg.top_k + p.j], ev);
    return 0;
  }

  // Token t's listed slots, writing their partials.
  int launch_parts(std::uint32_t t, const osmd_slot_list& l, const std::uint8_t** dev_table, float* parts) {
    const std::size_t D = m.cfg.geometry.hidden, I = m.cfg.geometry.inter, nslot = m.nslot(), K = m.cfg.top_k;
    osmd_moe_args a = ae;
    a.tokens = 1;
    a.x_norm = ae.x_norm + t * D;
    a.h = ae.h + t * nslot * I;
    a.slot_ptrs = dev_table + t * nslot;
    a.weights = ae.weights + t * K;
    a.shared_gate = ae.shared_gate + t;
    return osmd_moe_experts_parts(&a, l, parts + osmd_moe_parts_bytes(&m.cfg.geometry, m.nslot(), t) / sizeof(float),
                                  ctx.stream());
  }

  // Runs the pending picks (and the shared expert, the first time), then
  // starts a new fill batch.
  int flush() {
    const std::uint32_t K = m.cfg.top_k;
    int rc = 0;
    float* parts = m.ensure_parts(tokens, &rc);
    if (parts == nullptr) return rc != 0 ? rc : 1;
    const bool shared = !shared_done && m.cfg.has_shared_expert;
    const std::uint8_t** dev = nullptr;
    rc = table(pend, shared, dev);
    if (rc != 0) return rc;
    std::vector<osmd_slot_list> first(tokens, osmd_slot_list{}), second(tokens, osmd_slot_list{});
    for (const Pick& p : pend) osmd_slot_list_add(split_hits && p.ready ? &first[p.t] : &second[p.t], p.j);
    if (shared)
      for (std::uint32_t t = 0; t < tokens; ++t) osmd_slot_list_add(&first[t], K);
    shared_done = true;
    for (std::uint32_t t = 0; t < tokens && rc == 0; ++t)
      if (first[t].count) rc = launch_parts(t, first[t], dev, parts);
    const int frc = cache.end_fills();
    if (rc == 0) rc = frc;
    for (std::uint32_t t = 0; t < tokens && rc == 0; ++t)
      if (second[t].count) rc = launch_parts(t, second[t], dev, parts);
    if (rc == 0) rc = mark(pend);
    cache.begin_fills();
    pend.clear();
    pend_keys.clear();
    filled.clear();
    used_parts = true;
    return rc;
  }

  // 0, a HIP error code, or -1 with the diagnostic set.
  int run() {
    const std::uint32_t K = m.cfg.top_k;
    const std::size_t D = m.cfg.geometry.hidden;
    shared_done = !m.cfg.has_shared_expert;
    auto fail = [&](std::string d) {
      (void)cache.end_fills();
      set_diag(diag, std::move(d));
      return -1;
    };
    cache.begin_fills();
    int rc = 0;
    for (std::uint32_t t = 0; t < tokens; ++t)
      for (std::uint32_t j = 0; j < K; ++j) {
        const std::uint32_t id = ids[t * K + j];
        const std::uint64_t key = LfuRecencyPolicy::make_key(cache_layer, id);
        if (!cache.contains(cache_layer, id)) {
          for (const std::uint64_t v : cache.victims_of(cache_layer, id))
            if (pend_keys.count(v) != 0) {
              rc = flush();
              if (rc != 0) return (void)cache.end_fills(), rc;
              break;
            }
        }
        const bool ready = cache.contains(cache_layer, id) && filled.count(key) == 0;
        std::string gd;
        HipResidentExpert* e = cache.get(cache_layer, id, &gd);
        if (e == nullptr) return fail("Qwen sparse MoE routed expert " + std::to_string(id) + " load failed: " + gd);
        if (e->input_dim() != D || e->output_dim() != D || e->intermediate_dim() != m.cfg.geometry.inter)
          return fail("Qwen sparse MoE routed expert geometry mismatch");
        if (!ready) filled.insert(key);
        pend.push_back({t, j, ready});
        pend_keys.insert(key);
      }
    std::size_t nready = 0;
    for (const Pick& p : pend) nready += p.ready ? 1U : 0U;
    if (!used_parts && (!split_hits || nready == 0 || nready == pend.size())) {
      // Every pick resident at once: the fused kernels.
      const std::uint8_t** dev = nullptr;
      rc = table(pend, m.cfg.has_shared_expert, dev);
      const int frc = cache.end_fills();
      if (rc == 0) rc = frc;
      osmd_moe_args a = ae;
      a.slot_ptrs = dev;
      if (rc == 0) rc = osmd_moe_experts(&a, ctx.stream());
      if (rc == 0) rc = mark(pend);
      return rc;
    }
    rc = flush();
    (void)cache.end_fills();
    if (rc == 0) rc = osmd_moe_combine(&ae, m.parts.as<const float>(), ctx.stream());
    return rc;
  }
};

}  // namespace

bool run_cached_stack(HipComputeContext& context, HipResidentExpertCache& cache,
                      std::span<HipMoeLayer* const> layers, const std::uint32_t* cache_layers,
                      std::span<const float> x, const std::uint32_t* pick_ids, const float* pick_weights,
                      float* y, std::string* diagnostic) noexcept {
  auto fail = [&](std::string d) {
    if (diagnostic) *diagnostic = std::move(d);
    return false;
  };
  bool pipelined = false;
  osmd_event ids_ready = nullptr;
  auto cleanup = [&]() {
    if (pipelined) {
      (void)osmd_stream_synchronize(context.stream());
      cache.end_pipeline();
      pipelined = false;
    }
    if (ids_ready != nullptr) osmd_event_destroy(ids_ready);
    ids_ready = nullptr;
  };
  try {
    const std::size_t n = layers.size();
    const bool given = pick_ids != nullptr;
    if (n == 0 || cache_layers == nullptr || y == nullptr || given != (pick_weights != nullptr))
      return fail("invalid arguments");
    auto* m0 = layers[0] ? MoeLayerAccess::impl(*layers[0]) : nullptr;
    if (m0 == nullptr || !layers[0]->valid()) return fail("layer 0: MoE layer is not valid");
    const std::size_t D = m0->cfg.geometry.hidden, K = m0->cfg.top_k;
    const std::uint32_t tokens = static_cast<std::uint32_t>(x.size() / (D ? D : 1));
    if (tokens == 0 || x.size() != tokens * D) return fail("qwen router: hidden vector size mismatch");
    if (!all_finite(x)) return fail("qwen router: hidden vector contains non-finite value");
    std::size_t E_max = 0;
    for (std::size_t i = 0; i < n; ++i) {
      auto* m = layers[i] ? MoeLayerAccess::impl(*layers[i]) : nullptr;
      const std::string at = "layer " + std::to_string(i) + ": ";
      if (m == nullptr || !layers[i]->valid()) return fail(at + "MoE layer is not valid");
      if (m->cfg.geometry.hidden != D) return fail("layers must share one hidden size");
      if (m->cfg.top_k != K) return fail("layers of one stack need one top_k");
      if (tokens > m->max_tokens) return fail(at + "qwen router: hidden vector size mismatch");
      if (m->norm_weight.get() == nullptr) return fail(at + "MoE sublayer decode needs an RMSNorm weight");
      if (given)
        for (std::size_t j = 0; j < tokens * K; ++j) {
          const std::size_t o = i * tokens * K + j;
          if (pick_ids[o] >= m->cfg.expert_count)
            return fail(at + "routed MoE pick " + std::to_string(pick_ids[o]) + " is out of range");
          if (!std::isfinite(pick_weights[o])) return fail(at + "routed MoE encountered a non-finite routing weight");
        }
      E_max = std::max<std::size_t>(E_max, m->cfg.expert_count);
    }
    if (!context.activate(diagnostic)) return false;
    const osmd_stream st = context.stream();
    for (std::size_t i = 0; i < n; ++i) MoeLayerAccess::impl(*layers[i])->begin_cached_call();

    // Device block: two activation buffers (layer outputs alternate), the
    // given picks' weights of every layer, and the routing outputs one layer
    // at a time. Pinned host mirror: x and the weights in, each layer's
    // routed ids out (device routing), y out.
    const std::size_t xb = x.size_bytes(), wb = given ? n * tokens * K * 4U : 0U, kb = tokens * K * 4U;
    const std::size_t o_a = 0, o_b = align256(xb), o_w = o_b + align256(xb), o_norm = o_w + align256(wb),
                      o_lg = o_norm + align256(xb), o_mass = o_lg + align256(tokens * E_max * 4U),
                      o_gate = o_mass + align256(tokens * 4U), o_rid = o_gate + align256(tokens * 4U),
                      o_rw = o_rid + align256(kb), o_hid = o_rw + align256(kb),
                      total = o_hid + (given ? 0U : n * align256(kb));
    DeviceBytes dev;
    PinnedBytes host;
    int rc = dev.allocate(total);
    if (rc == 0) rc = host.allocate(total);
    if (rc == 0 && !given) rc = osmd_event_create(&ids_ready);
    if (rc != 0) return cleanup(), fail(hip_error("cached stack: staging allocation failed", rc));
    auto* h = static_cast<std::uint8_t*>(host.get());
    auto* d = dev.as<std::uint8_t>();
    std::memcpy(h + o_a, x.data(), xb);
    if (given) std::memcpy(h + o_w, pick_weights, wb);
    rc = osmd_copy_d2d(d, h, o_norm, st);  // x (and every layer's given weights)
    if (rc != 0) return cleanup(), fail(hip_error("cached stack: input copy failed", rc));

    cache.begin_pipeline();
    pipelined = true;
    for (std::size_t i = 0; i < n; ++i) {
      auto* m = MoeLayerAccess::impl(*layers[i]);
      float* cur = reinterpret_cast<float*>(d + (i % 2 == 0 ? o_a : o_b));
      float* nxt = reinterpret_cast<float*>(d + (i % 2 == 0 ? o_b : o_a));
      osmd_moe_args ar = m->args(cur, nxt, tokens, nullptr, true);
      ar.x_norm = reinterpret_cast<float*>(d + o_norm);
      ar.logits = reinterpret_cast<float*>(d + o_lg);
      ar.ids = reinterpret_cast<std::uint32_t*>(d + o_rid);
      ar.weights = reinterpret_cast<float*>(d + o_rw);
      ar.mass = reinterpret_cast<float*>(d + o_mass);
      ar.shared_gate = reinterpret_cast<float*>(d + o_gate);
      const std::uint32_t* ids = nullptr;
      osmd_moe_args ae = ar;
      if (given) {
        // The router alone: the RMSNorm output and the shared gate (the
        // selection would be discarded).
        rc = osmd_moe_router(&ar, st);
        ids = pick_ids + i * tokens * K;
        ae.weights = reinterpret_cast<float*>(d + o_w) + i * tokens * K;
      } else {
        // Route and select on the device, then read the ids: the host decides
        // residency from them, as the reference's cache does.
        auto* hid = h + o_hid + i * align256(kb);
        rc = osmd_moe_route(&ar, st);
        if (rc == 0) rc = osmd_copy_d2d(hid, d + o_rid, align256(kb), st);
        if (rc == 0) rc = osmd_event_record(ids_ready, st);
        if (rc == 0) rc = osmd_event_synchronize(ids_ready);
        ids = reinterpret_cast<const std::uint32_t*>(hid);
      }
      if (rc != 0) return cleanup(), fail("layer " + std::to_string(i) + ": " + hip_error("cached stack routing failed", rc));
      std::string ld;
      CachedLayerRun run(context, cache, *m);
      run.cache_layer = cache_layers[i];
      run.tokens = tokens;
      run.ids = ids;
      run.ae = ae;
      run.pipelined = true;
      run.split_hits = !given;
      run.diag = &ld;
      rc = run.run();
      if (rc != 0) {
        cleanup();
        return fail("layer " + std::to_string(i) + ": " + (rc < 0 ? ld : hip_error("cached stack launch failed", rc)));
      }
    }
    const std::size_t o_y = n % 2 == 0 ? o_a : o_b;
    rc = osmd_copy_d2d(h + o_y, d + o_y, align256(xb), st);
    if (rc == 0) rc = osmd_stream_synchronize(st);
    cleanup();
    if (rc != 0) return fail(hip_error("cached stack failed", rc));
    std::memcpy(y, h + o_y, xb);
    return true;
  } catch (const std::exception& e) {
    cleanup();
    return fail(std::string("cached stack: ") + e.what());
  }
}

HipMoeResult run_qwen_sparse_moe_hip(HipComputeContext& context, HipResidentExpertCache& expert_cache,
                                     HipMoeLayer& layer_state, std::uint32_t layer,
                                     std::span<const float> hidden, bool sublayer,
                                     const HipMoePicks* picks) noexcept {
  HipMoeResult r;
  try {
    auto* m = MoeLayerAccess::impl(layer_state);
    if (m == nullptr || !layer_state.valid()) {
      r.diagnostic = "MoE layer is not valid";
      return r;
    }
    const std::size_t D = m->cfg.geometry.hidden, K = m->cfg.top_k;
    const std::uint32_t tokens = static_cast<std::uint32_t>(hidden.size() / (D ? D : 1));
    if (tokens == 0 || hidden.size() != tokens * D || tokens > m->max_tokens) {
      r.diagnostic = "qwen router: hidden vector size mismatch";
      return r;
    }
    if (!all_finite(hidden)) {
      r.diagnostic = "qwen router: hidden vector contains non-finite value";
      return r;
    }
    if (sublayer && m->norm_weight.get() == nullptr) {
      r.diagnostic = "MoE sublayer decode needs an RMSNorm weight";
      return r;
    }
    if (picks != nullptr) {
      if (picks->ids == nullptr || picks->weights == nullptr) {
        r.diagnostic = "routed MoE picks need ids and weights";
        return r;
      }
      for (std::size_t i = 0; i < tokens * K; ++i) {
        if (picks->ids[i] >= m->cfg.expert_count) {
          r.diagnostic = "routed MoE pick " + std::to_string(picks->ids[i]) + " is out of range";
          return r;
        }
        if (!std::isfinite(picks->weights[i])) {
          r.diagnostic = "routed MoE encountered a non-finite routing weight";  // routed_moe.cpp:33-37
          return r;
        }
      }
    }
    if (!context.activate(&r.diagnostic)) return r;
    m->begin_cached_call();
    const osmd_stream st = context.stream();
    const std::size_t E = m->cfg.expert_count;
    // Inputs and outputs of the call sit in one device block mirrored by
    // pinned host staging: [x | pick weights] then [y | normalised x | mass |
    // shared gate | logits | ids | weights]. With given picks that is one
    // copy in and one out; with device routing the ids come back first (one
    // wait). The copies are the library's 16-byte copy kernel reading or
    // writing the pinned staging directly (every block is a multiple of 256
    // bytes): for these few kilobytes it takes a third of the runtime's copy.
    const std::size_t xb = hidden.size_bytes(), kb = tokens * K * 4U, tb = tokens * 4U, eb = tokens * E * 4U;
    const std::size_t o_x = 0, o_pw = align256(xb), o_out = o_pw + align256(kb), o_y = o_out,
                      o_norm = o_y + align256(xb), o_mass = o_norm + align256(xb), o_gate = o_mass + align256(tb),
                      o_lg = o_gate + align256(tb), o_rid = o_lg + align256(eb), o_rw = o_rid + align256(kb),
                      io_bytes = o_rw + align256(kb);
    if (m->host_io.size() < io_bytes || m->dev_io.size() < io_bytes) {
      m->host_io.reset();
      m->dev_io.reset();
      int arc = m->host_io.allocate(io_bytes);
      if (arc == 0) arc = m->dev_io.allocate(io_bytes);
      if (arc != 0) {
        m->host_io.reset();
        m->dev_io.reset();
        r.diagnostic = hip_error("Qwen sparse MoE staging allocation failed", arc);
        return r;
      }
    }
    auto* io = static_cast<std::uint8_t*>(m->host_io.get());
    auto* dio = m->dev_io.as<std::uint8_t>();
    auto dptr = [&](std::size_t off) { return reinterpret_cast<float*>(dio + off); };
    osmd_moe_args ar = m->args(dptr(o_x), dptr(o_y), tokens, nullptr, sublayer);
    ar.x_norm = dptr(o_norm);
    ar.logits = dptr(o_lg);
    ar.ids = reinterpret_cast<std::uint32_t*>(dio + o_rid);
    ar.weights = dptr(o_rw);
    ar.mass = dptr(o_mass);
    ar.shared_gate = dptr(o_gate);
    osmd_moe_args ae = ar;  // the experts read the picks' weights
    if (picks != nullptr) ae.weights = dptr(o_pw);

    std::memcpy(io + o_x, hidden.data(), xb);
    const std::uint32_t* ids = nullptr;
    int rc = 0;
    if (picks != nullptr) {
      // Given picks: x and their weights in, then the router alone (the
      // RMSNorm output, logits and shared gate; no selection).
      std::memcpy(io + o_pw, picks->weights, kb);
      rc = osmd_copy_d2d(dio, io, o_out, st);
      if (rc == 0) rc = osmd_moe_router(&ar, st);
      ids = picks->ids;
    } else {
      // Route on the device and read the ids back.
      rc = osmd_copy_d2d(dio + o_x, io + o_x, align256(xb), st);
      if (rc == 0) rc = osmd_moe_route(&ar, st);
      if (rc == 0) rc = osmd_copy_d2d(io + o_rid, dio + o_rid, align256(kb), st);
      if (rc == 0) rc = osmd_stream_synchronize(st);
      ids = reinterpret_cast<const std::uint32_t*>(io + o_rid);
    }
    if (rc != 0) {
      r.diagnostic = hip_error("Qwen sparse MoE routing failed", rc);
      return r;
    }
    // Every pick made resident in pick order and run (in rounds when the
    // budget cannot hold them all; device-routed calls run the already
    // resident picks while the misses are copied).
    std::string ld;
    CachedLayerRun run(context, expert_cache, *m);
    run.cache_layer = layer;
    run.tokens = tokens;
    run.ids = ids;
    run.ae = ae;
    run.split_hits = picks == nullptr;
    run.diag = &ld;
    rc = run.run();
    if (rc < 0) {
      r.diagnostic = ld;
      return r;
    }
    if (rc == 0) rc = osmd_copy_d2d(io + o_out, dio + o_out, io_bytes - o_out, st);
    if (rc == 0) rc = osmd_stream_synchronize(st);
    if (rc != 0) {
      r.diagnostic = hip_error("Qwen sparse MoE expert phase failed", rc);
      return r;
    }
    auto take = [&](std::size_t off, std::size_t cnt) {
      const float* f = reinterpret_cast<const float*>(io + off);
      return std::vector<float>(f, f + cnt);
    };
    r.values = take(o_y, hidden.size());
    if (sublayer) r.normalized = take(o_norm, hidden.size());
    if (picks != nullptr) {
      r.routing.ids.assign(picks->ids, picks->ids + tokens * K);
      r.routing.weights.assign(picks->weights, picks->weights + tokens * K);
      // The given weights' sum in pick order (no selection ran).
      r.routing.mass.assign(tokens, 0.0F);
      for (std::uint32_t t = 0; t < tokens; ++t)
        for (std::size_t j = 0; j < K; ++j) r.routing.mass[t] += picks->weights[t * K + j];
    } else {
      const auto* rid = reinterpret_cast<const std::uint32_t*>(io + o_rid);
      r.routing.ids.assign(rid, rid + tokens * K);
      r.routing.weights = take(o_rw, tokens * K);
      r.routing.mass = take(o_mass, tokens);
    }
    r.routing.shared_gate = take(o_gate, tokens);
    if (!m->cfg.has_shared_expert) std::fill(r.routing.shared_gate.begin(), r.routing.shared_gate.end(), 0.0F);
    r.routing.logits = take(o_lg, tokens * E);
    r.executed = true;
    r.diagnostic = "Qwen sparse MoE combined routed and shared experts on the device.";
  } catch (const std::exception& e) {
    r.values.clear();
    r.diagnostic = std::string("Qwen sparse MoE exception: ") + e.what();
  }
  return r;
}

}  // namespace osm
