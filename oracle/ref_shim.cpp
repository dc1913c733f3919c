// ref_shim.cpp -- extern "C" entry points over the reference's own CPU code.
//
// TEST INFRASTRUCTURE ONLY. Compiled together with the reference's sources
// (src/cpu/reference_ops.cpp, src/model/qwen_router.cpp,
// src/model/shared_expert.cpp, src/cache/expert_cache.cpp) where they lie
// under the reference checkout, into oracle/_ref/libosm_ref.so. It lets the
// tests check the oracle restatement against the reference itself, and gives
// bench.py a CPU baseline that runs the reference's own functions. Nothing
// here is part of the product.

#include <cstdint>
#include <cstring>
#include <exception>
#include <span>
#include <stdexcept>
#include <string>
#include <vector>

#include "orbi/streammoe/cache/expert_cache.hpp"
#include "orbi/streammoe/cpu/reference_ops.hpp"
#include "orbi/streammoe/model/qwen_router.hpp"
#include "orbi/streammoe/model/shared_expert.hpp"
#include "orbi/streammoe/storage/expert_storage.hpp"

namespace sm = orbi::streammoe;

namespace {

thread_local std::string g_err;

template <typename F>
int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::invalid_argument& e) {
    g_err = e.what();
    return 1;
  } catch (const std::exception& e) {
    g_err = e.what();
    return 2;
  }
}

// Storage double matching the reference test's FakeStorage behaviour:
// pattern bytes (layer*37 + expert*11 + i) & 0xFF, optional one-shot failure.
class PatternStorage final : public sm::ExpertStorage {
 public:
  explicit PatternStorage(std::size_t stride) : stride_(stride) {}
  std::size_t expert_stride_bytes() const noexcept override { return stride_; }
  void read_experts(std::span<sm::ExpertReadRequest> reqs) override {
    ++batches;
    if (fail_next) {
      fail_next = false;
      throw std::runtime_error("synthetic read failure");
    }
    for (auto& r : reqs)
      for (std::size_t i = 0; i < stride_; ++i)
        r.destination[i] = static_cast<std::byte>(
            (r.id.layer * 37U + r.id.expert * 11U + static_cast<std::uint32_t>(i)) & 0xFFU);
  }
  bool fail_next = false;
  std::uint64_t batches = 0;

 private:
  std::size_t stride_;
};

struct RefHostCache {
  PatternStorage storage;
  sm::ExpertCache cache;
  RefHostCache(std::size_t stride, std::size_t budget, std::size_t min_slots)
      : storage(stride), cache(storage, budget, min_slots) {}
};

std::vector<float> dequant(const std::uint32_t* packed, std::size_t rows,
                           std::size_t packed_cols, const float* s,
                           const float* b, std::uint32_t group) {
  const std::size_t ng = rows * (packed_cols * 8U / group);
  return sm::cpu::dequantize_affine_rows(
      std::span<const std::uint32_t>(packed, rows * packed_cols), rows,
      packed_cols, std::span<const float>(s, ng), std::span<const float>(b, ng),
      sm::cpu::AffineQuantSpec{.bits = 4, .group_size = group});
}

}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_err.c_str(); }

int ref_dequantize_affine_rows(const std::uint32_t* packed, std::size_t packed_len,
                               std::size_t rows, std::size_t packed_cols,
                               const float* scales, std::size_t scales_len,
                               const float* biases, std::size_t biases_len,
                               std::uint32_t bits, std::uint32_t group, float* out) {
  return guarded([&] {
    const auto v = sm::cpu::dequantize_affine_rows(
        std::span<const std::uint32_t>(packed, packed_len), rows, packed_cols,
        std::span<const float>(scales, scales_len),
        std::span<const float>(biases, biases_len),
        sm::cpu::AffineQuantSpec{.bits = bits, .group_size = group});
    std::memcpy(out, v.data(), v.size() * sizeof(float));
  });
}

int ref_matvec_row_major(const float* w, std::size_t w_len, std::size_t out_dim,
                         std::size_t in_dim, const float* x, std::size_t x_len,
                         float* out) {
  return guarded([&] {
    const auto v = sm::cpu::matvec_row_major(std::span<const float>(w, w_len), out_dim,
                                             in_dim, std::span<const float>(x, x_len));
    std::memcpy(out, v.data(), v.size() * sizeof(float));
  });
}

int ref_rms_norm_inplace(float* values, std::size_t values_len, std::size_t rows,
                         std::size_t dim, const float* weight, std::size_t weight_len,
                         float eps) {
  return guarded([&] {
    sm::cpu::rms_norm_inplace(std::span<float>(values, values_len), rows, dim,
                              std::span<const float>(weight, weight_len), eps);
  });
}

int ref_route_top_k(const float* logits, std::size_t n, std::size_t k, int normalize,
                    std::uint32_t* ids, float* probs) {
  return guarded([&] {
    const auto picks =
        sm::cpu::route_top_k(std::span<const float>(logits, n), k, normalize != 0);
    for (std::size_t i = 0; i < picks.size(); ++i) {
      ids[i] = picks[i].expert;
      probs[i] = picks[i].probability;
    }
  });
}

int ref_swiglu_inplace(float* gate, std::size_t n, const float* up) {
  return guarded([&] {
    sm::cpu::swiglu_inplace(std::span<float>(gate, n), std::span<const float>(up, n));
  });
}

int ref_route_qwen_top_k(const float* hidden, std::size_t hidden_len,
                         const float* router, std::size_t router_len,
                         std::size_t hidden_size, std::size_t expert_count,
                         std::size_t top_k, int norm, float* logits,
                         std::uint32_t* ids, float* weights, float* mass) {
  return guarded([&] {
    const auto r = sm::route_qwen_top_k_cpu(
        std::span<const float>(hidden, hidden_len),
        std::span<const float>(router, router_len),
        sm::QwenRouterConfig{.hidden_size = hidden_size,
                             .expert_count = expert_count,
                             .top_k = top_k,
                             .norm_topk_prob = norm != 0});
    if (logits) std::memcpy(logits, r.logits.data(), r.logits.size() * sizeof(float));
    for (std::size_t i = 0; i < r.picks.size(); ++i) {
      ids[i] = r.picks[i].expert;
      weights[i] = r.picks[i].weight;
    }
    if (mass) *mass = r.selected_probability_mass;
  });
}

int ref_run_shared_expert(const float* hidden, std::size_t hidden_size,
                          const float* gate, const float* up, const float* down,
                          const float* scalar, std::size_t inter, float* out,
                          float* out_gate) {
  const auto r = sm::run_shared_expert_cpu(
      std::span<const float>(hidden, hidden_size),
      sm::SharedExpertWeights{
          .gate_proj = std::span<const float>(gate, inter * hidden_size),
          .up_proj = std::span<const float>(up, inter * hidden_size),
          .down_proj = std::span<const float>(down, hidden_size * inter),
          .scalar_gate = std::span<const float>(scalar, hidden_size)},
      sm::SharedExpertConfig{.hidden_size = hidden_size, .intermediate_size = inter});
  if (!r.executed) {
    g_err = r.diagnostic;
    return 1;
  }
  std::memcpy(out, r.values.data(), r.values.size() * sizeof(float));
  *out_gate = r.scalar_gate;
  return 0;
}

// The reference's CPU composition of one sparse-MoE token, as its sublayer
// test builds it (tests/checkpoint_moe_sublayer_test.cpp:613-677): route on
// the fp32 router, per pick dequantize the three projections and run
// matvec -> swiglu -> matvec, accumulate weight*expert in pick order, then add
// run_shared_expert_cpu over the dequantized shared projections. Projections
// arrive as (packed, fp32 scales, fp32 biases) triples; experts[e] holds
// expert e's nine pointers in gate/up/down x packed/scales/biases order.
int ref_sparse_moe(const float* hidden, const float* router, std::uint32_t expert_count,
                   std::uint32_t top_k, const void* const* experts,
                   const void* const* shared, const float* shared_scalar,
                   std::uint32_t h, std::uint32_t inter, std::uint32_t group,
                   float* out, std::uint32_t* ids, float* weights) {
  return guarded([&] {
    const auto route = sm::route_qwen_top_k_cpu(
        std::span<const float>(hidden, h),
        std::span<const float>(router, static_cast<std::size_t>(expert_count) * h),
        sm::QwenRouterConfig{.hidden_size = h,
                             .expert_count = expert_count,
                             .top_k = top_k,
                             .norm_topk_prob = true});
    auto proj = [&](const void* const* p, std::size_t out_dim, std::size_t in_dim,
                    std::span<const float> x) {
      const auto dense = dequant(static_cast<const std::uint32_t*>(p[0]), out_dim,
                                 in_dim / 8U, static_cast<const float*>(p[1]),
                                 static_cast<const float*>(p[2]), group);
      return sm::cpu::matvec_row_major(dense, out_dim, in_dim, x);
    };
    std::vector<float> acc(h, 0.0F);
    const std::span<const float> xs(hidden, h);
    for (std::size_t i = 0; i < route.picks.size(); ++i) {
      const auto& pk = route.picks[i];
      const void* const* e = experts + static_cast<std::size_t>(pk.expert) * 9U;
      auto g = proj(e + 0, inter, h, xs);
      const auto u = proj(e + 3, inter, h, xs);
      sm::cpu::swiglu_inplace(g, u);
      const auto y = proj(e + 6, h, inter, g);
      for (std::size_t j = 0; j < h; ++j) acc[j] += pk.weight * y[j];
      ids[i] = pk.expert;
      weights[i] = pk.weight;
    }
    if (shared != nullptr) {
      const auto dg = dequant(static_cast<const std::uint32_t*>(shared[0]), inter, h / 8U,
                              static_cast<const float*>(shared[1]),
                              static_cast<const float*>(shared[2]), group);
      const auto du = dequant(static_cast<const std::uint32_t*>(shared[3]), inter, h / 8U,
                              static_cast<const float*>(shared[4]),
                              static_cast<const float*>(shared[5]), group);
      const auto dd = dequant(static_cast<const std::uint32_t*>(shared[6]), h, inter / 8U,
                              static_cast<const float*>(shared[7]),
                              static_cast<const float*>(shared[8]), group);
      const auto s = sm::run_shared_expert_cpu(
          xs,
          sm::SharedExpertWeights{.gate_proj = dg,
                                  .up_proj = du,
                                  .down_proj = dd,
                                  .scalar_gate = std::span<const float>(shared_scalar, h)},
          sm::SharedExpertConfig{.hidden_size = h, .intermediate_size = inter});
      if (!s.executed) throw std::runtime_error(s.diagnostic);
      for (std::size_t j = 0; j < h; ++j) acc[j] += s.values[j];
    }
    std::memcpy(out, acc.data(), h * sizeof(float));
  });
}

void* ref_host_cache_create(std::size_t stride, std::size_t budget, std::size_t min_slots) {
  try {
    return new RefHostCache(stride, budget, min_slots);
  } catch (const std::exception& e) {
    g_err = e.what();
    return nullptr;
  }
}

void ref_host_cache_destroy(void* c) { delete static_cast<RefHostCache*>(c); }

int ref_host_cache_fetch(void* hc, std::uint32_t layer, const std::uint32_t* experts,
                         std::size_t n, int fail_read, std::uint64_t* out_slots) {
  auto* c = static_cast<RefHostCache*>(hc);
  c->storage.fail_next = fail_read != 0;
  const int rc = guarded([&] {
    const auto entries =
        c->cache.fetch(layer, std::span<const std::uint32_t>(experts, n));
    for (std::size_t i = 0; i < entries.size(); ++i) out_slots[i] = entries[i].slot;
  });
  c->storage.fail_next = false;
  return rc;
}

std::int64_t ref_host_cache_resident_slot(void* hc, std::uint32_t layer, std::uint32_t expert) {
  const auto s = static_cast<RefHostCache*>(hc)->cache.resident_slot(layer, expert);
  return s.has_value() ? static_cast<std::int64_t>(*s) : -1;
}

void ref_host_cache_stats(void* hc, std::uint64_t* o) {
  const auto s = static_cast<RefHostCache*>(hc)->cache.stats();
  o[0] = s.hits;
  o[1] = s.misses;
  o[2] = s.allocated_slots;
  o[3] = s.capacity_slots;
  o[4] = s.logical_bytes;
  o[5] = s.budget_bytes;
}

std::uint64_t ref_host_cache_storage_batches(void* hc) {
  return static_cast<RefHostCache*>(hc)->storage.batches;
}

}  // extern "C"
