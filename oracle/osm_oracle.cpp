// osm_oracle.cpp -- CPU oracle for the q4 routed-MoE hot path.
//
// TEST INFRASTRUCTURE ONLY: the checker for the HIP product library. Only
// tests/, the smoke() check and bench.py's cpu_baseline leg load it; the
// product never does.
//
// Each function restates one reference function in this file's own code and
// keeps the reference's arithmetic: the same summation order, the same
// std::exp / std::sqrt calls, the same tie rule and the same error cases.
// Compile with -ffp-contract=off so no multiply-add is fused where the
// reference's scalar loop rounds twice.
//
// Pinning (which checks tie this restatement to the reference) is listed per
// function in tests/test_oracle_*.py; in brief: reference known-answer tests
// (tests/cpu_reference_test.cpp, qwen_router_test.cpp, shared_expert_test.cpp,
// expert_cache_test.cpp, vulkan_resident_expert_cache_test.cpp), the
// reference CPU subset compiled from its own sources into oracle/_ref, and
// closed forms / fp64 brute force.

#include "osm_oracle.h"

#include <algorithm>
#include <bit>
#include <cmath>
#include <cstring>
#include <limits>
#include <optional>
#include <stdexcept>
#include <string>
#include <thread>
#include <tuple>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace {

thread_local std::string g_error;

int fail_invalid(const char* what) {
  g_error = what;
  return 1;
}
int fail_runtime(const char* what) {
  g_error = what;
  return 2;
}

// ---------------------------------------------------------------------------
// src/cpu/reference_ops.cpp:11-67 -- affine dequant. Word lanes are read low
// nibble first; lane j of word w is logical column w*per_word + j; value is
// scale[row, col/group] * q + bias[row, col/group] (one multiply, one add).
int dequant_rows(const uint32_t* packed, size_t packed_len, size_t rows,
                 size_t packed_cols, const float* scales, size_t scales_len,
                 const float* biases, size_t biases_len, uint32_t bits,
                 uint32_t group, float* out) {
  if (bits != 4U && bits != 8U)
    return fail_invalid("affine dequant: only 4-bit and 8-bit are supported");
  if (group == 0U) return fail_invalid("affine dequant: group_size must be non-zero");
  if (rows == 0U || packed_cols == 0U)
    return fail_invalid("affine dequant: rows and packed_cols must be non-zero");
  const size_t per_word = 32U / bits;
  const size_t cols = packed_cols * per_word;
  if (cols % group != 0U)
    return fail_invalid("affine dequant: logical columns must be divisible by group_size");
  const size_t groups = cols / group;
  if (packed_len != rows * packed_cols)
    return fail_invalid("affine dequant: packed size mismatch");
  if (scales_len != rows * groups || biases_len != rows * groups)
    return fail_invalid("affine dequant: scale/bias size mismatch");

  const uint32_t mask = (1U << bits) - 1U;
  for (size_t r = 0; r < rows; ++r) {
    const uint32_t* row_words = packed + r * packed_cols;
    const float* row_s = scales + r * groups;
    const float* row_b = biases + r * groups;
    float* row_out = out + r * cols;
    for (size_t w = 0; w < packed_cols; ++w) {
      uint32_t word = row_words[w];
      for (size_t j = 0; j < per_word; ++j) {
        const size_t c = w * per_word + j;
        const float q = static_cast<float>(word & mask);
        const float prod = row_s[c / group] * q;
        row_out[c] = prod + row_b[c / group];
        word >>= bits;
      }
    }
  }
  return 0;
}

// reference_ops.cpp:69-94 -- row-major matvec, one fp32 accumulator per row,
// columns summed left to right.
int matvec(const float* w, size_t w_len, size_t out_dim, size_t in_dim,
           const float* x, size_t x_len, float* y) {
  if (out_dim == 0U || in_dim == 0U)
    return fail_invalid("matvec: dimensions must be non-zero");
  if (w_len != out_dim * in_dim) return fail_invalid("matvec: weight size mismatch");
  if (x_len != in_dim) return fail_invalid("matvec: input size mismatch");
  for (size_t r = 0; r < out_dim; ++r) {
    const float* row = w + r * in_dim;
    float acc = 0.0F;
    for (size_t c = 0; c < in_dim; ++c) {
      const float prod = row[c] * x[c];
      acc = acc + prod;
    }
    y[r] = acc;
  }
  return 0;
}

// reference_ops.cpp:96-128 -- RMSNorm: sum of squares in order, scale =
// 1/sqrt(sum/dim + eps), then v *= scale * w (scale*w rounded first).
int rms_norm(float* v, size_t v_len, size_t rows, size_t dim, const float* w,
             size_t w_len, float eps) {
  if (rows == 0U || dim == 0U || v_len != rows * dim)
    return fail_invalid("rms_norm: invalid shape");
  if (w_len != 0U && w_len != dim) return fail_invalid("rms_norm: weight size mismatch");
  if (eps < 0.0F) return fail_invalid("rms_norm: eps must be non-negative");
  for (size_t r = 0; r < rows; ++r) {
    float* row = v + r * dim;
    float ss = 0.0F;
    for (size_t i = 0; i < dim; ++i) {
      const float sq = row[i] * row[i];
      ss = ss + sq;
    }
    const float mean = ss / static_cast<float>(dim);
    const float scale = 1.0F / std::sqrt(mean + eps);
    for (size_t i = 0; i < dim; ++i) {
      const float wi = (w_len == 0U) ? 1.0F : w[i];
      const float f = scale * wi;
      row[i] = row[i] * f;
    }
  }
  return 0;
}

// reference_ops.cpp:130-151 -- softmax: subtract the max, std::exp, running
// fp32 sum in index order, then divide every entry by the sum.
int softmax(float* v, size_t n) {
  if (n == 0U) return fail_invalid("softmax: input must not be empty");
  float mx = v[0];
  for (size_t i = 1; i < n; ++i)
    if (mx < v[i]) mx = v[i];
  float sum = 0.0F;
  for (size_t i = 0; i < n; ++i) {
    v[i] = std::exp(v[i] - mx);
    sum = sum + v[i];
  }
  if (!(sum > 0.0F) || !std::isfinite(sum))
    return fail_runtime("softmax: invalid normalization sum");
  for (size_t i = 0; i < n; ++i) v[i] = v[i] / sum;
  return 0;
}

struct Pick {
  uint32_t id;
  float p;
};

// reference_ops.cpp:153-212 -- top-k over softmax probabilities. Experts are
// visited in id order; the kept list stays sorted by probability, descending,
// with a stable sort, and a candidate only displaces the last kept entry when
// its probability is strictly larger. Net effect: order by (p desc, id asc).
int top_k(const float* logits, size_t n, size_t k, bool normalize,
          std::vector<Pick>& picks) {
  if (n == 0U) return fail_invalid("router: logits must not be empty");
  if (k == 0U || k > n) return fail_invalid("router: k must be within expert count");
  std::vector<float> p(logits, logits + n);
  if (int rc = softmax(p.data(), n)) return rc;
  picks.clear();
  auto by_prob = [](const Pick& a, const Pick& b) { return a.p > b.p; };
  for (size_t e = 0; e < n; ++e) {
    const Pick cand{static_cast<uint32_t>(e), p[e]};
    if (picks.size() < k) {
      picks.push_back(cand);
      std::stable_sort(picks.begin(), picks.end(), by_prob);
    } else if (cand.p > picks.back().p) {
      picks.back() = cand;
      std::stable_sort(picks.begin(), picks.end(), by_prob);
    }
  }
  if (normalize) {
    float s = 0.0F;
    for (const auto& pk : picks) s = s + pk.p;
    if (!(s > 0.0F) || !std::isfinite(s))
      return fail_runtime("router: selected probability sum is invalid");
    for (auto& pk : picks) pk.p = pk.p / s;
  }
  return 0;
}

// reference_ops.cpp:214-232
float sigmoid_f(float v) { return 1.0F / (1.0F + std::exp(-v)); }
float silu_f(float v) { return v * sigmoid_f(v); }

// src/model/qwen_router.cpp:11-94 -- validation, finite scans, logits by
// matvec, raw top-k, selected mass summed in pick order, optional
// renormalisation by the mass.
int route_qwen(const float* hidden, size_t hidden_len, const float* wr,
               size_t wr_len, size_t hidden_size, size_t experts, size_t k,
               bool norm, std::vector<float>& logits, std::vector<Pick>& picks,
               float& mass) {
  if (hidden_size == 0U || experts == 0U || k == 0U)
    return fail_invalid("qwen router: dimensions and top_k must be non-zero");
  if (k > experts) return fail_invalid("qwen router: top_k cannot exceed expert_count");
  if (experts > std::numeric_limits<uint32_t>::max())
    return fail_invalid("qwen router: expert_count exceeds routed-expert id range");
  if (hidden_len != hidden_size) return fail_invalid("qwen router: hidden vector size mismatch");
  if (experts > std::numeric_limits<size_t>::max() / hidden_size)
    return fail_invalid("qwen router: weight shape overflows size_t");
  if (wr_len != experts * hidden_size)
    return fail_invalid("qwen router: router weight size mismatch");
  for (size_t i = 0; i < hidden_len; ++i)
    if (!std::isfinite(hidden[i]))
      return fail_invalid("qwen router: hidden vector contains non-finite value");
  for (size_t i = 0; i < wr_len; ++i)
    if (!std::isfinite(wr[i]))
      return fail_invalid("qwen router: router weight contains non-finite value");
  logits.assign(experts, 0.0F);
  if (int rc = matvec(wr, wr_len, experts, hidden_size, hidden, hidden_len, logits.data()))
    return rc;
  if (int rc = top_k(logits.data(), experts, k, false, picks)) return rc;
  mass = 0.0F;
  for (const auto& pk : picks) mass = mass + pk.p;
  if (!(mass > 0.0F) || !std::isfinite(mass))
    return fail_runtime("qwen router: selected probability mass is invalid");
  if (norm)
    for (auto& pk : picks) pk.p = pk.p / mass;
  return 0;
}

// src/model/shared_expert.cpp:11-87 -- gate/up matvec, SwiGLU, down matvec,
// scalar gate dot in index order, sigmoid, scale every output.
int shared_expert(const float* hidden, size_t hidden_len, const float* g,
                  size_t g_len, const float* u, size_t u_len, const float* d,
                  size_t d_len, const float* sg, size_t sg_len, size_t h,
                  size_t inter, float* out, float* out_scale) {
  if (h == 0U || inter == 0U) return fail_invalid("shared expert dimensions must be non-zero");
  if (hidden_len != h) return fail_invalid("shared expert hidden size mismatch");
  if (g_len != inter * h || u_len != inter * h || d_len != h * inter || sg_len != h)
    return fail_invalid("shared expert weight geometry mismatch");
  std::vector<float> gate(inter), up(inter);
  if (int rc = matvec(g, g_len, inter, h, hidden, hidden_len, gate.data())) return rc;
  if (int rc = matvec(u, u_len, inter, h, hidden, hidden_len, up.data())) return rc;
  for (size_t i = 0; i < inter; ++i) gate[i] = silu_f(gate[i]) * up[i];
  if (int rc = matvec(d, d_len, h, inter, gate.data(), inter, out)) return rc;
  float logit = 0.0F;
  for (size_t i = 0; i < h; ++i) {
    const float prod = sg[i] * hidden[i];
    logit = logit + prod;
  }
  const float scale = sigmoid_f(logit);
  if (!std::isfinite(scale)) return fail_invalid("shared expert scalar gate is non-finite");
  for (size_t i = 0; i < h; ++i) out[i] = out[i] * scale;
  *out_scale = scale;
  return 0;
}

// src/backend/vulkan_qpack_expert.cpp:54-56 -- bf16 widens by a 16-bit shift.
float bf16_widen(uint16_t v) { return std::bit_cast<float>(static_cast<uint32_t>(v) << 16); }

// vulkan_qpack_expert.cpp:58-87 -- IEEE half decode including subnormals
// (renormalised by shifting the mantissa up) and inf/nan.
float f16_widen(uint16_t v) {
  const uint32_t sign = static_cast<uint32_t>(v & 0x8000U) << 16;
  uint32_t ex = (v >> 10) & 0x1FU;
  uint32_t man = v & 0x3FFU;
  uint32_t bits;
  if (ex == 0U) {
    if (man == 0U) {
      bits = sign;
    } else {
      int e = -14;
      while ((man & 0x400U) == 0U) {
        man <<= 1;
        --e;
      }
      man &= 0x3FFU;
      bits = sign | (static_cast<uint32_t>(e + 127) << 23) | (man << 13);
    }
  } else if (ex == 0x1FU) {
    bits = sign | 0x7F800000U | (man << 13);
  } else {
    bits = sign | ((ex + 112U) << 23) | (man << 13);
  }
  return std::bit_cast<float>(bits);
}

size_t meta_size(int dt) { return dt == ORACLE_META_F32 ? 4U : 2U; }

// Widen one metadata section to fp32, as float_section does at admission
// (vulkan_qpack_expert.cpp:89-145).
std::vector<float> widen(const uint8_t* p, size_t count, int dt) {
  std::vector<float> out(count);
  for (size_t i = 0; i < count; ++i) {
    if (dt == ORACLE_META_F32) {
      uint32_t b;
      std::memcpy(&b, p + 4 * i, 4);
      out[i] = std::bit_cast<float>(b);
    } else {
      uint16_t b;
      std::memcpy(&b, p + 2 * i, 2);
      out[i] = (dt == ORACLE_META_F16) ? f16_widen(b) : bf16_widen(b);
    }
  }
  return out;
}

// Expert blob = the qpack section order gate.{weight,scales,biases},
// up.{...}, down.{...}, each section contiguous (the layout written by
// tests/vulkan_resident_expert_cache_test.cpp:138-162 and
// docs/OSM-39B-QPACK-EXPERT-GEOMETRY.md).
struct Proj {
  const uint32_t* packed;
  std::vector<float> s, b;
  size_t out_dim, packed_cols;
};

struct BlobView {
  Proj gate, up, down;
};

BlobView bind_blob(const uint8_t* blob, uint32_t hidden, uint32_t inter,
                   uint32_t group, int dt) {
  const size_t ms = meta_size(dt);
  size_t off = 0;
  auto proj = [&](size_t out_dim, size_t in_dim) {
    Proj p;
    p.out_dim = out_dim;
    p.packed_cols = in_dim / 8U;
    p.packed = reinterpret_cast<const uint32_t*>(blob + off);
    off += out_dim * p.packed_cols * 4U;
    const size_t ng = out_dim * (in_dim / group);
    p.s = widen(blob + off, ng, dt);
    off += ng * ms;
    p.b = widen(blob + off, ng, dt);
    off += ng * ms;
    return p;
  };
  BlobView v;
  v.gate = proj(inter, hidden);
  v.up = proj(inter, hidden);
  v.down = proj(hidden, inter);
  return v;
}

int projection(const Proj& p, uint32_t group, const float* x, float* y) {
  std::vector<float> dense(p.out_dim * p.packed_cols * 8U);
  if (int rc = dequant_rows(p.packed, p.out_dim * p.packed_cols, p.out_dim,
                            p.packed_cols, p.s.data(), p.s.size(), p.b.data(),
                            p.b.size(), 4U, group, dense.data()))
    return rc;
  return matvec(dense.data(), dense.size(), p.out_dim, p.packed_cols * 8U, x,
                p.packed_cols * 8U, y);
}

// tests/checkpoint_moe_sublayer_test.cpp:512-548 (cpu_expert) -- one expert:
// dequantize each projection, matvec, SwiGLU in place, down matvec.
int expert_forward(const uint8_t* blob, uint32_t hidden, uint32_t inter,
                   uint32_t group, int dt, const float* x, float* out) {
  const BlobView v = bind_blob(blob, hidden, inter, group, dt);
  std::vector<float> g(inter), u(inter);
  if (int rc = projection(v.gate, group, x, g.data())) return rc;
  if (int rc = projection(v.up, group, x, u.data())) return rc;
  for (uint32_t i = 0; i < inter; ++i) g[i] = silu_f(g[i]) * u[i];
  return projection(v.down, group, g.data(), out);
}

// Shared expert from a q4 blob: dequantize to dense fp32 and run the
// shared_expert restatement (checkpoint_moe_sublayer_test.cpp:623-644).
int shared_from_blob(const uint8_t* blob, const float* scalar_gate,
                     uint32_t hidden, uint32_t inter, uint32_t group, int dt,
                     const float* x, float* out, float* out_scale) {
  const BlobView v = bind_blob(blob, hidden, inter, group, dt);
  auto dense = [&](const Proj& p, std::vector<float>& d) {
    d.resize(p.out_dim * p.packed_cols * 8U);
    return dequant_rows(p.packed, p.out_dim * p.packed_cols, p.out_dim,
                        p.packed_cols, p.s.data(), p.s.size(), p.b.data(),
                        p.b.size(), 4U, group, d.data());
  };
  std::vector<float> dg, du, dd;
  if (int rc = dense(v.gate, dg)) return rc;
  if (int rc = dense(v.up, du)) return rc;
  if (int rc = dense(v.down, dd)) return rc;
  return shared_expert(x, hidden, dg.data(), dg.size(), du.data(), du.size(),
                       dd.data(), dd.size(), scalar_gate, hidden, hidden,
                       inter, out, out_scale);
}

// Sparse MoE for one token (checkpoint_moe_sublayer_test.cpp:613-677 and
// routed_moe.cpp:254-430): routing on the normalised hidden vector, routed
// outputs accumulated as acc[i] += weight * expert[i] in pick order, then the
// already-gated shared output added.
int sparse_moe(const float* hidden, const float* router, uint32_t experts,
               uint32_t k, bool norm, const uint8_t* const* blobs,
               const uint8_t* shared_blob, const float* shared_sg,
               uint32_t h, uint32_t inter, uint32_t group, int dt, float* out,
               uint32_t* ids, float* weights, float* mass_out, float* sg_out,
               float* logits_out) {
  std::vector<float> logits;
  std::vector<Pick> picks;
  float mass = 0.0F;
  if (int rc = route_qwen(hidden, h, router, static_cast<size_t>(experts) * h,
                          h, experts, k, norm, logits, picks, mass))
    return rc;
  std::vector<float> acc(h, 0.0F), e(h);
  for (size_t i = 0; i < picks.size(); ++i) {
    if (!std::isfinite(picks[i].p))
      return fail_runtime("Qwen sparse MoE encountered non-finite routing weight");
    if (int rc = expert_forward(blobs[picks[i].id], h, inter, group, dt, hidden, e.data()))
      return rc;
    for (uint32_t j = 0; j < h; ++j) {
      const float prod = picks[i].p * e[j];
      acc[j] = acc[j] + prod;
    }
    if (ids) ids[i] = picks[i].id;
    if (weights) weights[i] = picks[i].p;
  }
  float sg = 0.0F;
  if (shared_blob != nullptr) {
    if (int rc = shared_from_blob(shared_blob, shared_sg, h, inter, group, dt, hidden, e.data(), &sg))
      return rc;
    for (uint32_t j = 0; j < h; ++j) acc[j] = acc[j] + e[j];
  }
  std::memcpy(out, acc.data(), h * sizeof(float));
  if (mass_out) *mass_out = mass;
  if (sg_out) *sg_out = sg;
  if (logits_out) std::memcpy(logits_out, logits.data(), experts * sizeof(float));
  return 0;
}

// ---------------------------------------------------------------------------
// Seeded counter-based generator for the synthetic inputs. Every element is
// a pure function of (seed, a, b, tensor, index) so any expert of any layer
// can be regenerated on demand, on the host or the device, bit for bit.
uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

uint64_t stream_of(uint64_t seed, uint32_t a, uint32_t b, uint32_t t) {
  return mix64(mix64(mix64(seed) ^ a) ^ ((static_cast<uint64_t>(b) << 8) | t));
}

uint32_t fields16(uint64_t hsh) {
  return static_cast<uint32_t>((hsh & 0xFFFFU) + ((hsh >> 16) & 0xFFFFU) +
                               ((hsh >> 32) & 0xFFFFU) + (hsh >> 48));
}

// Irwin-Hall(12) over 16-bit uniforms taken from three chained hashes,
// centred and scaled to unit variance: the integer sum is exact (standard
// deviation sqrt(2^32-1), i.e. 2^16 to 6e-11), then one exact multiply by
// 2^-16. Support is [-6, 6].
float normal_at(uint64_t stream, uint64_t i) {
  const uint64_t h0 = mix64(stream + i), h1 = mix64(h0), h2 = mix64(h1);
  const int32_t s = static_cast<int32_t>(fields16(h0) + fields16(h1) + fields16(h2));
  return static_cast<float>(s - 393210) * 0x1p-16F;
}

uint16_t bf16_rne(float f) {
  uint32_t u = std::bit_cast<uint32_t>(f);
  if ((u & 0x7FFFFFFFU) > 0x7F800000U) return static_cast<uint16_t>((u >> 16) | 0x40U);
  u += 0x7FFFU + ((u >> 16) & 1U);
  return static_cast<uint16_t>(u >> 16);
}

enum : uint32_t {
  kTGateQ = 0, kTGateS = 1, kTGateB = 2, kTUpQ = 3, kTUpS = 4, kTUpB = 5,
  kTDownQ = 6, kTDownS = 7, kTDownB = 8, kTRouter = 16, kTSharedGate = 17,
  kTNorm = 18, kTTokens = 32,
};
constexpr uint32_t kLayerTensorId = 0xFFFFFFFEU;
constexpr uint32_t kTokenTensorId = 0xFFFFFFFDU;

void synth_projection(uint64_t seed, uint32_t layer, uint32_t expert,
                      uint32_t tq, uint32_t ts, uint32_t tb, size_t out_dim,
                      size_t in_dim, uint32_t group, int dt, uint8_t*& p) {
  const uint64_t sq = stream_of(seed, layer, expert, tq);
  const size_t words = out_dim * in_dim / 8U;
  for (size_t i = 0; i < words; ++i) {
    const uint32_t w = static_cast<uint32_t>(mix64(sq + i));
    std::memcpy(p + 4 * i, &w, 4);
  }
  p += words * 4U;
  const uint64_t ss = stream_of(seed, layer, expert, ts);
  const uint64_t sb = stream_of(seed, layer, expert, tb);
  const size_t ng = out_dim * (in_dim / group);
  const size_t ms = meta_size(dt);
  uint8_t* sp = p;
  uint8_t* bp = p + ng * ms;
  for (size_t i = 0; i < ng; ++i) {
    const uint16_t sbits = bf16_rne(std::fabs(normal_at(ss, i)) * 0.02F);
    const float sval = bf16_widen(sbits);
    const float noise = normal_at(sb, i) * 0.002F;
    const uint16_t bbits = bf16_rne(-8.0F * sval + noise);
    if (dt == ORACLE_META_F32) {
      const float bval = bf16_widen(bbits);
      std::memcpy(sp + 4 * i, &sval, 4);
      std::memcpy(bp + 4 * i, &bval, 4);
    } else {
      std::memcpy(sp + 2 * i, &sbits, 2);
      std::memcpy(bp + 2 * i, &bbits, 2);
    }
  }
  p += 2 * ng * ms;
}

// ---------------------------------------------------------------------------
// src/cache/expert_cache.cpp:11-221 -- host L1 slot cache. Fixed stride,
// max_slots = budget/stride, lazy slot growth, per-key frequency history,
// one tick per fetch, victims by min (frequency, last_use, slot) skipping
// slots already used by the current batch, and rollback of the new keys when
// the storage read throws. The storage is the reference test's FakeStorage
// (tests/expert_cache_test.cpp:22-60).
struct HostCache {
  struct Meta {
    std::optional<uint64_t> key;
    size_t freq = 0;
    uint64_t last = 0;
  };
  size_t stride, budget, max_slots;
  std::vector<std::vector<uint8_t>> slots;
  std::vector<Meta> meta;
  std::unordered_map<uint64_t, size_t> where;
  std::unordered_map<uint64_t, size_t> freq;
  uint64_t tick = 0;
  size_t hits = 0, misses = 0;
  uint64_t storage_batches = 0;

  static uint64_t key_of(uint32_t l, uint32_t e) { return (static_cast<uint64_t>(l) << 32) | e; }

  size_t victim(const std::unordered_set<size_t>& used) const {
    for (size_t s = 0; s < meta.size(); ++s)
      if (!meta[s].key.has_value()) return s;
    size_t best_slot = std::numeric_limits<size_t>::max();
    std::tuple<size_t, uint64_t, size_t> best{std::numeric_limits<size_t>::max(),
                                              std::numeric_limits<uint64_t>::max(),
                                              std::numeric_limits<size_t>::max()};
    for (size_t s = 0; s < meta.size(); ++s) {
      if (used.count(s)) continue;
      const auto score = std::make_tuple(meta[s].freq, meta[s].last, s);
      if (score < best) {
        best = score;
        best_slot = s;
      }
    }
    if (best_slot == std::numeric_limits<size_t>::max())
      throw std::runtime_error("expert cache: batch requires more simultaneous slots than budget allows");
    return best_slot;
  }

  size_t fill_slot(const std::unordered_set<size_t>& used) {
    if (slots.size() < max_slots) {
      slots.emplace_back(stride);
      meta.push_back({});
      return slots.size() - 1;
    }
    return victim(used);
  }

  static uint8_t pattern(uint32_t l, uint32_t e, size_t i) {
    return static_cast<uint8_t>((l * 37U + e * 11U + static_cast<uint32_t>(i)) & 0xFFU);
  }
};

// src/backend/vulkan_resident_expert_cache.cpp:18-188 -- device-side cache
// policy: byte budget, key (layer<<32)|expert, one tick per get, frequency
// history that survives eviction, hit refreshes (frequency, last_use), miss
// evicts min (frequency, last_use, key) while resident + incoming > budget.
struct DeviceCache {
  struct Node {
    size_t bytes, freq;
    uint64_t last;
  };
  size_t budget, resident = 0;
  std::unordered_map<uint64_t, Node> entries;
  std::unordered_map<uint64_t, size_t> history;
  uint64_t tick = 0;
  size_t hits = 0, misses = 0, loads = 0, evictions = 0;

  uint64_t victim() const {
    bool have = false;
    uint64_t vk = 0;
    std::tuple<size_t, uint64_t, uint64_t> best{};
    for (const auto& [k, n] : entries) {
      const auto score = std::make_tuple(n.freq, n.last, k);
      if (!have || score < best) {
        best = score;
        vk = k;
        have = true;
      }
    }
    if (!have) throw std::runtime_error("resident expert cache: no eviction victim available");
    return vk;
  }
};

}  // namespace

extern "C" {

const char* oracle_last_error(void) { return g_error.c_str(); }

int oracle_dequantize_affine_rows(const uint32_t* packed, size_t packed_len,
                                  size_t rows, size_t packed_cols,
                                  const float* scales, size_t scales_len,
                                  const float* biases, size_t biases_len,
                                  uint32_t bits, uint32_t group_size,
                                  float* out) {
  return dequant_rows(packed, packed_len, rows, packed_cols, scales, scales_len,
                      biases, biases_len, bits, group_size, out);
}

// src/conversion/single_expert_pilot.cpp:276-358 -- affine q4 quantizer. The
// reference's source needs nlohmann/json to compile, so it is not part of the
// reference build; this restatement is pinned by the reference's own test
// (a round trip through the pinned dequant) and by the argmin and grid
// properties in tests/test_oracle_pinning.py.
int oracle_quantize_affine_q4_rows(const float* values, size_t values_len, size_t rows,
                                   size_t cols, size_t group, uint32_t* packed,
                                   float* scales, float* biases, float* max_abs_error,
                                   double* mean_abs_error) {
  if (rows == 0U || cols == 0U || group == 0U || cols % 8U != 0U || cols % group != 0U ||
      rows > std::numeric_limits<size_t>::max() / cols || values_len != rows * cols)
    return fail_invalid("affine q4 quantizer: invalid matrix geometry");
  const size_t words = cols / 8U;
  const size_t groups = cols / group;
  std::fill(packed, packed + rows * words, 0U);
  float worst = 0.0F;
  double total = 0.0;
  for (size_t r = 0; r < rows; ++r) {
    for (size_t gi = 0; gi < groups; ++gi) {
      const float* v = values + r * cols + gi * group;
      float lo = std::numeric_limits<float>::infinity();
      float hi = -std::numeric_limits<float>::infinity();
      for (size_t i = 0; i < group; ++i) {
        if (!std::isfinite(v[i])) return fail_runtime("affine q4 quantizer: non-finite source weight");
        lo = std::min(lo, v[i]);
        hi = std::max(hi, v[i]);
      }
      const float range = hi - lo;
      const float scale = range > 0.0F ? range / 15.0F : 1.0F;
      const float bias = lo;
      scales[r * groups + gi] = scale;
      biases[r * groups + gi] = bias;
      const float allowed = range > 0.0F ? scale * 0.5001F + 1e-6F : 1e-6F;
      for (size_t i = 0; i < group; ++i) {
        const size_t col = gi * group + i;
        const float t = (v[i] - bias) / scale;
        // std::lround rounds halves away from zero; NaN (an overflowed range)
        // maps to 0 here rather than to an implementation-defined integer.
        const long n = std::isnan(t) ? 0L : std::lround(t);
        const uint32_t q = static_cast<uint32_t>(std::clamp(n, 0L, 15L));
        packed[r * words + col / 8U] |= q << (4U * (col % 8U));
        const float err = std::fabs(scale * static_cast<float>(q) + bias - v[i]);
        if (err > allowed) return fail_runtime("affine q4 quantizer: error above the group bound");
        worst = std::max(worst, err);
        total += static_cast<double>(err);
      }
    }
  }
  *max_abs_error = worst;
  *mean_abs_error = total / static_cast<double>(rows * cols);
  return 0;
}

int oracle_matvec_row_major(const float* weight, size_t weight_len,
                            size_t out_dim, size_t in_dim, const float* x,
                            size_t x_len, float* out) {
  return matvec(weight, weight_len, out_dim, in_dim, x, x_len, out);
}

int oracle_rms_norm_inplace(float* values, size_t values_len, size_t rows,
                            size_t dim, const float* weight, size_t weight_len,
                            float eps) {
  return rms_norm(values, values_len, rows, dim, weight, weight_len, eps);
}

int oracle_softmax_inplace(float* values, size_t n) { return softmax(values, n); }

int oracle_route_top_k(const float* logits, size_t n, size_t k,
                       int normalize_selected, uint32_t* out_ids,
                       float* out_probs) {
  std::vector<Pick> picks;
  if (int rc = top_k(logits, n, k, normalize_selected != 0, picks)) return rc;
  for (size_t i = 0; i < picks.size(); ++i) {
    out_ids[i] = picks[i].id;
    out_probs[i] = picks[i].p;
  }
  return 0;
}

float oracle_sigmoid(float v) { return sigmoid_f(v); }
float oracle_silu(float v) { return silu_f(v); }

int oracle_swiglu_inplace(float* gate, size_t gate_len, const float* up,
                          size_t up_len) {
  if (gate_len != up_len) return fail_invalid("swiglu: gate/up size mismatch");
  for (size_t i = 0; i < gate_len; ++i) gate[i] = silu_f(gate[i]) * up[i];
  return 0;
}

int oracle_route_qwen_top_k(const float* hidden, size_t hidden_len,
                            const float* router_weight, size_t router_len,
                            size_t hidden_size, size_t expert_count,
                            size_t top_k_n, int norm_topk_prob,
                            float* out_logits, uint32_t* out_ids,
                            float* out_weights, float* out_mass) {
  std::vector<float> logits;
  std::vector<Pick> picks;
  float mass = 0.0F;
  if (int rc = route_qwen(hidden, hidden_len, router_weight, router_len,
                          hidden_size, expert_count, top_k_n,
                          norm_topk_prob != 0, logits, picks, mass))
    return rc;
  if (out_logits) std::memcpy(out_logits, logits.data(), logits.size() * sizeof(float));
  for (size_t i = 0; i < picks.size(); ++i) {
    out_ids[i] = picks[i].id;
    out_weights[i] = picks[i].p;
  }
  if (out_mass) *out_mass = mass;
  return 0;
}

int oracle_run_shared_expert(const float* hidden, size_t hidden_len,
                             const float* gate_proj, size_t gate_len,
                             const float* up_proj, size_t up_len,
                             const float* down_proj, size_t down_len,
                             const float* scalar_gate, size_t scalar_len,
                             size_t hidden_size, size_t intermediate_size,
                             float* out_values, float* out_scalar_gate) {
  return shared_expert(hidden, hidden_len, gate_proj, gate_len, up_proj, up_len,
                       down_proj, down_len, scalar_gate, scalar_len,
                       hidden_size, intermediate_size, out_values,
                       out_scalar_gate);
}

float oracle_bf16_to_float(uint16_t bits) { return bf16_widen(bits); }

int oracle_libm_expf_checksums(uint32_t first, uint64_t count, uint32_t block, uint64_t* out) {
  if (count == 0 || block == 0 || out == nullptr || static_cast<uint64_t>(first) + count > (1ULL << 32)) return 1;
  const uint64_t nblocks = (count + block - 1) / block;
  const unsigned nt = std::max(1U, std::thread::hardware_concurrency());
  std::vector<std::thread> workers;
  for (unsigned w = 0; w < nt; ++w)
    workers.emplace_back([=] {
      for (uint64_t b = w; b < nblocks; b += nt) {
        uint64_t s = 0;
        for (uint64_t i = 0; i < block && b * block + i < count; ++i) {
          const float x = std::bit_cast<float>(static_cast<uint32_t>(first + b * block + i));
          s += static_cast<uint64_t>(std::bit_cast<uint32_t>(std::exp(x))) * (2 * i + 1);
        }
        out[b] = s;
      }
    });
  for (auto& t : workers) t.join();
  return 0;
}
float oracle_f16_to_float(uint16_t bits) { return f16_widen(bits); }

size_t oracle_expert_blob_bytes(uint32_t hidden, uint32_t inter, uint32_t group,
                                int meta_dtype) {
  const size_t ms = meta_size(meta_dtype);
  const size_t gu = static_cast<size_t>(inter) * hidden / 8U * 4U +
                    2U * static_cast<size_t>(inter) * (hidden / group) * ms;
  const size_t dn = static_cast<size_t>(hidden) * inter / 8U * 4U +
                    2U * static_cast<size_t>(hidden) * (inter / group) * ms;
  return 2U * gu + dn;
}

int oracle_expert_forward(const uint8_t* blob, uint32_t hidden, uint32_t inter,
                          uint32_t group, int meta_dtype, const float* x,
                          float* out) {
  return expert_forward(blob, hidden, inter, group, meta_dtype, x, out);
}

int oracle_q4_gemv(const uint32_t* packed, size_t out_dim, size_t packed_cols,
                   const float* scales, const float* biases, size_t group_size,
                   const float* x, float* y) {
  if (group_size == 0U || (packed_cols * 8U) % group_size != 0U)
    return fail_invalid("Q4 GEMV input dimension must be divisible by group_size.");
  const size_t ng = out_dim * (packed_cols * 8U / group_size);
  std::vector<float> dense(out_dim * packed_cols * 8U);
  if (int rc = dequant_rows(packed, out_dim * packed_cols, out_dim, packed_cols,
                            scales, ng, biases, ng, 4U,
                            static_cast<uint32_t>(group_size), dense.data()))
    return rc;
  return matvec(dense.data(), dense.size(), out_dim, packed_cols * 8U, x,
                packed_cols * 8U, y);
}

int oracle_qwen_sparse_moe(const float* hidden, const float* router_f32,
                           uint32_t expert_count, uint32_t top_k_n,
                           int norm_topk_prob, const uint8_t* const* experts,
                           const uint8_t* shared_blob,
                           const float* shared_scalar_gate,
                           uint32_t hidden_size, uint32_t inter,
                           uint32_t group, int meta_dtype, float* out,
                           uint32_t* out_ids, float* out_weights,
                           float* out_mass, float* out_shared_gate,
                           float* out_logits) {
  return sparse_moe(hidden, router_f32, expert_count, top_k_n,
                    norm_topk_prob != 0, experts, shared_blob,
                    shared_scalar_gate, hidden_size, inter, group, meta_dtype,
                    out, out_ids, out_weights, out_mass, out_shared_gate,
                    out_logits);
}

// src/model/checkpoint_moe_sublayer.cpp:138-199 with add_residual_cpu
// (:21-33): normalised = RMSNorm(residual); out = residual + MoE(normalised).
int oracle_moe_sublayer(const float* residual, const float* norm_weight,
                        float eps, const float* router_f32,
                        uint32_t expert_count, uint32_t top_k_n,
                        int norm_topk_prob, const uint8_t* const* experts,
                        const uint8_t* shared_blob,
                        const float* shared_scalar_gate, uint32_t hidden_size,
                        uint32_t inter, uint32_t group, int meta_dtype,
                        float* out_normalized, float* out, uint32_t* out_ids,
                        float* out_weights, float* out_shared_gate) {
  std::vector<float> norm(residual, residual + hidden_size);
  if (int rc = rms_norm(norm.data(), hidden_size, 1U, hidden_size, norm_weight,
                        hidden_size, eps))
    return rc;
  std::vector<float> moe(hidden_size);
  if (int rc = sparse_moe(norm.data(), router_f32, expert_count, top_k_n,
                          norm_topk_prob != 0, experts, shared_blob,
                          shared_scalar_gate, hidden_size, inter, group,
                          meta_dtype, moe.data(), out_ids, out_weights, nullptr,
                          out_shared_gate, nullptr))
    return rc;
  for (uint32_t i = 0; i < hidden_size; ++i) out[i] = residual[i] + moe[i];
  if (out_normalized) std::memcpy(out_normalized, norm.data(), hidden_size * sizeof(float));
  return 0;
}

// The sublayer with the routed experts given instead of routed: RMSNorm
// (checkpoint_moe_sublayer.cpp:158-183), each pick's expert on the
// normalised input accumulated in pick order as acc + w * out
// (routed_moe.cpp:31-62), the sigmoid-gated shared expert added as
// sparse_moe adds it, then the residual (:21-33). pick_blobs[i] is pick i's
// expert blob.
int oracle_moe_sublayer_picks(const float* residual, const float* norm_weight, float eps, const float* weights,
                              uint32_t k, const uint8_t* const* pick_blobs, const uint8_t* shared_blob,
                              const float* shared_scalar_gate, uint32_t hidden_size, uint32_t inter, uint32_t group,
                              int meta_dtype, float* out) {
  std::vector<float> norm(residual, residual + hidden_size);
  if (int rc = rms_norm(norm.data(), hidden_size, 1U, hidden_size, norm_weight, hidden_size, eps)) return rc;
  std::vector<float> acc(hidden_size, 0.0F), e(hidden_size);
  for (uint32_t i = 0; i < k; ++i) {
    if (!std::isfinite(weights[i])) return fail_runtime("routed MoE encountered a non-finite routing weight");
    if (int rc = expert_forward(pick_blobs[i], hidden_size, inter, group, meta_dtype, norm.data(), e.data()))
      return rc;
    for (uint32_t j = 0; j < hidden_size; ++j) {
      const float prod = weights[i] * e[j];
      acc[j] = acc[j] + prod;
    }
  }
  if (shared_blob != nullptr) {
    float sg = 0.0F;
    if (int rc = shared_from_blob(shared_blob, shared_scalar_gate, hidden_size, inter, group, meta_dtype, norm.data(),
                                  e.data(), &sg))
      return rc;
    for (uint32_t j = 0; j < hidden_size; ++j) acc[j] = acc[j] + e[j];
  }
  for (uint32_t j = 0; j < hidden_size; ++j) out[j] = residual[j] + acc[j];
  return 0;
}

uint64_t oracle_synth_stream(uint64_t seed, uint32_t a, uint32_t b, uint32_t tensor) {
  return stream_of(seed, a, b, tensor);
}

float oracle_synth_normal(uint64_t stream, uint64_t index) { return normal_at(stream, index); }

void oracle_synth_expert_blob(uint64_t seed, uint32_t layer, uint32_t expert,
                              uint32_t hidden, uint32_t inter, uint32_t group,
                              int meta_dtype, uint8_t* out) {
  uint8_t* p = out;
  synth_projection(seed, layer, expert, kTGateQ, kTGateS, kTGateB, inter, hidden, group, meta_dtype, p);
  synth_projection(seed, layer, expert, kTUpQ, kTUpS, kTUpB, inter, hidden, group, meta_dtype, p);
  synth_projection(seed, layer, expert, kTDownQ, kTDownS, kTDownB, hidden, inter, group, meta_dtype, p);
}

void oracle_synth_router_bf16(uint64_t seed, uint32_t layer, uint32_t expert_count,
                              uint32_t hidden, uint16_t* out) {
  const uint64_t s = stream_of(seed, layer, kLayerTensorId, kTRouter);
  const size_t n = static_cast<size_t>(expert_count) * hidden;
  for (size_t i = 0; i < n; ++i) out[i] = bf16_rne(normal_at(s, i) * 0.02F);
}

void oracle_synth_shared_gate_bf16(uint64_t seed, uint32_t layer, uint32_t hidden,
                                   uint16_t* out) {
  const uint64_t s = stream_of(seed, layer, kLayerTensorId, kTSharedGate);
  for (uint32_t i = 0; i < hidden; ++i) out[i] = bf16_rne(normal_at(s, i) * 0.02F);
}

void oracle_synth_norm_weight(uint64_t seed, uint32_t layer, uint32_t hidden, float* out) {
  const uint64_t s = stream_of(seed, layer, kLayerTensorId, kTNorm);
  for (uint32_t i = 0; i < hidden; ++i) {
    const float n = normal_at(s, i) * 0.02F;
    out[i] = 1.0F + n;
  }
}

void oracle_synth_tokens(uint64_t seed, uint32_t first_token, uint32_t count,
                         uint32_t hidden, float* out) {
  for (uint32_t t = 0; t < count; ++t) {
    const uint64_t s = stream_of(seed, first_token + t, kTokenTensorId, kTTokens);
    for (uint32_t i = 0; i < hidden; ++i) out[static_cast<size_t>(t) * hidden + i] = normal_at(s, i);
  }
}

struct oracle_host_cache {
  HostCache c;
};

oracle_host_cache* oracle_host_cache_create(size_t stride, size_t budget, size_t minimum_slots) {
  if (stride == 0U) {
    g_error = "expert cache: storage stride must be non-zero";
    return nullptr;
  }
  if (budget / stride < minimum_slots) {
    g_error = "expert cache: budget cannot satisfy minimum slot count";
    return nullptr;
  }
  auto* h = new oracle_host_cache;
  h->c.stride = stride;
  h->c.budget = budget;
  h->c.max_slots = budget / stride;
  return h;
}

void oracle_host_cache_destroy(oracle_host_cache* c) { delete c; }

int oracle_host_cache_fetch(oracle_host_cache* h, uint32_t layer, const uint32_t* experts,
                            size_t n, int fail_read, uint64_t* out_slots, int* out_bytes_ok) {
  HostCache& c = h->c;
  if (out_bytes_ok) *out_bytes_ok = 1;
  if (n == 0U) return 0;
  {
    std::unordered_set<uint64_t> distinct;
    for (size_t i = 0; i < n; ++i) distinct.insert(HostCache::key_of(layer, experts[i]));
    if (distinct.size() > c.max_slots)
      return fail_runtime("expert cache: request contains more distinct experts than cache slots");
  }
  try {
    ++c.tick;
    std::unordered_set<size_t> used;
    std::vector<size_t> result(n);
    std::vector<std::pair<size_t, uint32_t>> fills;
    for (size_t i = 0; i < n; ++i) {
      const uint64_t key = HostCache::key_of(layer, experts[i]);
      const size_t f = c.freq[key] + 1U;
      c.freq[key] = f;
      auto it = c.where.find(key);
      if (it != c.where.end()) {
        ++c.hits;
        c.meta[it->second].freq = f;
        c.meta[it->second].last = c.tick;
        used.insert(it->second);
        result[i] = it->second;
        continue;
      }
      ++c.misses;
      const size_t slot = c.fill_slot(used);
      if (c.meta[slot].key.has_value()) c.where.erase(*c.meta[slot].key);
      c.meta[slot].key = key;
      c.meta[slot].freq = f;
      c.meta[slot].last = c.tick;
      c.where[key] = slot;
      used.insert(slot);
      result[i] = slot;
      fills.emplace_back(slot, experts[i]);
    }
    if (!fills.empty()) {
      ++c.storage_batches;
      if (fail_read) {
        for (const auto& [slot, e] : fills) {
          (void)e;
          if (c.meta[slot].key.has_value()) c.where.erase(*c.meta[slot].key);
          c.meta[slot].key.reset();
          c.meta[slot].freq = 0;
          c.meta[slot].last = 0;
        }
        return fail_runtime("synthetic read failure");
      }
      for (const auto& [slot, e] : fills)
        for (size_t i = 0; i < c.stride; ++i) c.slots[slot][i] = HostCache::pattern(layer, e, i);
    }
    for (size_t i = 0; i < n; ++i) {
      out_slots[i] = result[i];
      if (out_bytes_ok)
        for (size_t b = 0; b < c.stride; ++b)
          if (c.slots[result[i]][b] != HostCache::pattern(layer, experts[i], b)) *out_bytes_ok = 0;
    }
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return 2;
  }
}

int64_t oracle_host_cache_resident_slot(oracle_host_cache* h, uint32_t layer, uint32_t expert) {
  auto it = h->c.where.find(HostCache::key_of(layer, expert));
  return it == h->c.where.end() ? -1 : static_cast<int64_t>(it->second);
}

void oracle_host_cache_stats(oracle_host_cache* h, uint64_t* o) {
  const HostCache& c = h->c;
  o[0] = c.hits;
  o[1] = c.misses;
  o[2] = c.slots.size();
  o[3] = c.max_slots;
  o[4] = c.slots.size() * c.stride;
  o[5] = c.budget;
}

uint64_t oracle_host_cache_storage_batches(oracle_host_cache* h) { return h->c.storage_batches; }

struct oracle_device_cache {
  DeviceCache c;
};

oracle_device_cache* oracle_device_cache_create(size_t budget_bytes) {
  if (budget_bytes == 0U) {
    g_error = "resident expert cache: budget must be non-zero";
    return nullptr;
  }
  auto* h = new oracle_device_cache;
  h->c.budget = budget_bytes;
  return h;
}

void oracle_device_cache_destroy(oracle_device_cache* c) { delete c; }

int oracle_device_cache_get(oracle_device_cache* h, uint32_t layer, uint32_t expert,
                            size_t accounted_bytes, uint64_t* out_evicted, size_t cap,
                            size_t* out_n_evicted) {
  DeviceCache& c = h->c;
  if (out_n_evicted) *out_n_evicted = 0;
  try {
    ++c.tick;
    const uint64_t key = (static_cast<uint64_t>(layer) << 32) | expert;
    const size_t f = c.history[key] + 1U;
    c.history[key] = f;
    auto it = c.entries.find(key);
    if (it != c.entries.end()) {
      ++c.hits;
      it->second.freq = f;
      it->second.last = c.tick;
      return 1;
    }
    ++c.misses;
    if (accounted_bytes == 0U) {
      g_error = "resident expert cache: resident expert byte accounting is zero";
      return -1;
    }
    if (accounted_bytes > c.budget) {
      g_error = "resident expert cache: one expert exceeds the configured budget";
      return -1;
    }
    size_t ne = 0;
    while (!c.entries.empty() && c.resident + accounted_bytes > c.budget) {
      const uint64_t v = c.victim();
      auto vi = c.entries.find(v);
      c.resident -= vi->second.bytes;
      c.entries.erase(vi);
      ++c.evictions;
      if (ne < cap && out_evicted) out_evicted[ne] = v;
      ++ne;
    }
    if (out_n_evicted) *out_n_evicted = ne;
    c.entries.emplace(key, DeviceCache::Node{accounted_bytes, f, c.tick});
    c.resident += accounted_bytes;
    ++c.loads;
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return -2;
  }
}

int oracle_device_cache_contains(oracle_device_cache* h, uint32_t layer, uint32_t expert) {
  return h->c.entries.count((static_cast<uint64_t>(layer) << 32) | expert) ? 1 : 0;
}

void oracle_device_cache_stats(oracle_device_cache* h, uint64_t* o) {
  const DeviceCache& c = h->c;
  o[0] = c.hits;
  o[1] = c.misses;
  o[2] = c.loads;
  o[3] = c.evictions;
  o[4] = c.entries.size();
  o[5] = c.resident;
  o[6] = c.budget;
}

}  // extern "C"
