// synth.hip -- seeded synthetic weights and tokens, generated in HBM.
//
// A 48-layer expert stack is ~43.5 GB, too large to build on the host, so the
// benchmark and the full-size tests generate it on the device. Every element
// is a pure function of (seed, a, b, tensor, index): a SplitMix64-style
// finaliser over a counter, an Irwin-Hall(12) normal from twelve 16-bit
// draws scaled to unit variance (support +-6 sigma), and round-to-nearest-even to bf16. Only exact
// integer steps and separately rounded IEEE multiplies and adds are used
// (contraction is off for this file), so the same element computed on the
// host is bit-identical.
//
// Distributions (per expert projection): nibbles uniform on 0..15 (the low
// 32 bits of the hash); scale = bf16(|N(0,1)| * 0.02); bias =
// bf16(-8 * scale + N(0,1) * 0.002). Router and shared-gate vector:
// bf16(N(0,1) * 0.02). RMSNorm weight: 1 + N(0,1) * 0.02 (fp32). Tokens:
// N(0,1) (fp32).
#include "device_common.hpp"

// Every multiply and add below rounds on its own, as on the host: no fused
// multiply-add contraction anywhere in this file.
#pragma clang fp contract(off)

namespace {

using namespace osmk;

enum : uint32_t {
  kTGateQ = 0, kTGateS = 1, kTGateB = 2, kTUpQ = 3, kTUpS = 4, kTUpB = 5,
  kTDownQ = 6, kTDownS = 7, kTDownB = 8, kTRouter = 16, kTSharedGate = 17,
  kTNorm = 18, kTTokens = 32,
};
constexpr uint32_t kLayerTensorId = 0xFFFFFFFEu;
constexpr uint32_t kTokenTensorId = 0xFFFFFFFDu;

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__host__ __device__ __forceinline__ uint64_t stream_of(uint64_t seed, uint32_t a, uint32_t b,
                                                       uint32_t t) {
  return mix64(mix64(mix64(seed) ^ a) ^ ((static_cast<uint64_t>(b) << 8) | t));
}

// Sum of the four 16-bit fields of a 64-bit hash.
__device__ __forceinline__ uint32_t fields16(uint64_t h) {
  return static_cast<uint32_t>((h & 0xFFFFu) + ((h >> 16) & 0xFFFFu) + ((h >> 32) & 0xFFFFu) +
                               (h >> 48));
}

// Irwin-Hall(12): twelve 16-bit uniforms from three chained hashes. The sum
// has mean 393210 and standard deviation sqrt(2^32 - 1), which is 2^16 to
// within 6e-11, so one exact multiply by 2^-16 gives unit variance with
// support [-6, 6].
__device__ __forceinline__ float normal_at(uint64_t stream, uint64_t i) {
  const uint64_t h0 = mix64(stream + i), h1 = mix64(h0), h2 = mix64(h1);
  const int32_t s = static_cast<int32_t>(fields16(h0) + fields16(h1) + fields16(h2));
  return static_cast<float>(s - 393210) * 0x1p-16f;
}

__device__ __forceinline__ uint16_t bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

struct ProjSpec {
  uint32_t tq, ts, tb;
  size_t q_off, s_off, b_off;
  size_t words, groups;
};

// grid.y = expert index within the batch; grid.x strides over elements.
__global__ void synth_words_kernel(uint64_t seed, uint32_t layer, uint32_t first_expert,
                                   uint8_t* dst, size_t stride, ProjSpec ps) {
  const uint32_t e = first_expert + blockIdx.y;
  const uint64_t sq = stream_of(seed, layer, e, ps.tq);
  uint32_t* out = reinterpret_cast<uint32_t*>(dst + blockIdx.y * stride + ps.q_off);
  const size_t step = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < ps.words; i += step)
    out[i] = static_cast<uint32_t>(mix64(sq + i));
}

__global__ void synth_meta_kernel(uint64_t seed, uint32_t layer, uint32_t first_expert,
                                  uint8_t* dst, size_t stride, ProjSpec ps, uint32_t meta_dtype) {
  const uint32_t e = first_expert + blockIdx.y;
  const uint64_t ss = stream_of(seed, layer, e, ps.ts);
  const uint64_t sb = stream_of(seed, layer, e, ps.tb);
  uint8_t* base = dst + blockIdx.y * stride;
  const size_t step = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < ps.groups; i += step) {
    const uint16_t sbits = bf16_rne(fabsf(normal_at(ss, i)) * 0.02f);
    const float sval = bf16_to_f32(sbits);
    const float noise = normal_at(sb, i) * 0.002f;
    const uint16_t bbits = bf16_rne(-8.0f * sval + noise);
    if (meta_dtype == OSM_META_F32) {
      reinterpret_cast<float*>(base + ps.s_off)[i] = sval;
      reinterpret_cast<float*>(base + ps.b_off)[i] = bf16_to_f32(bbits);
    } else {
      reinterpret_cast<uint16_t*>(base + ps.s_off)[i] = sbits;
      reinterpret_cast<uint16_t*>(base + ps.b_off)[i] = bbits;
    }
  }
}

__global__ void synth_bf16_kernel(uint64_t stream, size_t n, float sigma, uint16_t* out) {
  const size_t step = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step)
    out[i] = bf16_rne(normal_at(stream, i) * sigma);
}

__global__ void synth_norm_kernel(uint64_t stream, uint32_t n, float* out) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = 1.0f + normal_at(stream, i) * 0.02f;
}

__global__ void synth_tokens_kernel(uint64_t seed, uint32_t first_token, uint32_t hidden,
                                    float* out) {
  const uint64_t s = stream_of(seed, first_token + blockIdx.y, kTokenTensorId, kTTokens);
  float* row = out + static_cast<size_t>(blockIdx.y) * hidden;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
    row[i] = normal_at(s, i);
}

unsigned blocks_for(size_t n) {
  size_t b = (n + 255) / 256;
  if (b == 0) b = 1;
  if (b > 2048) b = 2048;
  return static_cast<unsigned>(b);
}

}  // namespace

extern "C" {

int osmd_synth_expert_blobs(uint64_t seed, uint32_t layer, uint32_t first_expert, uint32_t count,
                            osm_expert_geometry g, uint8_t* dst, size_t stride, osmd_stream s) {
  if (count == 0) return 0;
  const hipStream_t st = static_cast<hipStream_t>(s);
  const osm_expert_offsets off = osm_expert_layout(g);
  const size_t gu_words = static_cast<size_t>(g.inter) * g.hidden / 8u;
  const size_t gu_groups = static_cast<size_t>(g.inter) * (g.hidden / g.group);
  const size_t dn_words = static_cast<size_t>(g.hidden) * g.inter / 8u;
  const size_t dn_groups = static_cast<size_t>(g.hidden) * (g.inter / g.group);
  const ProjSpec specs[3] = {
      {kTGateQ, kTGateS, kTGateB, off.gate_q, off.gate_s, off.gate_b, gu_words, gu_groups},
      {kTUpQ, kTUpS, kTUpB, off.up_q, off.up_s, off.up_b, gu_words, gu_groups},
      {kTDownQ, kTDownS, kTDownB, off.down_q, off.down_s, off.down_b, dn_words, dn_groups},
  };
  // Experts go in chunks of up to 65535 along grid.y.
  for (uint32_t e0 = 0; e0 < count; e0 += 65535u) {
    const uint32_t n = (count - e0 < 65535u) ? count - e0 : 65535u;
    uint8_t* d = dst + static_cast<size_t>(e0) * stride;
    for (const ProjSpec& ps : specs) {
      synth_words_kernel<<<dim3(blocks_for(ps.words) > 64 ? 64 : blocks_for(ps.words), n), 256, 0, st>>>(
          seed, layer, first_expert + e0, d, stride, ps);
      synth_meta_kernel<<<dim3(blocks_for(ps.groups) > 16 ? 16 : blocks_for(ps.groups), n), 256, 0, st>>>(
          seed, layer, first_expert + e0, d, stride, ps, g.meta_dtype);
    }
  }
  return launch_status();
}

int osmd_synth_router_bf16(uint64_t seed, uint32_t layer, uint32_t experts, uint32_t hidden,
                           uint16_t* dst, osmd_stream s) {
  const size_t n = static_cast<size_t>(experts) * hidden;
  synth_bf16_kernel<<<blocks_for(n), 256, 0, static_cast<hipStream_t>(s)>>>(
      stream_of(seed, layer, kLayerTensorId, kTRouter), n, 0.02f, dst);
  return launch_status();
}

int osmd_synth_shared_gate_bf16(uint64_t seed, uint32_t layer, uint32_t hidden, uint16_t* dst,
                                osmd_stream s) {
  synth_bf16_kernel<<<blocks_for(hidden), 256, 0, static_cast<hipStream_t>(s)>>>(
      stream_of(seed, layer, kLayerTensorId, kTSharedGate), hidden, 0.02f, dst);
  return launch_status();
}

int osmd_synth_norm_weight(uint64_t seed, uint32_t layer, uint32_t hidden, float* dst,
                           osmd_stream s) {
  synth_norm_kernel<<<(hidden + 255) / 256, 256, 0, static_cast<hipStream_t>(s)>>>(
      stream_of(seed, layer, kLayerTensorId, kTNorm), hidden, dst);
  return launch_status();
}

int osmd_synth_tokens(uint64_t seed, uint32_t first_token, uint32_t count, uint32_t hidden,
                      float* dst, osmd_stream s) {
  if (count == 0) return 0;
  synth_tokens_kernel<<<dim3((hidden + 255) / 256, count), 256, 0, static_cast<hipStream_t>(s)>>>(
      seed, first_token, hidden, dst);
  return launch_status();
}

}  // extern "C"
