// moe_grouped.hip -- the routed-MoE sublayer for many tokens at once
// (decode batches and prefill chunks) as grouped GEMMs on the matrix cores.
//
// The reference has no multi-token MoE: its sessions push tokens through the
// sublayer one at a time (src/session/greedy_token_session.cpp:170-192), so a
// batch is the per-token loop of run_qwen_sparse_moe_vulkan_accum
// (src/model/routed_moe.cpp:254-430). Here every (token, slot) pair is
// bucketed by expert and each expert's weights are read once for all of its
// tokens:
//
//   prepare      x (fp32 or bf16) -> bf16 split terms, per-group sums
//   router GEMM  logits = x . router^T (3 split terms: fp32-equivalent)
//   select       per-token top-k (the decode path's selection kernel)
//   bucket       per-expert counts, offsets, pair positions, tile list
//   gate/up      per tile: SwiGLU(x W_gate^T, x W_up^T) -> h [pair, I]
//   prepare      h -> bf16 split terms, per-group sums
//   down         per tile: weight * (h W_down^T) -> partial [pair, D]
//   combine      y[t] = sum over slots in pick order, shared last (+ x)
//
// MFMA operands. v_mfma_f32_16x16x32_bf16: A is 16 rows x 32 k, B is 32 k x
// 16 columns, D is 16 x 16 fp32; lane l holds A row l%16 and B column l%16
// for k-slot l/16 (8 consecutive k), and D rows 4*(l/16)..+3 of column l%16.
// Here A rows are tokens and B columns are weight rows, so a lane's D values
// share one weight row and need one scale and bias per group.
//
// A packed weight word (8 nibbles) is one lane's B operand: with
// p_j = ((w >> 4j) & 0x000F000F) | 0x43004300 each 16-bit half is the bf16
// value 128 + q, exactly, for nibbles (j, j+4). The k order inside a word is
// therefore [0,4,1,5,2,6,3,7]; activation terms are stored in that order so A
// and B agree. The +128 is folded into the group's bias term:
// s*sum(q*x) + b*sum(x) = s*D + (b - 128*s)*sum(x).
//
// Activations are split into bf16 terms t_0 + t_1 + ... (t_0 = bf16(x),
// t_1 = bf16(x - t_0), ...), each term one more MFMA into the same
// accumulator: products of bf16 pairs are exact in fp32, so 2 terms carry 16
// significant bits and 3 terms all 24.
#include "device_common.hpp"

namespace {

using namespace osmk;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kTileTokens = 16;  // MFMA rows (tokens or pairs)
constexpr uint32_t kBlockRows = 16;   // MFMA columns (weight rows)
constexpr uint32_t kGroupedWaves = 4;
constexpr uint32_t kGroupedThreads = kGroupedWaves * kWave;
constexpr uint32_t kRowBlocksPerWave = 2;
constexpr uint32_t kRowsPerWorkgroup = kGroupedWaves * kRowBlocksPerWave * kBlockRows;  // 128
constexpr uint32_t kRouterSplit = 3;
constexpr uint32_t kRouterGemmMinTokens = 64;
constexpr uint32_t kActSplit = 2;

__device__ __forceinline__ uint16_t bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// k position inside a packed word of operand element e (see header).
__device__ __forceinline__ constexpr int word_k(int e) { return (e >> 1) + ((e & 1) << 2); }

__device__ __forceinline__ bf16x8 as_operand(uint4 v) {
  const u32x4 u = {v.x, v.y, v.z, v.w};
  return __builtin_bit_cast(bf16x8, u);
}

__device__ __forceinline__ bf16x8 nibble_operand(uint32_t w) {
  const uint32_t m = 0x000F000Fu, bias = 0x43004300u;
  const u32x4 v = {(w & m) | bias, ((w >> 4) & m) | bias, ((w >> 8) & m) | bias, ((w >> 12) & m) | bias};
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// prepare: rows [R, K] (fp32, or bf16 when XBF16) -> terms [R][NS][K] bf16 in
// word order and sums [R][K/G] of the values the terms represent. One thread
// per (row, group).
template <bool XBF16, int NS>
__global__ void prepare_kernel(const void* __restrict__ x, uint32_t R, uint32_t K, uint32_t G,
                               uint16_t* __restrict__ terms, float* __restrict__ sums) {
  const uint32_t groups = K / G;
  const size_t n = static_cast<size_t>(R) * groups;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint32_t r = static_cast<uint32_t>(i / groups), g = static_cast<uint32_t>(i % groups);
    float total = 0.0f;
    for (uint32_t wd = g * (G / 8u); wd < (g + 1u) * (G / 8u); ++wd) {
      float v[8];
      if constexpr (XBF16) {
        const uint4 raw = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + static_cast<size_t>(r) * K + wd * 8u);
        const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[2 * j] = bf16_to_f32(w4[j] & 0xFFFFu);
          v[2 * j + 1] = bf16_to_f32(w4[j] >> 16);
        }
      } else {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + static_cast<size_t>(r) * K + wd * 8u);
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
      }
      float rep[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        uint16_t out[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int k = word_k(e);
          out[e] = bf16_rne(v[k] - rep[k]);
          rep[k] += bf16_to_f32(out[e]);
        }
        uint4 pk;
        pk.x = out[0] | (static_cast<uint32_t>(out[1]) << 16);
        pk.y = out[2] | (static_cast<uint32_t>(out[3]) << 16);
        pk.z = out[4] | (static_cast<uint32_t>(out[5]) << 16);
        pk.w = out[6] | (static_cast<uint32_t>(out[7]) << 16);
        *reinterpret_cast<uint4*>(terms + (static_cast<size_t>(r) * NS + s) * K + wd * 8u) = pk;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) total += rep[k];
    }
    sums[i] = total;
  }
}

// ---------------------------------------------------------------------------
// Router GEMM: logits [T, E] and, as row E, the shared gate sigmoid(w_sg . x).
// Workgroup = 16 tokens x 4 waves x 16 router rows (bf16).
template <int NS>
__global__ __launch_bounds__(kGroupedThreads) void router_gemm_kernel(
    const uint16_t* __restrict__ terms, uint32_t T, uint32_t D, const uint16_t* __restrict__ router,
    const uint16_t* __restrict__ shared_gate_vec, uint32_t E, float* __restrict__ logits,
    float* __restrict__ shared_gate) {
  const uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const uint32_t t0 = blockIdx.y * kTileTokens;
  const uint32_t nrows = E + (shared_gate_vec ? 1u : 0u);
  const uint32_t m = lane % 16u, q = lane / 16u;
  const uint32_t row = (blockIdx.x * kGroupedWaves + wave) * kBlockRows + m;
  const uint32_t rr = row < nrows ? row : nrows - 1u;
  const uint16_t* wrow = rr < E ? router + static_cast<size_t>(rr) * D : shared_gate_vec;
  const uint32_t tok = (t0 + m < T) ? t0 + m : T - 1u;
  const uint16_t* arow = terms + static_cast<size_t>(tok) * NS * D;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (uint32_t k0 = 0; k0 < D; k0 += 32u) {
    // B: 8 router values of row rr at k0 + 8q, reordered to word order.
    const uint4 raw = ldg16(wrow + k0 + 8u * q);
    const uint32_t h4[4] = {raw.x, raw.y, raw.z, raw.w};
    uint16_t h[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h[2 * j] = static_cast<uint16_t>(h4[j] & 0xFFFFu);
      h[2 * j + 1] = static_cast<uint16_t>(h4[j] >> 16);
    }
    uint4 bv;
    bv.x = h[word_k(0)] | (static_cast<uint32_t>(h[word_k(1)]) << 16);
    bv.y = h[word_k(2)] | (static_cast<uint32_t>(h[word_k(3)]) << 16);
    bv.z = h[word_k(4)] | (static_cast<uint32_t>(h[word_k(5)]) << 16);
    bv.w = h[word_k(6)] | (static_cast<uint32_t>(h[word_k(7)]) << 16);
    const bf16x8 b = as_operand(bv);
#pragma unroll
    for (int s = 0; s < NS; ++s) acc = mfma(as_operand(ldg16(arow + static_cast<size_t>(s) * D + k0 + 8u * q)), b, acc);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {  // D rows 4q + j are tokens, column m the router row
    const uint32_t t = t0 + 4u * q + j;
    if (t < T && row < nrows) {
      if (row < E)
        logits[static_cast<size_t>(t) * E + row] = acc[j];
      else
        shared_gate[t] = 1.0f / (1.0f + expf(-acc[j]));  // reference_ops.cpp:214-216
    }
  }
}

// ---------------------------------------------------------------------------
// bucket: one workgroup. Pair i = token * nslot + slot; slot < k is routed to
// ids[t, slot], slot k (when there is a shared expert) to bucket E. Pairs of
// one bucket land contiguously; their order inside it does not matter, since
// every output row depends only on its own token. Tiles of up to 16 pairs
// cover each non-empty bucket.
struct Tile {
  uint32_t expert, start, count, pad;
};

constexpr uint32_t kBucketThreads = 1024;
constexpr uint32_t kMaxBuckets = OSMD_MAX_EXPERTS + 1u;

__global__ __launch_bounds__(kBucketThreads) void bucket_kernel(
    const uint32_t* __restrict__ ids, const float* __restrict__ weights, const float* __restrict__ shared_gate,
    uint32_t T, uint32_t k, uint32_t nslot, uint32_t E, uint32_t* __restrict__ perm,
    uint32_t* __restrict__ pair_pos, float* __restrict__ pair_w, Tile* __restrict__ tiles,
    uint32_t* __restrict__ tile_count) {
  __shared__ uint32_t counts[kMaxBuckets], offsets[kMaxBuckets], cursor[kMaxBuckets], tbase[kMaxBuckets];
  __shared__ uint32_t scan[kBucketThreads];
  const uint32_t tid = threadIdx.x;
  const uint32_t nb = E + (nslot > k ? 1u : 0u);
  const uint32_t P = T * nslot;
  for (uint32_t b = tid; b < nb; b += kBucketThreads) counts[b] = 0u, cursor[b] = 0u;
  __syncthreads();
  for (uint32_t i = tid; i < P; i += kBucketThreads) {
    const uint32_t t = i / nslot, j = i % nslot;
    uint32_t e = j < k ? ids[static_cast<size_t>(t) * k + j] : E;
    e = e < nb ? e : nb - 1u;
    atomicAdd(&counts[e], 1u);
  }
  __syncthreads();
  // Exclusive scans of the counts and of the tile counts, two buckets per
  // thread at most (nb <= 1025).
  for (int pass = 0; pass < 2; ++pass) {
    uint32_t local = 0;
    for (uint32_t b = tid * 2u; b < tid * 2u + 2u && b < nb; ++b)
      local += pass == 0 ? counts[b] : (counts[b] + kTileTokens - 1u) / kTileTokens;
    scan[tid] = local;
    __syncthreads();
    for (uint32_t off = 1; off < kBucketThreads; off <<= 1) {
      const uint32_t v = tid >= off ? scan[tid - off] : 0u;
      __syncthreads();
      scan[tid] += v;
      __syncthreads();
    }
    uint32_t run = scan[tid] - local;
    for (uint32_t b = tid * 2u; b < tid * 2u + 2u && b < nb; ++b) {
      if (pass == 0) {
        offsets[b] = run;
        run += counts[b];
      } else {
        tbase[b] = run;
        run += (counts[b] + kTileTokens - 1u) / kTileTokens;
      }
    }
    if (pass == 1 && tid == kBucketThreads - 1u) *tile_count = scan[tid];
    __syncthreads();
  }
  for (uint32_t b = tid; b < nb; b += kBucketThreads) {
    const uint32_t n = counts[b];
    for (uint32_t s = 0; s * kTileTokens < n; ++s) {
      Tile tl;
      tl.expert = b;
      tl.start = offsets[b] + s * kTileTokens;
      tl.count = n - s * kTileTokens < kTileTokens ? n - s * kTileTokens : kTileTokens;
      tl.pad = 0u;
      tiles[tbase[b] + s] = tl;
    }
  }
  for (uint32_t i = tid; i < P; i += kBucketThreads) {
    const uint32_t t = i / nslot, j = i % nslot;
    uint32_t e = j < k ? ids[static_cast<size_t>(t) * k + j] : E;
    e = e < nb ? e : nb - 1u;
    const uint32_t pos = offsets[e] + atomicAdd(&cursor[e], 1u);
    perm[pos] = i;
    pair_pos[i] = pos;
    pair_w[pos] = j < k ? weights[static_cast<size_t>(t) * k + j] : (shared_gate ? shared_gate[t] : 1.0f);
  }
}

// ---------------------------------------------------------------------------
// Grouped q4 GEMM over the tile list. Workgroup = one tile (<= 16 pairs) x
// 128 weight rows (4 waves x 2 blocks of 16). PROJ == 2: gate and up with
// SwiGLU -> h[pair, row]; PROJ == 1: down, times the pair's weight ->
// out[pair, row]. A rows: the pair's token (PROJ 2) or the pair (PROJ 1).
//
// K runs in chunks of 32 * NSTEP columns. The A chunk (both bf16 terms of the
// tile's 16 rows) and its group sums are staged in LDS, double-buffered, and
// shared by the four waves; each wave keeps the next chunk's packed words and
// metadata in flight in registers while it multiplies the current one, so a
// chunk's memory latency hides behind the previous chunk's MFMAs.
//
// S = G / 32 MFMA steps per group; lane k-slot q uses words S*q .. S*q+S-1
// of each group (step s: word S*q + s), so one lane load covers a group.
struct GroupedParams {
  osm_expert_geometry g;
  const uint16_t* terms;  // A terms [rows][kActSplit][K]
  const float* sums;      // [rows][K/G]
  const uint32_t* perm;   // [P] pair -> token * nslot + slot
  const float* pair_w;    // [P]
  const Tile* tiles;
  const uint32_t* tile_count;
  const uint8_t* const* expert_table;  // [E]
  const uint8_t* shared_expert;        // bucket E
  const uint8_t* fallback;
  uint32_t expert_count, nslot;
  float* out;  // [P][N]
};

// Metadata of GPC consecutive groups of one row, kept as loaded: 16-bit
// values two to a register (bf16 / f16), f32 one to a register.
template <int META, int GPC>
struct MetaRun {
  static constexpr int kRegs = META == OSM_META_F32 ? GPC : (GPC + 1) / 2;
  uint32_t r[kRegs];
  __device__ __forceinline__ void load(const uint8_t* base, size_t idx) {
    if constexpr (META != OSM_META_F32 && GPC == 4) {
      const uint2 v = ldg8(base + idx * 2u);
      r[0] = v.x;
      r[1] = v.y;
    } else if constexpr (META == OSM_META_F32 && GPC == 4) {
      const uint4 v = ldg16(base + idx * 4u);
      r[0] = v.x; r[1] = v.y; r[2] = v.z; r[3] = v.w;
    } else if constexpr (META == OSM_META_F32) {
#pragma unroll
      for (int i = 0; i < GPC; ++i) r[i] = meta_bits<META>(base, idx + i);
    } else {
#pragma unroll
      for (int i = 0; i < kRegs; ++i) {
        const uint32_t lo = meta_bits<META>(base, idx + 2 * i);
        const uint32_t hi = 2 * i + 1 < GPC ? meta_bits<META>(base, idx + 2 * i + 1) : 0u;
        r[i] = lo | (hi << 16);
      }
    }
  }
  __device__ __forceinline__ float get(int i) const {
    if constexpr (META == OSM_META_F32)
      return __uint_as_float(r[i]);
    else
      return meta_widen<META>((r[i >> 1] >> (16 * (i & 1))) & 0xFFFFu);
  }
};

template <int S>
__device__ __forceinline__ void word_run(const uint8_t* p, uint32_t* out) {
  if constexpr (S == 4) {
    const uint4 v = ldg16(p);
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  } else if constexpr (S == 2) {
    const uint2 v = ldg8(p);
    out[0] = v.x; out[1] = v.y;
  } else {
    out[0] = ldg<uint32_t>(p);
  }
}

template <int META, int PROJ, int S, int NSTEP>
__global__ __launch_bounds__(kGroupedThreads) void grouped_kernel(GroupedParams p) {
  constexpr int GPC = NSTEP / S;        // groups per chunk
  constexpr uint32_t KC = 32u * NSTEP;  // columns per chunk
  constexpr uint32_t RS = KC + 8u;      // LDS row stride (bf16), padded against bank conflicts
  constexpr uint32_t kU4PerChunk = kActSplit * kTileTokens * KC / 8u;
  __shared__ __align__(16) uint16_t a_lds[2][kActSplit][kTileTokens][RS];
  __shared__ __align__(16) float xs_lds[2][GPC][kTileTokens];
  __shared__ uint32_t arow_lds[kTileTokens];

  const uint32_t tile_idx = blockIdx.x;
  if (tile_idx >= *p.tile_count) return;  // uniform over the workgroup
  const Tile tl = p.tiles[tile_idx];
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid % kWave, wave = tid / kWave;
  const uint32_t m = lane % 16u, q = lane / 16u;
  const uint32_t D = p.g.hidden, I = p.g.inter, G = p.g.group;
  const uint32_t K = PROJ == 2 ? D : I;
  const uint32_t N = PROJ == 2 ? I : D;
  const uint32_t ngroups = K / G;
  const uint32_t nchunks = K / KC;
  const osm_expert_offsets off = osm_expert_layout(p.g);

  const uint8_t* blob = tl.expert < p.expert_count ? p.expert_table[tl.expert] : p.shared_expert;
  if (blob == nullptr) blob = p.fallback;

  if (tid < kTileTokens) {  // A source row of each tile row (clamped into the tile)
    const uint32_t pair = tl.start + (tid < tl.count ? tid : tl.count - 1u);
    arow_lds[tid] = PROJ == 2 ? p.perm[pair] / p.nslot : pair;
  }
  __syncthreads();

  uint32_t wrow[kRowBlocksPerWave];
#pragma unroll
  for (uint32_t nb = 0; nb < kRowBlocksPerWave; ++nb) {
    const uint32_t r = blockIdx.y * kRowsPerWorkgroup + (wave * kRowBlocksPerWave + nb) * kBlockRows + m;
    wrow[nb] = r < N ? r : N - 1u;
  }
  const size_t q_off[2] = {PROJ == 2 ? off.gate_q : off.down_q, off.up_q};
  const size_t s_off[2] = {PROJ == 2 ? off.gate_s : off.down_s, off.up_s};
  const size_t b_off[2] = {PROJ == 2 ? off.gate_b : off.down_b, off.up_b};
  const size_t row_bytes = static_cast<size_t>(K) / 2u;

  // Register sets: packed words and metadata of one chunk.
  struct WSet {
    uint32_t w[kRowBlocksPerWave][PROJ][NSTEP];
    MetaRun<META, GPC> sb[kRowBlocksPerWave][PROJ], bb[kRowBlocksPerWave][PROJ];
  };
  auto load_w = [&](uint32_t c, WSet& W) {
    const uint32_t g0 = c * GPC;
#pragma unroll
    for (uint32_t nb = 0; nb < kRowBlocksPerWave; ++nb)
#pragma unroll
      for (int pr = 0; pr < PROJ; ++pr) {
        const uint8_t* qrow = blob + q_off[pr] + static_cast<size_t>(wrow[nb]) * row_bytes;
#pragma unroll
        for (int gg = 0; gg < GPC; ++gg)
          word_run<S>(qrow + ((g0 + gg) * (G / 8u) + S * q) * 4u, &W.w[nb][pr][gg * S]);
        const size_t mi = static_cast<size_t>(wrow[nb]) * ngroups + g0;
        W.sb[nb][pr].load(blob + s_off[pr], mi);
        W.bb[nb][pr].load(blob + b_off[pr], mi);
      }
  };
  // A chunk: 16-byte units, thread tid takes units tid, tid + 256, ...
  constexpr uint32_t kU4PerThread = (kU4PerChunk + kGroupedThreads - 1) / kGroupedThreads;
  uint4 areg[kU4PerThread];
  float xreg = 0.0f;
  auto load_a = [&](uint32_t c) {
    const uint32_t k0 = c * KC;
#pragma unroll
    for (uint32_t i = 0; i < kU4PerThread; ++i) {
      const uint32_t u = tid + i * kGroupedThreads;
      if (u < kU4PerChunk) {
        const uint32_t term = u / (kTileTokens * KC / 8u);
        const uint32_t rem = u % (kTileTokens * KC / 8u);
        const uint32_t row = rem / (KC / 8u), cu = rem % (KC / 8u);
        areg[i] = ldg16(p.terms + (static_cast<size_t>(arow_lds[row]) * kActSplit + term) * K + k0 + cu * 8u);
      }
    }
    if (tid < GPC * kTileTokens)
      xreg = p.sums[static_cast<size_t>(arow_lds[tid % kTileTokens]) * ngroups + c * GPC + tid / kTileTokens];
  };
  auto store_a = [&](uint32_t buf) {
#pragma unroll
    for (uint32_t i = 0; i < kU4PerThread; ++i) {
      const uint32_t u = tid + i * kGroupedThreads;
      if (u < kU4PerChunk) {
        const uint32_t term = u / (kTileTokens * KC / 8u);
        const uint32_t rem = u % (kTileTokens * KC / 8u);
        const uint32_t row = rem / (KC / 8u), cu = rem % (KC / 8u);
        *reinterpret_cast<uint4*>(&a_lds[buf][term][row][cu * 8u]) = areg[i];
      }
    }
    if (tid < GPC * kTileTokens) xs_lds[buf][tid / kTileTokens][tid % kTileTokens] = xreg;
  };

  f32x4 total[kRowBlocksPerWave][PROJ];
#pragma unroll
  for (uint32_t nb = 0; nb < kRowBlocksPerWave; ++nb)
#pragma unroll
    for (int pr = 0; pr < PROJ; ++pr) total[nb][pr] = f32x4{0.f, 0.f, 0.f, 0.f};

  WSet cur, nxt;
  load_w(0, cur);
  load_a(0);
  store_a(0);
  __syncthreads();
  for (uint32_t c = 0; c < nchunks; ++c) {
    const uint32_t buf = c & 1u;
    const bool more = c + 1u < nchunks;
    if (more) {
      load_w(c + 1u, nxt);
      load_a(c + 1u);
    }
#pragma unroll
    for (int gg = 0; gg < GPC; ++gg) {
      bf16x8 a[S][kActSplit];
#pragma unroll
      for (int s2 = 0; s2 < S; ++s2)
#pragma unroll
        for (uint32_t t = 0; t < kActSplit; ++t)
          a[s2][t] = as_operand(*reinterpret_cast<const uint4*>(&a_lds[buf][t][m][(gg * (G / 8u) + S * q + s2) * 8u]));
      const float4 xs = *reinterpret_cast<const float4*>(&xs_lds[buf][gg][4u * q]);
#pragma unroll
      for (uint32_t nb = 0; nb < kRowBlocksPerWave; ++nb)
#pragma unroll
        for (int pr = 0; pr < PROJ; ++pr) {
          f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s2 = 0; s2 < S; ++s2) {
            const bf16x8 b = nibble_operand(cur.w[nb][pr][gg * S + s2]);
#pragma unroll
            for (uint32_t t = 0; t < kActSplit; ++t) d = mfma(a[s2][t], b, d);
          }
          const float sc = cur.sb[nb][pr].get(gg);
          const float cb = cur.bb[nb][pr].get(gg) - 128.0f * sc;
          total[nb][pr][0] += sc * d[0] + cb * xs.x;
          total[nb][pr][1] += sc * d[1] + cb * xs.y;
          total[nb][pr][2] += sc * d[2] + cb * xs.z;
          total[nb][pr][3] += sc * d[3] + cb * xs.w;
        }
    }
    if (more) store_a(buf ^ 1u);
    __syncthreads();
    if (more) cur = nxt;
  }

#pragma unroll
  for (uint32_t nb = 0; nb < kRowBlocksPerWave; ++nb) {
    const uint32_t r = blockIdx.y * kRowsPerWorkgroup + (wave * kRowBlocksPerWave + nb) * kBlockRows + m;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t pj = 4u * q + j;
      if (pj < tl.count && r < N) {
        const size_t o = static_cast<size_t>(tl.start + pj) * N + r;
        if constexpr (PROJ == 2)
          p.out[o] = silu_mul(total[nb][0][j], total[nb][1][j]);
        else
          p.out[o] = p.pair_w[tl.start + pj] * total[nb][0][j];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// combine: y[t, r] = sum over slots 0..nslot-1 of partial[pos(t, slot), r]
// (routed picks in pick order, the shared expert last), plus x when the
// residual form is asked for.
__global__ void combine_kernel(const float* __restrict__ partial, const uint32_t* __restrict__ pair_pos,
                               uint32_t T, uint32_t D, uint32_t nslot, const float* __restrict__ residual,
                               float* __restrict__ y) {
  const size_t n = static_cast<size_t>(T) * D;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint32_t t = static_cast<uint32_t>(i / D), r = static_cast<uint32_t>(i % D);
    float acc = 0.0f;
    for (uint32_t j = 0; j < nslot; ++j) acc += partial[static_cast<size_t>(pair_pos[t * nslot + j]) * D + r];
    y[i] = residual ? residual[i] + acc : acc;
  }
}

template <int META, int PROJ, int S>
void launch_grouped_s(const GroupedParams& gp, dim3 grid, hipStream_t st) {
  // gate/up keep two projections' words in flight: 128-column chunks keep
  // the registers under 256 (two waves per SIMD); down takes 256 columns.
  const uint32_t K = PROJ == 2 ? gp.g.hidden : gp.g.inter;
  if (PROJ == 1 && K % 256u == 0)
    grouped_kernel<META, PROJ, S, 8><<<grid, kGroupedThreads, 0, st>>>(gp);
  else
    grouped_kernel<META, PROJ, S, 4><<<grid, kGroupedThreads, 0, st>>>(gp);  // K % 128 == 0
}

template <int META, int PROJ>
void launch_grouped_meta(const GroupedParams& gp, dim3 grid, hipStream_t st) {
  switch (gp.g.group) {
    case 32: launch_grouped_s<META, PROJ, 1>(gp, grid, st); break;
    case 64: launch_grouped_s<META, PROJ, 2>(gp, grid, st); break;
    default: launch_grouped_s<META, PROJ, 4>(gp, grid, st); break;
  }
}

template <int PROJ>
void launch_grouped(const GroupedParams& gp, dim3 grid, hipStream_t st) {
  switch (gp.g.meta_dtype) {
    case OSM_META_F32: launch_grouped_meta<OSM_META_F32, PROJ>(gp, grid, st); break;
    case OSM_META_F16: launch_grouped_meta<OSM_META_F16, PROJ>(gp, grid, st); break;
    default: launch_grouped_meta<OSM_META_BF16, PROJ>(gp, grid, st); break;
  }
}

unsigned blocks_for(size_t n, unsigned cap) {
  size_t b = (n + 255) / 256;
  if (b == 0) b = 1;
  return static_cast<unsigned>(b < cap ? b : cap);
}

}  // namespace

extern "C" {

size_t osmd_moe_grouped_max_tiles(uint32_t tokens, uint32_t nslot, uint32_t experts) {
  const size_t pairs = static_cast<size_t>(tokens) * nslot;
  const size_t buckets = experts + 1u;
  return (buckets < pairs ? buckets : pairs) + pairs / kTileTokens + 1u;
}

int osmd_moe_grouped(const osmd_moe_grouped_args* a, osmd_stream s) {
  const hipStream_t st = static_cast<hipStream_t>(s);
  const osmd_moe_args& m = a->moe;
  const osm_expert_geometry g = m.geom;
  const uint32_t T = m.tokens, D = g.hidden, I = g.inter, G = g.group;
  const uint32_t has_shared = (m.flags & OSMD_MOE_SHARED) ? 1u : 0u;
  const uint32_t nslot = m.top_k + has_shared;
  const uint32_t P = T * nslot;
  const size_t max_tiles = osmd_moe_grouped_max_tiles(T, nslot, m.expert_count);

  // Input (optionally normalised) -> router terms.
  const void* xin = m.x;
  bool xbf16 = a->x_bf16 != 0;
  if (m.flags & OSMD_MOE_RMSNORM) {
    int r = osmd_rms_norm(static_cast<const float*>(m.x), m.norm_weight, m.x_norm, T, D, m.rms_eps, s);
    if (r != 0) return r;
    xin = m.x_norm;
    xbf16 = false;
  }
  const size_t groups = static_cast<size_t>(T) * (D / G);
  int r = 0;
  // Up to 64 tokens the per-token router kernel (one wavefront per router
  // row and token) has the shorter latency; beyond, the MFMA router GEMM.
  if (m.router_dtype == OSM_META_BF16 && (xbf16 || T > kRouterGemmMinTokens)) {
    if (xbf16)
      prepare_kernel<true, kRouterSplit><<<blocks_for(groups, 4096), 256, 0, st>>>(xin, T, D, G, a->x_terms, a->x_sums);
    else
      prepare_kernel<false, kRouterSplit><<<blocks_for(groups, 4096), 256, 0, st>>>(xin, T, D, G, a->x_terms, a->x_sums);
    const uint32_t nrows = m.expert_count + has_shared;
    router_gemm_kernel<kRouterSplit><<<dim3((nrows + kGroupedWaves * kBlockRows - 1) / (kGroupedWaves * kBlockRows),
                                            (T + kTileTokens - 1) / kTileTokens),
                                       kGroupedThreads, 0, st>>>(
        a->x_terms, T, D, static_cast<const uint16_t*>(m.router),
        has_shared ? static_cast<const uint16_t*>(m.shared_gate_vec) : nullptr, m.expert_count, m.logits,
        m.shared_gate);
  } else {
    // The decode router kernel, one token per grid row (fp32 input).
    osmd_moe_args ra = m;
    ra.flags &= ~static_cast<uint32_t>(OSMD_MOE_RMSNORM);  // x is normalised above
    ra.x = static_cast<const float*>(xin);
    if (xbf16) return 1;  // the caller only passes bf16 input with a bf16 router
    r = osmd_moe_router(&ra, s);
    if (r != 0) return r;
  }
  r = osmd_moe_select(&m, s);
  if (r != 0) return r;
  bucket_kernel<<<1, kBucketThreads, 0, st>>>(m.ids, m.weights, has_shared ? m.shared_gate : nullptr, T, m.top_k,
                                              nslot, m.expert_count, a->perm, a->pair_pos, a->pair_w,
                                              static_cast<Tile*>(a->tiles), a->tile_count);

  // The gate/up GEMM reads the router terms' first kActSplit terms: re-pack
  // them with that stride (prepare writes the split the GEMM wants).
  if (xbf16)
    prepare_kernel<true, kActSplit><<<blocks_for(groups, 4096), 256, 0, st>>>(xin, T, D, G, a->x_terms, a->x_sums);
  else
    prepare_kernel<false, kActSplit><<<blocks_for(groups, 4096), 256, 0, st>>>(xin, T, D, G, a->x_terms, a->x_sums);

  GroupedParams gp{};
  gp.g = g;
  gp.terms = a->x_terms;
  gp.sums = a->x_sums;
  gp.perm = a->perm;
  gp.pair_w = a->pair_w;
  gp.tiles = static_cast<const Tile*>(a->tiles);
  gp.tile_count = a->tile_count;
  gp.expert_table = m.expert_table;
  gp.shared_expert = m.shared_expert;
  gp.fallback = m.fallback_blob;
  gp.expert_count = m.expert_count;
  gp.nslot = nslot;
  gp.out = a->h;
  const dim3 grid_gu(static_cast<unsigned>(max_tiles), (I + kRowsPerWorkgroup - 1) / kRowsPerWorkgroup);
  launch_grouped<2>(gp, grid_gu, st);
  const size_t hgroups = static_cast<size_t>(P) * (I / G);
  prepare_kernel<false, kActSplit><<<blocks_for(hgroups, 4096), 256, 0, st>>>(a->h, P, I, G, a->h_terms, a->h_sums);
  gp.terms = a->h_terms;
  gp.sums = a->h_sums;
  gp.out = a->partial;
  const dim3 grid_dn(static_cast<unsigned>(max_tiles), (D + kRowsPerWorkgroup - 1) / kRowsPerWorkgroup);
  launch_grouped<1>(gp, grid_dn, st);
  combine_kernel<<<blocks_for(static_cast<size_t>(T) * D, 4096), 256, 0, st>>>(
      a->partial, a->pair_pos, T, D, nslot, (m.flags & OSMD_MOE_RESIDUAL) ? static_cast<const float*>(m.x) : nullptr,
      m.y);
  return launch_status();
}

}  // extern "C"
