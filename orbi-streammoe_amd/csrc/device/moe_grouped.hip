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
//   gate/up      per tile and K range: partial x W_gate^T, x W_up^T
//   SwiGLU       h = SwiGLU(sum over ranges) -> bf16 split terms, group sums
//   down         per tile and K range: weight * (h W_down^T) -> partials
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
// cover each non-empty bucket; a tile carries its expert's blob address, and
// tile_rows[tile][j] holds the token of its pair j (entries j >= count are
// not written), so the GEMMs find weights and activation rows one load
// after their workgroup starts.
struct Tile {
  const uint8_t* blob;
  uint32_t start, count;
};
static_assert(sizeof(Tile) == 16, "tile record");

constexpr uint32_t kBucketThreads = 1024;
constexpr uint32_t kMaxBuckets = OSMD_MAX_EXPERTS + 1u;

__global__ __launch_bounds__(kBucketThreads) void bucket_kernel(
    const uint32_t* __restrict__ ids, const float* __restrict__ weights, const float* __restrict__ shared_gate,
    uint32_t T, uint32_t k, uint32_t nslot, uint32_t E, const uint8_t* const* __restrict__ expert_table,
    const uint8_t* shared_expert, const uint8_t* fallback, uint32_t* __restrict__ pair_pos,
    float* __restrict__ pair_w, Tile* __restrict__ tiles, uint32_t* __restrict__ tile_rows,
    uint32_t* __restrict__ tile_count, uint32_t max_tiles) {
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
    if (pass == 1) {
      if (tid == kBucketThreads - 1u) *tile_count = scan[tid];
      // Tiles past the last real one are empty (count 0): the GEMM grids
      // span the whole capacity and their workgroups read only their tile.
      for (uint32_t t = scan[kBucketThreads - 1u] + tid; t < max_tiles; t += kBucketThreads)
        tiles[t] = Tile{fallback, 0u, 0u};
    }
    __syncthreads();
  }
  for (uint32_t b = tid; b < nb; b += kBucketThreads) {
    const uint32_t n = counts[b];
    const uint8_t* blob = b < E ? expert_table[b] : shared_expert;
    if (blob == nullptr) blob = fallback;
    for (uint32_t s = 0; s * kTileTokens < n; ++s) {
      Tile tl;
      tl.blob = blob;
      tl.start = offsets[b] + s * kTileTokens;
      tl.count = n - s * kTileTokens < kTileTokens ? n - s * kTileTokens : kTileTokens;
      tiles[tbase[b] + s] = tl;
    }
  }
  for (uint32_t i = tid; i < P; i += kBucketThreads) {
    const uint32_t t = i / nslot, j = i % nslot;
    uint32_t e = j < k ? ids[static_cast<size_t>(t) * k + j] : E;
    e = e < nb ? e : nb - 1u;
    const uint32_t in_bucket = atomicAdd(&cursor[e], 1u);
    const uint32_t pos = offsets[e] + in_bucket;
    tile_rows[(tbase[e] + in_bucket / kTileTokens) * kTileTokens + in_bucket % kTileTokens] = t;
    pair_pos[i] = pos;
    pair_w[pos] = j < k ? weights[static_cast<size_t>(t) * k + j] : (shared_gate ? shared_gate[t] : 1.0f);
  }
}

// ---------------------------------------------------------------------------
// Grouped q4 GEMMs over the tile list, split along K.
//
// A workgroup of 4 waves takes one tile (<= 16 pairs), one block of weight
// rows and one K range of KS = 32 * NSTEP columns. Every wave first issues
// all of its packed-word and metadata loads for the range, then every thread
// issues its share of the tile's activation terms for the range (rows past
// the tile's count are not staged: MFMA rows read the last real row instead)
// before storing them to LDS, behind one barrier. A wave so costs one memory
// round trip and no per-chunk synchronisation, and a compute unit keeps
// about 100 KB of weights in flight (three workgroups).
//   gate/up: 64 rows per workgroup; waves 0-1 gate, waves 2-3 up, 32 rows
//            each; part[split][proj][pair][row] partial sums.
//   down:    128 rows per workgroup (32 per wave), times the pair weight;
//            out[split][pair][row].
// S = G / 32 MFMA steps per group; lane k-slot q uses words S*q .. S*q+S-1
// of each group (step s: word S*q + s), so one lane load covers a group.
struct SplitParams {
  osm_expert_geometry g;
  const uint16_t* terms;  // A terms [rows][kActSplit][K]
  const float* sums;      // [rows][K/G]
  const uint32_t* tile_rows;  // [tiles][16] token of each pair of a tile
  const float* pair_w;    // [P]
  const Tile* tiles;
  uint32_t P;
  uint32_t max_tiles;  // tile capacity of the workspace
  uint32_t row_blocks, nsplit;
  float* out;
};

// Workgroup -> (tile, K range, row block). Workgroups are dealt to the 8
// XCDs round-robin (workgroup b runs on XCD b % 8), so tile t is given to
// XCD t % 8 and all of its K ranges and row blocks run there, one after the
// other: the tile's activation rows are read into one L2 only, and the K
// ranges of the same weight rows are fetched together.
constexpr uint32_t kXcds = 8;
struct SplitWork {
  uint32_t tile, split, row_block;
};
__device__ __forceinline__ SplitWork split_work(const SplitParams& p) {
  const uint32_t b = blockIdx.x, per_tile = p.row_blocks * p.nsplit;
  const uint32_t i = b / kXcds;
  SplitWork w;
  w.tile = (i / per_tile) * kXcds + b % kXcds;
  w.split = i % per_tile % p.nsplit;
  w.row_block = i % per_tile / p.nsplit;
  return w;
}
uint32_t split_grid(uint32_t max_tiles, uint32_t row_blocks, uint32_t nsplit) {
  return (max_tiles + kXcds - 1) / kXcds * kXcds * row_blocks * nsplit;
}

// Metadata of N consecutive groups of one row, kept as loaded: 16-bit values
// two to a register (bf16 / f16), f32 one to a register. The run starts at a
// multiple of N (K is a multiple of the range), so vector loads are aligned.
template <int META, int N>
struct MetaRun {
  static constexpr int kBytes = N * (META == OSM_META_F32 ? 4 : 2);
  static constexpr int kRegs = (kBytes + 3) / 4;
  uint32_t r[kRegs];
  __device__ __forceinline__ void load(const uint8_t* base, size_t idx) {
    const uint8_t* ptr = base + idx * (META == OSM_META_F32 ? 4u : 2u);
    if constexpr (kBytes % 16 == 0) {
#pragma unroll
      for (int i = 0; i < kBytes / 16; ++i) {
        const uint4 v = ldg16(ptr + 16 * i);
        r[4 * i] = v.x; r[4 * i + 1] = v.y; r[4 * i + 2] = v.z; r[4 * i + 3] = v.w;
      }
    } else if constexpr (kBytes == 8) {
      const uint2 v = ldg8(ptr);
      r[0] = v.x;
      r[1] = v.y;
    } else if constexpr (kBytes == 4) {
      r[0] = ldg<uint32_t>(ptr);
    } else {
      r[0] = ldg<uint16_t>(ptr);
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

constexpr uint32_t kWaveRows = 2u * kBlockRows;  // 32 weight rows per wave
constexpr uint32_t kSplitWaves = 4;
constexpr uint32_t kSplitThreads = kSplitWaves * kWave;
// Weight rows per workgroup: gate/up 64 (waves 0-1 gate, 2-3 up, same
// rows), down 128. Four waves measured faster than eight (8 waves need more
// than 128 VGPRs, so one workgroup per compute unit).
template <int PROJ>
constexpr uint32_t split_rows() {
  return PROJ == 2 ? kSplitWaves / 2u * kWaveRows : kSplitWaves * kWaveRows;
}

template <int META, int PROJ, int S, int NSTEP>
__global__ __launch_bounds__(kSplitThreads) void split_kernel(SplitParams p) {
  constexpr uint32_t KS = 32u * NSTEP;
  constexpr int GPR = NSTEP / S;  // groups per range
  constexpr uint32_t RS = KS + 8u;  // LDS row stride (bf16), padded against bank conflicts
  constexpr uint32_t kWgRows = split_rows<PROJ>();
  constexpr uint32_t kUnitCols = KS / 8u;  // 16-byte units per staged row
  constexpr uint32_t kUnitsPerThread = kActSplit * kTileTokens * kUnitCols / kSplitThreads;
  static_assert(kActSplit * kTileTokens * kUnitCols % kSplitThreads == 0, "staging units");
  static_assert(GPR * kTileTokens <= kSplitThreads, "group sums: one per thread");
  __shared__ __align__(16) uint16_t a_lds[kActSplit][kTileTokens][RS];
  __shared__ __align__(16) float xs_lds[GPR][kTileTokens];

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid % kWave, wave = tid / kWave;
  const uint32_t m = lane % 16u, q = lane / 16u;
  // The tile and (gate/up) the token of tile row m are loaded together
  // (tile < the workspace's capacity, so both reads are in bounds; rows >=
  // count hold stale tokens, never used). Tiles past the last real one have
  // count 0.
  const SplitWork wk = split_work(p);
  if (wk.tile >= p.max_tiles) return;  // the grid rounds the tiles up to whole XCD rounds
  Tile tl = p.tiles[wk.tile];
  uint32_t lane_act = PROJ == 2 ? p.tile_rows[wk.tile * kTileTokens + m] : 0u;
  // The whole record and the arguments the load addresses need are fetched
  // before the exit test (left alone, the compiler loads them after it, one
  // more memory round trip on every workgroup's critical path).
  osm_expert_geometry geo = p.g;
  const uint16_t* terms = p.terms;
  asm volatile("" : "+s"(tl.blob), "+s"(tl.start), "+s"(tl.count), "+s"(geo.hidden), "+s"(geo.inter),
               "+s"(geo.group), "+s"(terms));
  if (tl.count == 0u) return;  // uniform over the workgroup
  const uint32_t split = wk.split;
  const uint32_t D = geo.hidden, I = geo.inter, G = geo.group;
  const uint32_t K = PROJ == 2 ? D : I;
  const uint32_t N = PROJ == 2 ? I : D;
  const uint32_t ngroups = K / G;
  const uint32_t g0 = split * GPR;
  const osm_expert_offsets off = osm_expert_layout(geo);
  const uint8_t* blob = tl.blob;

  constexpr uint32_t kProjWaves = PROJ == 2 ? kSplitWaves / 2u : kSplitWaves;
  const uint32_t pr = wave / kProjWaves;
  const uint32_t rows = tl.count;

  // Activation row of tile row m: its token (gate/up, loaded above before the
  // weights, so that waiting for it never waits for them: the counter of
  // vector loads retires in issue order) or the pair itself (down).
  if constexpr (PROJ == 1) lane_act = tl.start + m;
  const uint32_t row_base = wk.row_block * kWgRows + (wave % kProjWaves) * kWaveRows;
  const size_t q_off = PROJ == 2 ? (pr ? off.up_q : off.gate_q) : off.down_q;
  const size_t s_off = PROJ == 2 ? (pr ? off.up_s : off.gate_s) : off.down_s;
  const size_t b_off = PROJ == 2 ? (pr ? off.up_b : off.gate_b) : off.down_b;

  // 1. This wave's packed words and metadata for the whole range, issued now.
  uint32_t w[2][NSTEP];
  MetaRun<META, GPR> sb[2], bb[2];
#pragma unroll
  for (uint32_t nb = 0; nb < 2u; ++nb) {
    uint32_t r = row_base + nb * kBlockRows + m;
    r = r < N ? r : N - 1u;
    const uint8_t* qrow = blob + q_off + static_cast<size_t>(r) * (K / 2u);
#pragma unroll
    for (int gg = 0; gg < GPR; ++gg) word_run<S>(qrow + ((g0 + gg) * (G / 8u) + S * q) * 4u, &w[nb][gg * S]);
    const size_t mi = static_cast<size_t>(r) * ngroups + g0;
    sb[nb].load(blob + s_off, mi);
    bb[nb].load(blob + b_off, mi);
  }

  // 2. The tile's activation rows for this range into LDS: all loads first,
  // then the stores. Unit u: term u / (16 * KS/8), tile row (u / (KS/8)) % 16,
  // 16-byte column unit u % (KS/8).
  auto act_row = [&](uint32_t j) -> uint32_t { return __shfl(lane_act, static_cast<int>(j)); };
  uint4 stage[kUnitsPerThread];
#pragma unroll
  for (uint32_t i = 0; i < kUnitsPerThread; ++i) {
    const uint32_t u = tid + i * kSplitThreads;
    const uint32_t term = u / (kTileTokens * kUnitCols), row = (u / kUnitCols) % kTileTokens, cu = u % kUnitCols;
    const uint32_t arow = act_row(row);  // every lane active here: the shuffle reads real lanes
    if (row < rows)
      stage[i] = ldg16(terms + (static_cast<size_t>(arow) * kActSplit + term) * K + split * KS + cu * 8u);
  }
  float xsum = 0.0f;
  const uint32_t sg = tid / kTileTokens, srow = tid % kTileTokens;
  const uint32_t sarow = act_row(srow);
  if (sg < GPR && srow < rows) xsum = p.sums[static_cast<size_t>(sarow) * ngroups + g0 + sg];
#pragma unroll
  for (uint32_t i = 0; i < kUnitsPerThread; ++i) {
    const uint32_t u = tid + i * kSplitThreads;
    const uint32_t term = u / (kTileTokens * kUnitCols), row = (u / kUnitCols) % kTileTokens, cu = u % kUnitCols;
    if (row < rows) *reinterpret_cast<uint4*>(&a_lds[term][row][cu * 8u]) = stage[i];
  }
  if (sg < GPR && srow < rows) xs_lds[sg][srow] = xsum;
  __syncthreads();

  // 3. MFMAs. MFMA row m reads tile row min(m, count - 1); the D rows of
  // lane q are tile rows 4q .. 4q+3 (those past count are not stored).
  const uint32_t ar = m < rows ? m : rows - 1u;
  uint32_t xr[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) xr[j] = 4u * q + j < rows ? 4u * q + j : rows - 1u;
  f32x4 total[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int gg = 0; gg < GPR; ++gg) {
    bf16x8 a[S][kActSplit];
#pragma unroll
    for (int s2 = 0; s2 < S; ++s2)
#pragma unroll
      for (uint32_t t = 0; t < kActSplit; ++t)
        a[s2][t] = as_operand(*reinterpret_cast<const uint4*>(&a_lds[t][ar][(gg * (G / 8u) + S * q + s2) * 8u]));
    float xs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xs[j] = xs_lds[gg][xr[j]];
#pragma unroll
    for (uint32_t nb = 0; nb < 2u; ++nb) {
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 < S; ++s2) {
        const bf16x8 b = nibble_operand(w[nb][gg * S + s2]);
#pragma unroll
        for (uint32_t t = 0; t < kActSplit; ++t) d = mfma(a[s2][t], b, d);
      }
      const float sc = sb[nb].get(gg);
      const float cb = bb[nb].get(gg) - 128.0f * sc;
#pragma unroll
      for (int j = 0; j < 4; ++j) total[nb][j] += sc * d[j] + cb * xs[j];
    }
  }

  // 4. Partial sums of this range.
#pragma unroll
  for (uint32_t nb = 0; nb < 2u; ++nb) {
    const uint32_t r = row_base + nb * kBlockRows + m;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t pj = 4u * q + j;
      if (pj < rows && r < N) {
        const size_t pair = tl.start + pj;
        if constexpr (PROJ == 2)
          p.out[((static_cast<size_t>(split) * 2u + pr) * p.P + pair) * N + r] = total[nb][j];
        else
          p.out[(static_cast<size_t>(split) * p.P + pair) * N + r] = p.pair_w[pair] * total[nb][j];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// h = SwiGLU of the gate and up sums over the K splits (split order), written
// directly as bf16 terms in word order with per-group sums for the down GEMM.
// One thread per (pair, 8-column word); the G/8 threads of a group are
// adjacent lanes of one wavefront and add their sums by butterfly.
__global__ void swiglu_terms_kernel(const float* __restrict__ part, uint32_t nsplit, uint32_t P, uint32_t I,
                                    uint32_t G, uint16_t* __restrict__ terms, float* __restrict__ sums) {
  const uint32_t words = I / 8u, wpg = G / 8u;
  const size_t n = static_cast<size_t>(P) * words;  // a multiple of wpg, so groups never straddle waves
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  const size_t plane = static_cast<size_t>(P) * I;
  for (size_t i0 = static_cast<size_t>(blockIdx.x) * blockDim.x; i0 < n; i0 += stride) {
    const size_t i = i0 + threadIdx.x;
    float total = 0.0f;
    if (i < n) {
      const size_t pair = i / words, wd = i % words;
      const float* gp = part + pair * I + wd * 8u;
      float gs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, us[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (uint32_t sp = 0; sp < nsplit; ++sp) {
        const float4* g4 = reinterpret_cast<const float4*>(gp + 2u * sp * plane);
        const float4* u4 = reinterpret_cast<const float4*>(gp + (2u * sp + 1u) * plane);
        const float4 ga = g4[0], gb = g4[1], ua = u4[0], ub = u4[1];
        gs[0] += ga.x; gs[1] += ga.y; gs[2] += ga.z; gs[3] += ga.w;
        gs[4] += gb.x; gs[5] += gb.y; gs[6] += gb.z; gs[7] += gb.w;
        us[0] += ua.x; us[1] += ua.y; us[2] += ua.z; us[3] += ua.w;
        us[4] += ub.x; us[5] += ub.y; us[6] += ub.z; us[7] += ub.w;
      }
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = silu_mul(gs[k], us[k]);
      float rep[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (uint32_t t = 0; t < kActSplit; ++t) {
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
        *reinterpret_cast<uint4*>(terms + (pair * kActSplit + t) * I + wd * 8u) = pk;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) total += rep[k];
    }
    for (uint32_t m = 1; m < wpg; m <<= 1) total += __shfl_xor(total, static_cast<int>(m));
    if (i < n && i % wpg == 0) sums[i / wpg] = total;
  }
}

// ---------------------------------------------------------------------------
// combine: y[t, r] = sum over slots 0..nslot-1 (routed picks in pick order,
// the shared expert last) of the down partials summed over K splits, plus x
// when the residual form is asked for.
__global__ void combine_kernel(const float* __restrict__ partial, uint32_t nsplit, uint32_t P,
                               const uint32_t* __restrict__ pair_pos, uint32_t T, uint32_t D, uint32_t nslot,
                               const float* __restrict__ residual, float* __restrict__ y) {
  const size_t n = static_cast<size_t>(T) * D;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint32_t t = static_cast<uint32_t>(i / D), r = static_cast<uint32_t>(i % D);
    float acc = 0.0f;
    for (uint32_t j = 0; j < nslot; ++j) {
      const size_t pos = pair_pos[t * nslot + j];
      for (uint32_t s = 0; s < nsplit; ++s) acc += partial[(static_cast<size_t>(s) * P + pos) * D + r];
    }
    y[i] = residual ? residual[i] + acc : acc;
  }
}

// Columns per K range: the largest of 512 / 256 / 128 that divides K.
uint32_t range_cols(uint32_t K) { return K % 512u == 0 ? 512u : (K % 256u == 0 ? 256u : 128u); }

template <int META, int PROJ, int S>
void launch_split_s(const SplitParams& sp, dim3 grid, hipStream_t st) {
  switch (range_cols(PROJ == 2 ? sp.g.hidden : sp.g.inter)) {
    case 512: split_kernel<META, PROJ, S, 16><<<grid, kSplitThreads, 0, st>>>(sp); break;
    case 256: split_kernel<META, PROJ, S, 8><<<grid, kSplitThreads, 0, st>>>(sp); break;
    default: split_kernel<META, PROJ, S, 4><<<grid, kSplitThreads, 0, st>>>(sp); break;
  }
}

template <int META, int PROJ>
void launch_split_meta(const SplitParams& sp, dim3 grid, hipStream_t st) {
  switch (sp.g.group) {
    case 32: launch_split_s<META, PROJ, 1>(sp, grid, st); break;
    case 64: launch_split_s<META, PROJ, 2>(sp, grid, st); break;
    default: launch_split_s<META, PROJ, 4>(sp, grid, st); break;
  }
}

template <int PROJ>
void launch_split(const SplitParams& sp, dim3 grid, hipStream_t st) {
  switch (sp.g.meta_dtype) {
    case OSM_META_F32: launch_split_meta<OSM_META_F32, PROJ>(sp, grid, st); break;
    case OSM_META_F16: launch_split_meta<OSM_META_F16, PROJ>(sp, grid, st); break;
    default: launch_split_meta<OSM_META_BF16, PROJ>(sp, grid, st); break;
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

uint32_t osmd_moe_grouped_splits(uint32_t cols) { return cols / range_cols(cols); }

int osmd_moe_grouped(const osmd_moe_grouped_args* a, osmd_stream s) {
  const hipStream_t st = static_cast<hipStream_t>(s);
  const osmd_moe_args& m = a->moe;
  const osm_expert_geometry g = m.geom;
  const uint32_t T = m.tokens, D = g.hidden, I = g.inter, G = g.group;
  const uint32_t has_shared = (m.flags & OSMD_MOE_SHARED) ? 1u : 0u;
  const uint32_t nslot = m.top_k + has_shared;
  const uint32_t P = T * nslot;
  const size_t max_tiles = osmd_moe_grouped_max_tiles(T, nslot, m.expert_count);
  uint32_t* tile_rows = reinterpret_cast<uint32_t*>(static_cast<Tile*>(a->tiles) + max_tiles);

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
                                              nslot, m.expert_count, m.expert_table, m.shared_expert,
                                              m.fallback_blob, a->pair_pos, a->pair_w, static_cast<Tile*>(a->tiles),
                                              tile_rows, a->tile_count, static_cast<uint32_t>(max_tiles));

  // The expert GEMMs take 2 terms per activation; the router's 3-term data
  // is re-packed (its group sums must be of the terms the GEMMs multiply).
  if (xbf16)
    prepare_kernel<true, kActSplit><<<blocks_for(groups, 4096), 256, 0, st>>>(xin, T, D, G, a->x_terms, a->x_sums);
  else
    prepare_kernel<false, kActSplit><<<blocks_for(groups, 4096), 256, 0, st>>>(xin, T, D, G, a->x_terms, a->x_sums);

  SplitParams sp{};
  sp.g = g;
  sp.terms = a->x_terms;
  sp.sums = a->x_sums;
  sp.tile_rows = tile_rows;
  sp.pair_w = a->pair_w;
  sp.tiles = static_cast<const Tile*>(a->tiles);
  sp.P = P;
  sp.max_tiles = static_cast<uint32_t>(max_tiles);
  sp.out = a->gu_part;
  const uint32_t gu_splits = osmd_moe_grouped_splits(D);
  sp.row_blocks = (I + split_rows<2>() - 1) / split_rows<2>();
  sp.nsplit = gu_splits;
  launch_split<2>(sp, dim3(split_grid(sp.max_tiles, sp.row_blocks, sp.nsplit)), st);
  const size_t hwords = static_cast<size_t>(P) * (I / 8u);
  swiglu_terms_kernel<<<blocks_for(hwords, 4096), 256, 0, st>>>(a->gu_part, gu_splits, P, I, G, a->h_terms,
                                                                a->h_sums);
  sp.terms = a->h_terms;
  sp.sums = a->h_sums;
  sp.out = a->partial;
  const uint32_t dn_splits = osmd_moe_grouped_splits(I);
  sp.row_blocks = (D + split_rows<1>() - 1) / split_rows<1>();
  sp.nsplit = dn_splits;
  launch_split<1>(sp, dim3(split_grid(sp.max_tiles, sp.row_blocks, sp.nsplit)), st);
  combine_kernel<<<blocks_for(static_cast<size_t>(T) * D, 4096), 256, 0, st>>>(
      a->partial, dn_splits, P, a->pair_pos, T, D, nslot,
      (m.flags & OSMD_MOE_RESIDUAL) ? static_cast<const float*>(m.x) : nullptr, m.y);
  return launch_status();
}

}  // extern "C"
