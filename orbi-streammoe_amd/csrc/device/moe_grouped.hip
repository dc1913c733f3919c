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
#include <type_traits>

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
constexpr uint32_t kRouterGemmMinTokens = 16;
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

// The eight nibbles q of a packed word as the bf16 integers 128 + q, in MFMA
// operand order: register j holds nibble j (low half) and nibble j + 4 (high
// half), i.e. ((w >> 4j) & 0x000F000F) | 0x43004300. Two masks split the word
// into one byte per nibble (lo: nibbles 0, 2, 4, 6; hi: 1, 3, 5, 7), and each
// register is one byte permutation of lo or hi with 0x43, the high byte of
// 128.0 in bf16: seven instructions per word instead of eleven.
// v_perm_b32(s0, s1, sel): result byte i = byte sel.byte[i] of {s0, s1}
// (selectors 0-3 pick bytes of s1, 4-7 bytes of s0).
__device__ __forceinline__ bf16x8 nibble_operand(uint32_t w) {
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu, k = 0x43434343u;
  const uint32_t even = 0x04020400u;  // bytes 0 and 2 of s1: nibbles 0, 4 (lo) or 1, 5 (hi)
  const uint32_t odd = 0x04030401u;   // bytes 1 and 3 of s1: nibbles 2, 6 (lo) or 3, 7 (hi)
  const u32x4 v = {__builtin_amdgcn_perm(k, lo, even), __builtin_amdgcn_perm(k, hi, even),
                   __builtin_amdgcn_perm(k, lo, odd), __builtin_amdgcn_perm(k, hi, odd)};
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// bf16 rows widened to fp32 (exact), for the per-token router kernel when the
// router is not bf16 and so cannot run as the MFMA GEMM.
__global__ void widen_bf16_kernel(const uint16_t* __restrict__ x, size_t n, float* __restrict__ out) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    out[i] = bf16_to_f32(x[i]);
}

// ---------------------------------------------------------------------------
// prepare: rows [R, K] (fp32, or bf16 when XBF16) -> terms [R][NS][K] bf16 in
// word order and sums [R][K/G] of the values the first two terms represent
// (the expert GEMMs read terms 0 and 1 of this layout; the router GEMM reads
// all three when NS = 3). A bf16 input needs one term (NS = 1): it is exact.
// One thread per (row, 8-column word); the G/8 threads of a group are
// adjacent lanes of one wavefront and add their sums by butterfly.
template <bool XBF16, int NS>
__global__ void prepare_kernel(const void* __restrict__ x, uint32_t R, uint32_t K, uint32_t G,
                               uint16_t* __restrict__ terms, float* __restrict__ sums,
                               float* __restrict__ norms) {
  // A bf16 input is its own first term: one term is exact, and the expert
  // GEMMs then read just that one.
  static_assert(NS >= kActSplit || XBF16, "the expert GEMMs read the first two terms of an fp32 input");
  constexpr int kSumTerms = NS < kActSplit ? NS : kActSplit;
  const uint32_t words = K / 8u, wpg = G / 8u;
  const size_t n = static_cast<size_t>(R) * words;  // a multiple of wpg, so groups never straddle waves
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i0 = static_cast<size_t>(blockIdx.x) * blockDim.x; i0 < n; i0 += stride) {
    const size_t i = i0 + threadIdx.x;
    float total = 0.0f, sq = 0.0f;
    if (i < n) {
      const uint32_t r = static_cast<uint32_t>(i / words), wd = static_cast<uint32_t>(i % words);
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
#pragma unroll
      for (int k = 0; k < 8; ++k) sq += v[k] * v[k];
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
        if (s + 1 == kSumTerms) {
#pragma unroll
          for (int k = 0; k < 8; ++k) total += rep[k];
        }
      }
    }
    // Sum of the group's G/8 words, then written by its first lane.
    for (uint32_t m = 1; m < wpg; m <<= 1) total += __shfl_xor(total, static_cast<int>(m), kWave);
    if (i < n && (i % wpg) == 0u) sums[i / wpg] = total;
    if (norms != nullptr) {
      // Euclidean norm of each 32-column chunk (4 words), rounded up: the
      // router GEMM's error bounds take |w . x| <= |w| |x| per chunk. The
      // fp32 sum of 32 squares is within 32 u of the true one, so 1 + 2^-20
      // covers it and the square root's rounding.
      sq += __shfl_xor(sq, 1, kWave);
      sq += __shfl_xor(sq, 2, kWave);
      if (i < n && (i % 4u) == 0u) norms[i / 4u] = sqrtf(sq) * (1.0f + 0x1p-20f);
    }
  }
}

// ---------------------------------------------------------------------------
// Router GEMM: partial logits [T, E] and, as column E, the shared-gate dot
// w_sg . x, one plane per K range (the selection adds the planes in order
// and applies the sigmoid). A workgroup is 16 tokens x 64 router rows (4
// waves x 16, bf16) x one K range of R = 32 * NSTEP columns, for TT
// consecutive token tiles. The tile's activation terms are staged in LDS once
// and read by all four waves; each wave's router values for the range are
// loaded before the staging, so both streams are in flight together.
// Splitting K keeps a workgroup's reads small (48 KB of terms, 64 KB of
// router rows at R = 512) and the grid large; a wave that read its own copy
// of the terms, over all of K, moved 4x more bytes through L2 than the tile
// holds.
//
// The launch is one-dimensional and a multiple of 8 long. Workgroup L runs on
// XCD L % 8 (workgroups are dispatched to the XCDs round-robin) and takes
// item (L % 8) * (launch / 8) + L / 8 of the (router block, token group, K
// range) items in K-range-major order, so an XCD's workgroups share a run of
// one K range's router rows and token tiles in that XCD's L2 instead of every
// XCD reading all of the router and all of the terms.
//
// Every logit plane also gets its part of the bound on the distance from
// the reference's sequentially summed logit (bplanes, when BOUNDS;
// reference_ops.cpp:85-93). Per 32-column step the MFMAs start from zero
// (smallest term first) and the step sums are added in fp32, so with u =
// 2^-24 and a the step's sum |w| |x| (at most |w_chunk| |x_chunk|, the
// norms of the router rows and inputs, rnorm and xnorm):
//  - the MFMAs form each bf16 product exactly and add 33 operands per
//    instruction; in any order, with each addition faithful (or with all
//    operands aligned to the largest and truncated), that errs by at most
//    66 u of the operands' absolute sum, about 70 u a per step;
//  - adding the step sums errs by at most u |running sum| per step;
//  - the reference's 32 partial sums within the step are at most
//    32 (|running sum before it| + a).
// Bound plane p gets sum over steps of 32 (|before| + a) + |after| +
// router_gemm_bound_coef(D) a, evaluated as 33 (|s_1| + ... + |s_{n-1}|) +
// |s_n| + (32 + coef) (sum of a), s_i the running sum after step i (s_0 =
// 0). The selection adds R |start of the range| for each range after the
// first and scales the total.
// The steps' MFMAs are independent (each starts from zero), so a batch of
// them is issued before their sums join the running sums in step order.
template <int NS, int NSTEP, int TT, bool BOUNDS>
__global__ __launch_bounds__(kGroupedThreads) void router_gemm_kernel(
    const uint16_t* __restrict__ terms, uint32_t T, uint32_t D, const uint16_t* __restrict__ router,
    const uint16_t* __restrict__ shared_gate_vec, uint32_t E, float* __restrict__ planes,
    const float* __restrict__ rnorm, const float* __restrict__ xnorm, float* __restrict__ bplanes, uint32_t gx,
    uint32_t gy, uint32_t gz) {
  constexpr uint32_t R = 32u * NSTEP;
  constexpr uint32_t RS = R + 8u;  // LDS row stride (bf16), padded against bank conflicts
  constexpr uint32_t kUnitCols = R / 8u;
  constexpr uint32_t kUnitsPerThread = NS * kTileTokens * kUnitCols / kGroupedThreads;
  constexpr int kBatch = 4;  // steps whose MFMAs are issued together
  static_assert(NS * kTileTokens * kUnitCols % kGroupedThreads == 0, "staging units");
  static_assert(NSTEP % 4 == 0, "input norms read four steps at a time");
  __shared__ __align__(16) uint16_t a_lds[NS][kTileTokens][RS];
  __shared__ __align__(16) float xn_lds[kTileTokens][NSTEP];
  const uint32_t n8 = gridDim.x / 8u;
  const uint32_t item = (blockIdx.x % 8u) * n8 + blockIdx.x / 8u;
  if (item >= gx * gy * gz) return;  // the launch's padding (workgroup-uniform, before any barrier)
  const uint32_t bx = item % gx, by = (item / gx) % gy, bz = item / (gx * gy);
  const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const uint32_t k0 = bz * R;
  const uint32_t nrows = E + (shared_gate_vec ? 1u : 0u);
  const uint32_t m = lane % 16u, q = lane / 16u;
  const uint32_t row = (bx * kGroupedWaves + wave) * kBlockRows + m;
  const uint32_t rr = row < nrows ? row : nrows - 1u;
  const uint16_t* wrow = (rr < E ? router + static_cast<size_t>(rr) * D : shared_gate_vec) + k0;

  // 1. B: this wave's router values for the range, kept for all TT token
  // tiles of the workgroup; then the first tile's terms (unit u: term u /
  // (16 * R/8), token row (u / (R/8)) % 16, 16-byte column unit u % (R/8);
  // rows past T load the last token).
  uint4 raw[NSTEP];
#pragma unroll
  for (int st = 0; st < NSTEP; ++st) raw[st] = ldg16(wrow + 32u * st + 8u * q);
  float wn[NSTEP];
  if constexpr (BOUNDS) {
    const float* rn = rnorm + static_cast<size_t>(rr) * (D / 32u) + k0 / 32u;
#pragma unroll
    for (int st = 0; st < NSTEP; ++st) wn[st] = rn[st];
  }
  uint4 stage[kUnitsPerThread];
  float xn = 0.0f;
  auto fetch = [&](uint32_t t0) {
#pragma unroll
    for (uint32_t i = 0; i < kUnitsPerThread; ++i) {
      const uint32_t u = tid + i * kGroupedThreads;
      const uint32_t term = u / (kTileTokens * kUnitCols), r = (u / kUnitCols) % kTileTokens, cu = u % kUnitCols;
      const uint32_t tok = t0 + r < T ? t0 + r : T - 1u;
      stage[i] = ldg16(terms + (static_cast<size_t>(tok) * NS + term) * D + k0 + cu * 8u);
    }
    if (BOUNDS && tid < kTileTokens * NSTEP) {
      const uint32_t r = tid / NSTEP, st = tid % NSTEP;
      const uint32_t tok = t0 + r < T ? t0 + r : T - 1u;
      xn = xnorm[static_cast<size_t>(tok) * (D / 32u) + k0 / 32u + st];
    }
  };
  const uint32_t tile0 = by * TT;
  fetch(tile0 * kTileTokens);

  // B operands: 8 router values of row rr in word order per step.
  bf16x8 bop[NSTEP];
#pragma unroll
  for (int st = 0; st < NSTEP; ++st) {
    const uint32_t h4[4] = {raw[st].x, raw[st].y, raw[st].z, raw[st].w};
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
    bop[st] = as_operand(bv);
  }

#pragma unroll 1
  for (uint32_t tt = 0; tt < TT; ++tt) {
    const uint32_t t0 = (tile0 + tt) * kTileTokens;
    if (t0 >= T) break;  // workgroup-uniform
    if (tt > 0u) __syncthreads();  // the previous tile's LDS operands are read
#pragma unroll
    for (uint32_t i = 0; i < kUnitsPerThread; ++i) {
      const uint32_t u = tid + i * kGroupedThreads;
      const uint32_t term = u / (kTileTokens * kUnitCols), r = (u / kUnitCols) % kTileTokens, cu = u % kUnitCols;
      *reinterpret_cast<uint4*>(&a_lds[term][r][cu * 8u]) = stage[i];
    }
    if (BOUNDS && tid < kTileTokens * NSTEP) xn_lds[tid / NSTEP][tid % NSTEP] = xn;
    __syncthreads();
    // The next tile's terms are in flight while this one computes.
    if (tt + 1u < TT && t0 + kTileTokens < T) fetch(t0 + kTileTokens);

    // 2. MFMAs: A = token m's terms at k0 + 32 st + 8q (word order), B = 8
    // router values of row rr. Each step starts from zero, smallest term
    // first; its sum joins the running sums in fp32, in step order.
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float sabs[4] = {0.f, 0.f, 0.f, 0.f};
    const float ca = 32.0f + router_gemm_bound_coef(D);
#pragma unroll
    for (int b0 = 0; b0 < NSTEP; b0 += kBatch) {
      f32x4 part[kBatch];
#pragma unroll
      for (int s = 0; s < kBatch; ++s) {
        part[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = NS - 1; t >= 0; --t)
          part[s] = mfma(as_operand(*reinterpret_cast<const uint4*>(&a_lds[t][m][32u * (b0 + s) + 8u * q])),
                         bop[b0 + s], part[s]);
      }
#pragma unroll
      for (int s = 0; s < kBatch; ++s) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[j] = acc[j] + part[s][j];
          if (BOUNDS && b0 + s + 1 < NSTEP) sabs[j] += fabsf(acc[j]);
        }
      }
    }

    // 3. Plane bz, [T][E + 1] (column E: the shared gate, when there is
    // one): D rows 4q + j are tokens, column m the router row.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t t = t0 + 4u * q + j;
      float ap = 0.0f;
      if constexpr (BOUNDS) {
        const float4* xr = reinterpret_cast<const float4*>(&xn_lds[4u * q + j][0]);
#pragma unroll
        for (int c = 0; c < NSTEP / 4; ++c) {
          const float4 xv = xr[c];
          ap = fmaf(wn[4 * c + 0], xv.x, ap);
          ap = fmaf(wn[4 * c + 1], xv.y, ap);
          ap = fmaf(wn[4 * c + 2], xv.z, ap);
          ap = fmaf(wn[4 * c + 3], xv.w, ap);
        }
      }
      if (t < T && row < nrows) {
        const size_t o = (static_cast<size_t>(bz) * T + t) * (E + 1u) + row;
        planes[o] = acc[j];
        if constexpr (BOUNDS) bplanes[o] = 33.0f * sabs[j] + fabsf(acc[j]) + ca * ap;
      }
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
// The scattered outputs (tile rows, pair weights) are assembled in LDS and
// written out in order when they fit: 12,288 tile-row entries (768 tiles) and
// 8,192 pairs, a 512-token chunk of top-10 + shared with room to spare.
constexpr uint32_t kBucketStageRows = 12288;
constexpr uint32_t kBucketStagePairs = 8192;

// ceil(2^32 / nslot) for nslot > 1: with m = (2^32 + r) / nslot, r < nslot,
// i m / 2^32 exceeds i / nslot by i r / (nslot 2^32) < 1 / nslot for i <
// 2^24, so the high product's floor is i / nslot exactly (a 32-bit division
// is dozens of instructions, per pair, on the bucket pass's one compute unit).
uint32_t slot_magic(uint32_t nslot) {
  return nslot > 1u ? static_cast<uint32_t>((0x100000000ull + nslot - 1u) / nslot) : 0u;
}

// Pairs a thread holds in registers from the first load to the scatter
// (REG): 8 cover P <= 8,192 (a 512-token chunk of top-10 + shared is 5,632),
// 1 covers P <= 1,024 (a 64-token decode step is 704) with a fraction of the
// code; pairs beyond are read again from memory in each pass.
constexpr uint32_t kNoBucket = 0xFFFFFFFFu;

template <int REG>
__global__ __launch_bounds__(kBucketThreads) void bucket_kernel(
    const uint32_t* __restrict__ ids, const float* __restrict__ weights, const float* __restrict__ shared_gate,
    uint32_t T, uint32_t k, uint32_t nslot, uint32_t E, const uint8_t* const* __restrict__ expert_table,
    const uint8_t* shared_expert, const uint8_t* fallback, uint32_t* __restrict__ pair_pos,
    float* __restrict__ pair_w, Tile* __restrict__ tiles, uint32_t* __restrict__ tile_rows,
    uint32_t* __restrict__ tile_count, uint32_t max_tiles, uint32_t magic) {
  __shared__ uint32_t counts[kMaxBuckets], offsets[kMaxBuckets], cursor[kMaxBuckets], tbase[kMaxBuckets];
  __shared__ uint32_t wave_total[kBucketThreads / kWave];
  __shared__ uint32_t s_rows[kBucketStageRows];
  __shared__ float s_w[kBucketStagePairs];
  __shared__ uint32_t s_tiles;
  const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const uint32_t nb = E + (nslot > k ? 1u : 0u);
  const uint32_t P = T * nslot;
  // Token of pair i as a high product (slot_magic; one slot: the pair index).
  auto token_of = [&](uint32_t i) { return nslot > 1u ? __umulhi(i, magic) : i; };
  // Bucket and weight of pair i: slot < k is routed (ids clamped to E - 1,
  // as an out-of-range id is never produced), slot k the shared expert E.
  auto pair_of = [&](uint32_t i, uint32_t& e, float& w) {
    const uint32_t t = token_of(i), j = i - t * nslot;
    if (j < k) {
      const size_t o = static_cast<size_t>(t) * k + j;
      e = ids[o];
      e = e < E ? e : E - 1u;
      w = weights[o];
    } else {
      e = E;
      w = shared_gate ? shared_gate[t] : 1.0f;
    }
  };

  // Every global read of the pass is requested here, before any wait: the
  // experts and weights of this thread's first pairs and the blobs of
  // buckets tid and tid + 1024 (nb <= 1025).
  uint32_t pe[REG];
  float pw[REG];
#pragma unroll
  for (int r = 0; r < REG; ++r) {
    const uint32_t i = tid + r * kBucketThreads;
    pe[r] = kNoBucket;
    pw[r] = 0.0f;
    if (i < P) pair_of(i, pe[r], pw[r]);
  }
  auto blob_of = [&](uint32_t b) -> const uint8_t* {
    const uint8_t* blob = b < E ? expert_table[b] : shared_expert;
    return blob ? blob : fallback;
  };
  const uint8_t* blob0 = tid < nb ? blob_of(tid) : fallback;
  const uint8_t* blob1 = tid + kBucketThreads < nb ? blob_of(tid + kBucketThreads) : fallback;
  constexpr uint32_t kRegSpan = REG * kBucketThreads;

  for (uint32_t b = tid; b < nb; b += kBucketThreads) counts[b] = 0u, cursor[b] = 0u;
  __syncthreads();
  // Routed pairs only: the shared expert's bucket (E) holds one pair per
  // token, in token order, so it needs no counting or cursor.
#pragma unroll
  for (int r = 0; r < REG; ++r)
    if (pe[r] < E) atomicAdd(&counts[pe[r]], 1u);
  for (uint32_t i = kRegSpan + tid; i < P; i += kBucketThreads) {
    uint32_t e;
    float w;
    pair_of(i, e, w);
    if (e < E) atomicAdd(&counts[e], 1u);
  }
  if (nb > E && tid == 0) counts[E] = T;
  __syncthreads();
  // Exclusive scans of the counts and of the tile counts, two buckets per
  // thread at most (nb <= 1025): a wavefront scan, then each thread adds the
  // totals of the wavefronts before its own.
  for (int pass = 0; pass < 2; ++pass) {
    uint32_t local = 0;
    for (uint32_t b = tid * 2u; b < tid * 2u + 2u && b < nb; ++b)
      local += pass == 0 ? counts[b] : (counts[b] + kTileTokens - 1u) / kTileTokens;
    uint32_t incl = local;
    for (uint32_t off = 1; off < kWave; off <<= 1) {
      const uint32_t v = __shfl_up(incl, off, kWave);
      incl += lane >= off ? v : 0u;
    }
    if (lane == kWave - 1u) wave_total[wave] = incl;
    __syncthreads();
    uint32_t before = 0, all = 0;
    for (uint32_t w = 0; w < kBucketThreads / kWave; ++w) {
      before += w < wave ? wave_total[w] : 0u;
      all += wave_total[w];
    }
    uint32_t run = before + incl - local;
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
      if (tid == 0) {
        *tile_count = all;
        s_tiles = all;
      }
      // Tiles past the last real one are empty (count 0): the GEMM grids
      // span the whole capacity and their workgroups read only their tile.
      for (uint32_t t = all + tid; t < max_tiles; t += kBucketThreads) tiles[t] = Tile{fallback, 0u, 0u};
    }
    __syncthreads();
  }
  for (uint32_t h = 0; h < 2u; ++h) {
    const uint32_t b = tid + h * kBucketThreads;
    if (b >= nb) break;
    const uint32_t n = counts[b];
    for (uint32_t s = 0; s * kTileTokens < n; ++s) {
      Tile tl;
      tl.blob = h == 0u ? blob0 : blob1;
      tl.start = offsets[b] + s * kTileTokens;
      tl.count = n - s * kTileTokens < kTileTokens ? n - s * kTileTokens : kTileTokens;
      tiles[tbase[b] + s] = tl;
    }
  }
  const uint32_t ntiles = s_tiles;  // written before the last scan's barrier
  const bool stage = ntiles * kTileTokens <= kBucketStageRows && P <= kBucketStagePairs;
  auto scatter = [&](uint32_t i, uint32_t e, float w) {
    const uint32_t t = token_of(i);
    const uint32_t in_bucket = e == E ? t : atomicAdd(&cursor[e], 1u);
    const uint32_t pos = offsets[e] + in_bucket;
    const uint32_t slot = (tbase[e] + in_bucket / kTileTokens) * kTileTokens + in_bucket % kTileTokens;
    pair_pos[i] = pos;
    if (stage) {
      s_rows[slot] = t;
      s_w[pos] = w;
    } else {
      tile_rows[slot] = t;
      pair_w[pos] = w;
    }
  };
#pragma unroll
  for (int r = 0; r < REG; ++r)
    if (pe[r] != kNoBucket) scatter(tid + r * kBucketThreads, pe[r], pw[r]);
  for (uint32_t i = kRegSpan + tid; i < P; i += kBucketThreads) {
    uint32_t e;
    float w;
    pair_of(i, e, w);
    scatter(i, e, w);
  }
  if (stage) {
    // In order: entries of a tile past its count hold whatever LDS held
    // (no GEMM reads them).
    __syncthreads();
    for (uint32_t i = tid; i < ntiles * kTileTokens; i += kBucketThreads) tile_rows[i] = s_rows[i];
    for (uint32_t i = tid; i < P; i += kBucketThreads) pair_w[i] = s_w[i];
  }
}

// ---------------------------------------------------------------------------
// Grouped q4 GEMMs over the tile list, split along K.
//
// A work item is one tile (<= 16 pairs), H consecutive K ranges of KS = 32 *
// NSTEP columns and a run of item_blocks consecutive row blocks; a workgroup
// of 4 waves works through items b, b + grid, ... (persistent, one grid of as
// many workgroups as are resident). Per item it stages the tile's activation
// terms for its ranges into LDS once (rows past the tile's count are not
// staged: MFMA rows read the last real row instead), then streams the
// (block, range) sub-blocks' weights with one in flight ahead of the one
// being computed: the packed words and metadata of sub-block i+1 (the next
// item's first, after the last) are issued before sub-block i's MFMAs. A
// block's totals carry over its H ranges. A block is 32 weight rows per wave:
//   gate/up: 64 rows per workgroup; waves 0-1 gate, waves 2-3 up, 32 rows
//            each; part[split][proj][pair][row] partial sums.
//   down:    128 rows per workgroup (32 per wave), times the pair weight;
//            out[split][pair][row].
// S = G / 32 MFMA steps per group; lane k-slot q uses words S*q .. S*q+S-1
// of each group (step s: word S*q + s), so one lane load covers a group.
struct SplitParams {
  osm_expert_geometry g;
  const uint16_t* terms;  // A terms [rows][term_count][K]; the GEMM reads the first NT
  uint32_t term_count;
  const float* sums;      // [rows][K/G]
  const uint32_t* tile_rows;  // [tiles][16] token of each pair of a tile
  const float* pair_w;    // [P]
  const Tile* tiles;
  uint32_t P;
  uint32_t max_tiles;   // tile capacity of the workspace
  uint32_t nsplit;      // partials per row: K ranges / H
  uint32_t item_blocks; // row blocks per item (item_blocks(H))
  uint32_t chunks;      // items per tile and K range
  uint32_t items;       // tiles (rounded to whole XCD rounds) x K ranges x chunks
  float* out;
  // Gate/up with SwiGLU fused (one partial per row, group 64): h as bf16
  // terms and per-group sums, the layout swiglu_terms_kernel writes.
  uint16_t* h_terms;
  float* h_sums;
};

// Work item -> (tile, K range, first row block). Workgroups are dealt to the
// 8 XCDs round-robin (workgroup b runs on XCD b % 8) and take items b, b +
// grid, ... with the grid a multiple of 8, so item b runs on XCD b % 8 too.
// Tile t is given to XCD t % 8 and all of its items run there: the tile's
// activation rows are read into one L2 only, and the K ranges of the same
// weight rows are fetched together.
constexpr uint32_t kXcds = 8;
// Row blocks per work item, a compile-time even number so that the kernel's
// two weight buffers alternate in straight-line code; a run past the last
// row block loads clamped rows and stores nothing.
constexpr uint32_t kItemBlocks = 4;
// Row blocks per item when an item covers H K ranges: four ranges (all of a
// 2048-column K) take two blocks, so that a tile still splits into as many
// items and the persistent grid stays balanced.
constexpr uint32_t item_blocks(int H) { return H >= 4 ? kItemBlocks / 2u : kItemBlocks; }
// s_waitcnt operand: vector memory counter 0, the others at their maximum.
constexpr int kWaitVmcnt0 = 0x0F70;
struct SplitWork {
  uint32_t tile, split, first_block;
};
__device__ __forceinline__ SplitWork split_work(const SplitParams& p, uint32_t b) {
  const uint32_t per_tile = p.chunks * p.nsplit;
  const uint32_t i = b / kXcds;
  SplitWork w;
  w.tile = (i / per_tile) * kXcds + b % kXcds;
  w.split = i % per_tile % p.nsplit;
  w.first_block = i % per_tile / p.nsplit * p.item_blocks;
  return w;
}
uint32_t split_items(uint32_t max_tiles, uint32_t nsplit, uint32_t chunks) {
  return (max_tiles + kXcds - 1) / kXcds * kXcds * nsplit * chunks;
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

// Wave-uniform copies of values every lane holds alike. The builtin works on
// (signed) int: each 32-bit half goes through uint32_t, so that the low half
// of a pointer is zero-extended, not sign-extended, when widened.
__device__ __forceinline__ uint32_t uniform_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}
__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* ptr) {
  const uint64_t v = reinterpret_cast<uintptr_t>(ptr);
  const uint64_t lo = uniform_u32(static_cast<uint32_t>(v)), hi = uniform_u32(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>((hi << 32) | lo));
}

// One work item's tile as a workgroup sees it: the record (count 0 for an
// empty tile or one past the capacity) and, in lane m, the activation row of
// tile row m.
struct TileView {
  const uint8_t* blob;
  uint32_t start, count, lane_act;
};

// 16 bytes per lane from global memory straight into LDS: lane l's bytes
// land at dst + 16 l (dst wave-uniform).
__device__ __forceinline__ void load_lds16(const void* src, void* dst) {
  __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

// A tile record as wave-uniform (scalar) values.
struct TileRec {
  const uint8_t* blob;
  uint32_t start, count;
};
__device__ __forceinline__ TileRec uniform_rec(const TileView& v) {
  return TileRec{uniform_ptr(v.blob), uniform_u32(v.start), uniform_u32(v.count)};
}

// Reads an item's tile record with vector loads: they leave the LDS counter
// alone, so the MFMA loop's LDS waits never wait for the next item's record
// (a scalar load would count there).
template <int PROJ>
__device__ __forceinline__ TileView fetch_tile(const SplitParams& p, const SplitWork& wk, uint32_t m) {
  TileView v{nullptr, 0u, 0u, 0u};
  if (wk.tile >= p.max_tiles) return v;
  const uint64_t* rec = reinterpret_cast<const uint64_t*>(p.tiles + wk.tile);
  const uint64_t r0 = __hip_atomic_load(const_cast<uint64_t*>(rec), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t r1 = __hip_atomic_load(const_cast<uint64_t*>(rec + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v.blob = reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(r0));
  v.start = static_cast<uint32_t>(r1);
  v.count = static_cast<uint32_t>(r1 >> 32);
  if constexpr (PROJ == 2) v.lane_act = p.tile_rows[wk.tile * kTileTokens + m];
  return v;
}

// One wave's weights of one row block over the K range: packed words and the
// scale / bias runs of its 2 x 16 rows.
template <int META, int S, int NSTEP>
struct BlockWeights {
  static constexpr int GPR = NSTEP / S;
  uint32_t w[2][NSTEP];
  MetaRun<META, GPR> sb[2], bb[2];
};

// Where one wave's weights live: projection offsets within a blob and the
// geometry of the matrix (N rows of K columns).
struct WaveMatrix {
  size_t q_off, s_off, b_off;
  uint32_t N, K, G, ngroups, wave_row;  // wave_row: the wave's first row within a block
};

// Groups of 64 columns (S = 2) load 16 bytes per lane: for the group pair
// (2p, 2p + 1) lane q reads words 4q .. 4q+3 of the pair's 16, so a row's four
// lanes read 64 contiguous bytes (an isolated stream of this shape runs at 5.7
// TB/s against 4.5 for 8 bytes per lane and group). compute_block then swaps
// halves between lanes q and q + 2 (v_permlane32_swap), after which lane q
// holds words 2 pi(q), 2 pi(q) + 1 of both groups, pi(q) = (q & 1) * 2 + q / 2.
template <int S>
constexpr bool kPairLoads = S == 2;
__device__ __forceinline__ uint32_t pair_slot(uint32_t q) { return ((q & 1u) << 1) | (q >> 1); }

template <int META, int S, int NSTEP, uint32_t kWgRows>
__device__ __forceinline__ void load_block(BlockWeights<META, S, NSTEP>& W, const WaveMatrix& mx,
                                           const uint8_t* blob, uint32_t block, uint32_t split, uint32_t m,
                                           uint32_t q) {
  constexpr int GPR = NSTEP / S;
  const uint32_t g0 = split * GPR;
#pragma unroll
  for (uint32_t nb = 0; nb < 2u; ++nb) {
    uint32_t r = block * kWgRows + mx.wave_row + nb * kBlockRows + m;
    r = r < mx.N ? r : mx.N - 1u;
    // A group is 32 S columns, 4 S words: the offsets of the runs within the
    // range are compile-time constants (load immediates).
    constexpr uint32_t kGroupWords = 4u * S;
    const uint8_t* qrow = blob + mx.q_off + static_cast<size_t>(r) * (mx.K / 2u) + g0 * kGroupWords * 4u;
    if constexpr (kPairLoads<S>) {
      static_assert(GPR % 2 == 0, "group pairs");
      const uint8_t* qlane = qrow + 16u * q;
#pragma unroll
      for (int gp = 0; gp < GPR / 2; ++gp) word_run<4>(qlane + 2u * gp * kGroupWords * 4u, &W.w[nb][4 * gp]);
    } else {
      const uint8_t* qlane = qrow + 4u * S * q;
#pragma unroll
      for (int gg = 0; gg < GPR; ++gg) word_run<S>(qlane + gg * kGroupWords * 4u, &W.w[nb][gg * S]);
    }
    const size_t mi = static_cast<size_t>(r) * mx.ngroups + g0;
    W.sb[nb].load(blob + mx.s_off, mi);
    W.bb[nb].load(blob + mx.b_off, mi);
  }
}

// H consecutive K ranges of the tile, staged together.
template <int PROJ, int NSTEP, int NT, int H>
struct SplitLds {
  static constexpr uint32_t KS = 32u * NSTEP;
  static constexpr uint32_t RS = KS + 8u;  // row stride (bf16), padded against bank conflicts
  uint16_t a[H][NT][kTileTokens][RS];
  __attribute__((aligned(16))) float xs[H][NSTEP][kTileTokens];  // group sums (at most NSTEP groups per range)
};

// MFMAs of one block against staged range `half` of the tile, added to
// `total` (cleared first when `first`), then, when `last`, its partial sums.
// MFMA row m reads tile row min(m, count - 1); the D rows of lane q are tile
// rows 4q .. 4q+3 (those past count are not stored).
// SwiGLU fused into gate/up: a 16-pair x 64-row exchange of the up sums, then
// of h (padded row against bank conflicts).
using FuseLds = float[kTileTokens][65];

template <int META, int PROJ, int S, int NSTEP, int NT, int H, uint32_t kWgRows, bool FUSE>
__device__ __forceinline__ void compute_block(const SplitParams& p, const SplitLds<PROJ, NSTEP, NT, H>& lds,
                                              const BlockWeights<META, S, NSTEP>& W, const WaveMatrix& mx,
                                              uint32_t block, uint32_t split, uint32_t half, bool first, bool last,
                                              f32x4 (&total)[2], const float (&pw4)[4], uint32_t start,
                                              uint32_t rows, uint32_t pr, uint32_t m, uint32_t q, FuseLds& fu) {
  constexpr int GPR = NSTEP / S;
  constexpr uint32_t G8 = (32u * S) / 8u;  // 16-byte units per group
  // The tile row indices pass through an opaque copy per block: every block
  // of an item reads the same LDS operands, and left alone the compiler keeps
  // all of them in registers across the blocks instead of re-reading them.
  uint32_t ar = m < rows ? m : rows - 1u;
  asm volatile("" : "+v"(ar));
  if (first) total[0] = total[1] = f32x4{0.f, 0.f, 0.f, 0.f};
  // k-slot of this lane within a group: its words are S * slot .. S * slot + S-1.
  const uint32_t slot = kPairLoads<S> ? pair_slot(q) : q;
  uint32_t pw[2][4];  // pair loads: the swapped words of the current group pair
#pragma unroll
  for (int gg = 0; gg < GPR; ++gg) {
    if constexpr (kPairLoads<S>) {
      if (gg % 2 == 0) {
#pragma unroll
        for (uint32_t nb = 0; nb < 2u; ++nb)
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            const auto r = __builtin_amdgcn_permlane32_swap(W.w[nb][2 * gg + s2], W.w[nb][2 * gg + 2 + s2], false, false);
            pw[nb][s2] = r[0];      // group gg
            pw[nb][2 + s2] = r[1];  // group gg + 1
          }
      }
    }
    bf16x8 a[S][NT];
#pragma unroll
    for (int s2 = 0; s2 < S; ++s2)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        a[s2][t] = as_operand(*reinterpret_cast<const uint4*>(&lds.a[half][t][ar][(gg * G8 + S * slot + s2) * 8u]));
    // The group sums of the lane's four D rows (tile rows 4q .. 4q+3) in one
    // read; rows past the count read stale sums, and their totals are
    // never stored.
    const float4 x4 = *reinterpret_cast<const float4*>(&lds.xs[half][gg][4u * q]);
    const float xs[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
    for (uint32_t nb = 0; nb < 2u; ++nb) {
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 < S; ++s2) {
        uint32_t word;
        if constexpr (kPairLoads<S>)
          word = pw[nb][(gg % 2) * 2 + s2];
        else
          word = W.w[nb][gg * S + s2];
        const bf16x8 b = nibble_operand(word);
#pragma unroll
        for (int t = 0; t < NT; ++t) d = mfma(a[s2][t], b, d);
      }
      const float sc = W.sb[nb].get(gg);
      const float cb = W.bb[nb].get(gg) - 128.0f * sc;
#pragma unroll
      // Two FMAs per element (written as one sum the compiler keeps a
      // multiply, an FMA and an add).
      for (int j = 0; j < 4; ++j) total[nb][j] = __builtin_fmaf(sc, d[j], __builtin_fmaf(cb, xs[j], total[nb][j]));
    }
  }
  if (!last) {
    // The totals carry into the block's next range: materialised here, so
    // the compiler does not sink this range's epilogue past the next
    // block's loads (which keeps every group's accumulators live and spills).
#pragma unroll
    for (uint32_t nb = 0; nb < 2u; ++nb)
#pragma unroll
      for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(total[nb][j]));
    return;
  }
  if constexpr (FUSE) {
    // The block's 64 rows are one group of h (G = 64) and the whole of K is
    // summed (one partial): h = SwiGLU(gate, up) is formed here, as
    // swiglu_terms_kernel forms it from the partials (0 + sum, the same
    // expression), and written as its bf16 terms and group sum. Up waves
    // hand their sums to the gate waves through LDS; the gate waves leave h
    // there; then 128 threads take (pair, 8-row word) each.
    static_assert(PROJ == 2 && kWgRows == 64u, "fused SwiGLU: gate/up blocks of 64 rows");
#pragma unroll
    for (uint32_t nb = 0; nb < 2u; ++nb)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (pr == 1u) fu[4u * q + j][mx.wave_row + nb * kBlockRows + m] = total[nb][j];
    __syncthreads();
    if (pr == 0u) {
#pragma unroll
      for (uint32_t nb = 0; nb < 2u; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float& cell = fu[4u * q + j][mx.wave_row + nb * kBlockRows + m];
          const float g = 0.0f + total[nb][j], u = 0.0f + cell;
          const float sig = __builtin_amdgcn_rcpf(1.0f + expf(-g));
          cell = g * sig * u;
        }
    }
    __syncthreads();
    const uint32_t tid = threadIdx.x;
    if (tid < kTileTokens * 8u) {
      const uint32_t pj = tid / 8u, wd = tid % 8u;
      const uint32_t I = mx.N;
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = fu[pj][wd * 8u + k];
      const size_t pair = start + pj;
      float rep[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (uint32_t t = 0; t < kActSplit; ++t) {
        uint16_t o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int k = word_k(e);
          o[e] = bf16_rne(v[k] - rep[k]);
          rep[k] += bf16_to_f32(o[e]);
        }
        uint4 pk;
        pk.x = o[0] | (static_cast<uint32_t>(o[1]) << 16);
        pk.y = o[2] | (static_cast<uint32_t>(o[3]) << 16);
        pk.z = o[4] | (static_cast<uint32_t>(o[5]) << 16);
        pk.w = o[6] | (static_cast<uint32_t>(o[7]) << 16);
        if (pj < rows) *reinterpret_cast<uint4*>(p.h_terms + (pair * kActSplit + t) * I + block * 64u + wd * 8u) = pk;
      }
      float gsum = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) gsum += rep[k];
      for (uint32_t x = 1; x < 8u; x <<= 1) gsum += __shfl_xor(gsum, static_cast<int>(x));
      if (pj < rows && wd == 0u) p.h_sums[pair * (I / 64u) + block] = gsum;
    }
    __syncthreads();  // fu is rewritten by the next block's epilogue
    return;
  }
#pragma unroll
  for (uint32_t nb = 0; nb < 2u; ++nb) {
    const uint32_t r = block * kWgRows + mx.wave_row + nb * kBlockRows + m;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t pj = 4u * q + j;
      if (pj < rows && r < mx.N) {
        const size_t pair = start + pj;
        if constexpr (PROJ == 2)
          p.out[((static_cast<size_t>(split) * 2u + pr) * p.P + pair) * mx.N + r] = total[nb][j];
        else
          p.out[(static_cast<size_t>(split) * p.P + pair) * mx.N + r] = pw4[j] * total[nb][j];
      }
    }
  }
}

// The workgroups are persistent: workgroup b takes items b, b + grid, ...
// (the grid a multiple of 8, so all of them on one XCD, and their tiles in
// ascending order). Empty tiles come last, so a workgroup stops at the first
// one. The next item's tile record is fetched while the current one is
// staged, and the next item's first block is in flight while the current
// item's last block computes.
template <int META, int PROJ, int S, int NSTEP, int NT, int H, bool FUSE>
__global__ __launch_bounds__(kSplitThreads) __attribute__((amdgpu_waves_per_eu(2))) void split_kernel(SplitParams p) {
  constexpr uint32_t KS = 32u * NSTEP;
  constexpr int GPR = NSTEP / S;  // groups per range
  constexpr uint32_t kWgRows = split_rows<PROJ>();
  constexpr uint32_t kUnitCols = KS / 8u;  // 16-byte units per staged row
  constexpr uint32_t kUnitsPerThread = NT * kTileTokens * kUnitCols / kSplitThreads;
  static_assert(NT * kTileTokens * kUnitCols % kSplitThreads == 0, "staging units");
  static_assert(H * GPR * kTileTokens % kSplitThreads == 0 || H * GPR * kTileTokens < kSplitThreads,
                "group sums: whole passes of the workgroup");
  constexpr uint32_t kSumPasses = (H * GPR * kTileTokens + kSplitThreads - 1u) / kSplitThreads;
  constexpr uint32_t kIB = item_blocks(H);
  constexpr uint32_t kProjWaves = PROJ == 2 ? kSplitWaves / 2u : kSplitWaves;
  __shared__ __align__(16) SplitLds<PROJ, NSTEP, NT, H> lds;
  __shared__ float fuse_lds[FUSE ? kTileTokens : 1][FUSE ? 65 : 1];
  FuseLds& fu = *reinterpret_cast<FuseLds*>(&fuse_lds[0][0]);  // referenced only when FUSE

  // Per-lane indices and the wave's matrix, derived from the thread index.
  // Inside the item loop the index is re-read opaquely, so that what derives
  // from it is recomputed per item rather than kept live (or spilled) across
  // the loop.
  auto wave_matrix = [&](uint32_t wave) {
    WaveMatrix mx;
    const osm_expert_offsets off = osm_expert_layout(p.g);
    const uint32_t pr = wave / kProjWaves;
    mx.K = PROJ == 2 ? p.g.hidden : p.g.inter;
    mx.N = PROJ == 2 ? p.g.inter : p.g.hidden;
    mx.G = p.g.group;
    mx.ngroups = mx.K / mx.G;
    mx.wave_row = (wave % kProjWaves) * kWaveRows;
    mx.q_off = PROJ == 2 ? (pr ? off.up_q : off.gate_q) : off.down_q;
    mx.s_off = PROJ == 2 ? (pr ? off.up_s : off.gate_s) : off.down_s;
    mx.b_off = PROJ == 2 ? (pr ? off.up_b : off.gate_b) : off.down_b;
    return mx;
  };

  uint32_t item = blockIdx.x;
  if (item >= p.items) return;
  SplitWork wk = split_work(p, item);
  // The loop carries the record as scalars and only the activation row of
  // tile row m per lane.
  uint32_t tid0 = threadIdx.x;
  asm volatile("" : "+v"(tid0));
  const TileView first = fetch_tile<PROJ>(p, wk, tid0 % 16u);
  TileRec tl = uniform_rec(first);
  uint32_t tl_lane_act = first.lane_act;
  // An empty first tile ends the workgroup at once (a tile past the capacity
  // has no blob at all).
  if (tl.count == 0u) return;
  // Weight register sets: sub-block s of an item is computed from W[s %
  // kNBuf] while the next kNBuf - 1 sub-blocks are in flight. (Three sets,
  // two sub-blocks in flight, measured no faster for the fused gate/up at 254
  // registers: its waves do not wait on the weights' latency.) kSub is even,
  // so every item starts at W[0].
  constexpr uint32_t kSub = kIB * H;  // sub-blocks per item
  constexpr uint32_t kNBuf = 2u;
  static_assert(kSub % kNBuf == 0u, "items start at W[0]");
  BlockWeights<META, S, NSTEP> W[kNBuf];
  // The first item's first kNBuf - 1 sub-blocks.
  {
    const WaveMatrix mx0 = wave_matrix(uniform_u32(tid0 / kWave));
#pragma unroll
    for (uint32_t s0 = 0; s0 + 1u < kNBuf; ++s0)
      load_block<META, S, NSTEP, kWgRows>(W[s0], mx0, tl.blob, wk.first_block + s0 / H, wk.split * H + s0 % H,
                                          tid0 % 16u, tid0 % kWave / 16u);
  }
  while (tl.count != 0u) {
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t lane = tid % kWave, wave = uniform_u32(tid / kWave);
    const uint32_t m = lane % 16u, q = lane / 16u;
    const uint32_t pr = wave / kProjWaves;
    const WaveMatrix mx = wave_matrix(wave);
    const uint8_t* blob = tl.blob;
    const uint32_t start = tl.start;
    const uint32_t rows = tl.count;
    const uint32_t split = wk.split, fb = wk.first_block;
    // Activation row of tile row m: its token (gate/up) or the pair itself (down).
    const uint32_t lane_act = PROJ == 2 ? tl_lane_act : start + m;

    // The tile's activation rows for this range, then the next item's record.
    // Unit u: term u / (16 * KS/8), tile row (u / (KS/8)) % 16, 16-byte
    // column unit u % (KS/8). With 512-column ranges a wave instruction
    // covers exactly one staged row, and the loads write LDS directly (lane
    // l's 16 bytes land at the row start + 16 l): no registers hold the tile,
    // and rows past the tile's count are skipped by a wave-uniform branch
    // (their LDS rows keep stale data that no MFMA row reads). Narrower
    // ranges go through registers, where rows past the count load the last
    // real row (no branch around the loads).
    auto act_row = [&](uint32_t j) -> uint32_t { return __shfl(lane_act, static_cast<int>(j)); };
    constexpr bool kDirect = kUnitCols == kWave;
    static_assert(kDirect || H == 1, "several ranges per item are staged directly");
    uint4 stage[kDirect ? 1u : kUnitsPerThread];
#pragma unroll
    for (int h = 0; h < H; ++h) {
#pragma unroll
      for (uint32_t i = 0; i < kUnitsPerThread; ++i) {
        const uint32_t u = tid + i * kSplitThreads;
        const uint32_t term = u / (kTileTokens * kUnitCols), row = (u / kUnitCols) % kTileTokens, cu = u % kUnitCols;
        const uint32_t arow = act_row(row < rows ? row : rows - 1u);
        const uint16_t* src =
            p.terms + (static_cast<size_t>(arow) * p.term_count + term) * mx.K + (split * H + h) * KS + cu * 8u;
        if constexpr (kDirect) {
          if (uniform_u32(row) < rows) load_lds16(src, &lds.a[h][term][row][0]);  // term, row: wave-uniform
        } else {
          stage[i] = ldg16(src);
        }
      }
    }
    // Group sums: thread (sg, srow) for sg < H * GPR (range sg / GPR), in
    // kSumPasses passes of the workgroup; the others load a valid element and
    // do not store it.
    const uint32_t srow = tid % kTileTokens;
    const uint32_t sarow = act_row(srow < rows ? srow : rows - 1u);
    float xsum[kSumPasses];
#pragma unroll
    for (uint32_t ps = 0; ps < kSumPasses; ++ps) {
      const uint32_t sg = (tid + ps * kSplitThreads) / kTileTokens;
      xsum[ps] = p.sums[static_cast<size_t>(sarow) * mx.ngroups + split * H * GPR + (sg < H * GPR ? sg : 0u)];
    }

    // down: the pair weights of this lane's four D rows (tile rows 4q..4q+3,
    // clamped), loaded with the staging. Loaded per block instead, each would
    // wait for every older load -- the next block's weights included.
    float pw4[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if constexpr (PROJ == 1) {
#pragma unroll
      for (int j = 0; j < 4; ++j) pw4[j] = p.pair_w[start + (4u * q + j < rows ? 4u * q + j : rows - 1u)];
    }
    const uint32_t next = item + gridDim.x;
    const SplitWork wk_next = split_work(p, next);
    const TileView tl_next = next < p.items ? fetch_tile<PROJ>(p, wk_next, m) : TileView{nullptr, 0u, 0u, 0u};

    if constexpr (kDirect) {
      // Every wave's direct loads have landed before the barrier (the other
      // waves read them).
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    } else {
#pragma unroll
      for (uint32_t i = 0; i < kUnitsPerThread; ++i) {
        const uint32_t u = tid + i * kSplitThreads;
        const uint32_t term = u / (kTileTokens * kUnitCols), row = (u / kUnitCols) % kTileTokens, cu = u % kUnitCols;
        *reinterpret_cast<uint4*>(&lds.a[0][term][row][cu * 8u]) = stage[i];
      }
    }
#pragma unroll
    for (uint32_t ps = 0; ps < kSumPasses; ++ps) {
      const uint32_t sg = (tid + ps * kSplitThreads) / kTileTokens;
      if (sg < H * GPR) lds.xs[sg / GPR][sg % GPR][srow] = xsum[ps];
    }
    __syncthreads();

    // The item's blocks, straight-line, so that each wait is for exactly the
    // block about to be computed. Before computing sub-block sb the loads of
    // sub-block sb + kNBuf - 1 are issued: this item's, or past its end the
    // next item's first ones (or, with no next item, this item's first ones
    // again, read and not used). The next record has arrived by the end of
    // the first block (its wait covers every older load) and turns into
    // scalars there.
    // Sub-block sb is range sb % H of block fb + sb / H; a block's H ranges
    // are consecutive sub-blocks and share its totals.
    TileRec next_rec{blob, 0u, 0u};
    f32x4 total[2];
#pragma unroll
    for (uint32_t sb = 0; sb < kSub; ++sb) {
      const uint32_t t = sb + kNBuf - 1u;
      if (t < kSub) {
        load_block<META, S, NSTEP, kWgRows>(W[t % kNBuf], mx, blob, fb + t / H, split * H + t % H, m, q);
      } else {
        const uint32_t u = t - kSub;
        const bool has_next = next_rec.count != 0u;
        load_block<META, S, NSTEP, kWgRows>(W[t % kNBuf], mx, has_next ? next_rec.blob : blob,
                                            (has_next ? wk_next.first_block : fb) + u / H,
                                            (has_next ? wk_next.split : split) * H + u % H, m, q);
      }
      __builtin_amdgcn_sched_barrier(0);
      compute_block<META, PROJ, S, NSTEP, NT, H, kWgRows, FUSE>(p, lds, W[sb % kNBuf], mx, fb + sb / H, split,
                                                               sb % H, sb % H == 0u, sb % H == H - 1u, total, pw4,
                                                               start, rows, pr, m, q, fu);
      if (sb == 0u) next_rec = uniform_rec(tl_next);
    }
    __syncthreads();  // the LDS tile is restaged by the next item
    item = next;
    wk = wk_next;
    tl = next_rec;
    tl_lane_act = tl_next.lane_act;
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
      for (int k = 0; k < 8; ++k) {
        // SwiGLU with the hardware reciprocal (within 1 ulp; the terms that
        // follow carry 16 significand bits): the IEEE division's ten
        // instructions per element were a sixth of this pass's vector work.
        const float sig = __builtin_amdgcn_rcpf(1.0f + expf(-gs[k]));
        v[k] = gs[k] * sig * us[k];
      }
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

// The same sums four columns per thread with 16-byte loads (D % 4 == 0,
// every row 16-byte aligned); each column's additions keep the order above.
__global__ void combine4_kernel(const float* __restrict__ partial, uint32_t nsplit, uint32_t P,
                                const uint32_t* __restrict__ pair_pos, uint32_t T, uint32_t D, uint32_t nslot,
                                const float* __restrict__ residual, float* __restrict__ y) {
  const uint32_t D4 = D / 4u;
  const size_t n = static_cast<size_t>(T) * D4;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint32_t t = static_cast<uint32_t>(i / D4), r4 = static_cast<uint32_t>(i % D4);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    uint32_t j = 0;
    if (nsplit == 1u) {
      // One K range (the usual case): up to twelve slots' positions, then
      // all their rows, are loaded before the adds, which keep slot order
      // (top-10 + shared: one round trip for the positions and one for the
      // rows). Slots past nslot load slot 0's row and are not added.
      constexpr uint32_t kBatch = 12;
      const float4* part4 = reinterpret_cast<const float4*>(partial);
      for (; j < nslot; j += kBatch) {
        uint32_t pos[kBatch];
#pragma unroll
        for (uint32_t q = 0; q < kBatch; ++q) pos[q] = pair_pos[t * nslot + (j + q < nslot ? j + q : 0u)];
        float4 v[kBatch];
#pragma unroll
        for (uint32_t q = 0; q < kBatch; ++q) v[q] = part4[static_cast<size_t>(pos[q]) * D4 + r4];
#pragma unroll
        for (uint32_t q = 0; q < kBatch; ++q) {
          if (j + q < nslot) {
            acc.x += v[q].x;
            acc.y += v[q].y;
            acc.z += v[q].z;
            acc.w += v[q].w;
          }
        }
      }
    }
    for (; j < nslot; ++j) {
      const size_t pos = pair_pos[t * nslot + j];
      for (uint32_t sp = 0; sp < nsplit; ++sp) {
        const float4 v = reinterpret_cast<const float4*>(partial + (static_cast<size_t>(sp) * P + pos) * D)[r4];
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
      }
    }
    if (residual) {
      const float4 x = reinterpret_cast<const float4*>(residual)[i];
      acc = make_float4(x.x + acc.x, x.y + acc.y, x.z + acc.z, x.w + acc.w);
    }
    reinterpret_cast<float4*>(y)[i] = acc;
  }
}

// Columns per K range of the router GEMM: the widest of 512 / 256 / 128 that
// divides the hidden size (a multiple of 128 on the grouped path).
uint32_t router_range(uint32_t D) { return D % 512u == 0 ? 512u : (D % 256u == 0 ? 256u : 128u); }

// Columns per K range: the widest of 512 / 256 / 128 that divides K and
// keeps one row's scale (or bias) run for the range within 16 bytes, so that
// a wave's two blocks of weights in flight fit its registers (512 columns
// for bf16 / f16 metadata at group 64, or any metadata at group 128).
uint32_t range_cols(const osm_expert_geometry& g, uint32_t K) {
  const uint32_t meta_bytes = g.meta_dtype == OSM_META_F32 ? 4u : 2u;
  for (uint32_t r = 512u; r > 128u; r /= 2u)
    if (K % r == 0u && r / g.group * meta_bytes <= 16u) return r;
  return 128u;
}

void set_item_blocks(SplitParams& sp, uint32_t row_blocks, uint32_t nsplit, uint32_t ib = kItemBlocks) {
  sp.nsplit = nsplit;
  sp.item_blocks = ib;
  sp.chunks = (row_blocks + ib - 1u) / ib;
  sp.items = split_items(sp.max_tiles, nsplit, sp.chunks);
}

// Workgroups of a persistent split kernel: as many as are resident at once
// (the instantiation's workgroups per compute unit times the compute units),
// a multiple of 8, and no more than there are items (also a multiple of 8).
// A larger grid would leave workgroups waiting for a free slot, to start
// their whole item list after the others end.
template <int META, int PROJ, int S, int NSTEP, int NT, int H, bool FUSE>
uint32_t split_grid(uint32_t items) {
  static const uint32_t per_cu = [] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, split_kernel<META, PROJ, S, NSTEP, NT, H, FUSE>,
                                                     kSplitThreads, 0) !=
            hipSuccess ||
        n < 1)
      n = 1;
    return static_cast<uint32_t>(n);
  }();
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    cus = 1;
  uint32_t grid = per_cu * static_cast<uint32_t>(cus) / kXcds * kXcds;
  if (grid < kXcds) grid = kXcds;
  return items < grid ? items : grid;
}

template <int META, int PROJ, int S, int NSTEP, int NT, int H, bool FUSE>
void launch_split_r(const SplitParams& sp, hipStream_t st) {
  // Only the ranges range_cols() can choose for this metadata and group are
  // instantiated (a wider one would not fit the registers).
  constexpr uint32_t kMetaBytes = META == OSM_META_F32 ? 4u : 2u;
  // Two ranges per item only with 512-column ranges (staged directly); the
  // fused SwiGLU only for gate/up at group 64 (S = 2).
  if constexpr (NSTEP / S * kMetaBytes <= 16u && (H == 1 || NSTEP == 16) && (!FUSE || (PROJ == 2 && S == 2)))
    split_kernel<META, PROJ, S, NSTEP, NT, H, FUSE>
        <<<split_grid<META, PROJ, S, NSTEP, NT, H, FUSE>(sp.items), kSplitThreads, 0, st>>>(sp);
}

template <int META, int PROJ, int S, int NT, int H, bool FUSE>
void launch_split_s(const SplitParams& sp, hipStream_t st) {
  switch (range_cols(sp.g, PROJ == 2 ? sp.g.hidden : sp.g.inter)) {
    case 512: launch_split_r<META, PROJ, S, 16, NT, H, FUSE>(sp, st); break;
    case 256: launch_split_r<META, PROJ, S, 8, NT, H, FUSE>(sp, st); break;
    default: launch_split_r<META, PROJ, S, 4, NT, H, FUSE>(sp, st); break;
  }
}

template <int META, int PROJ, int NT, int H, bool FUSE>
void launch_split_meta(const SplitParams& sp, hipStream_t st) {
  switch (sp.g.group) {
    case 32: launch_split_s<META, PROJ, 1, NT, H, FUSE>(sp, st); break;
    case 64: launch_split_s<META, PROJ, 2, NT, H, FUSE>(sp, st); break;
    default: launch_split_s<META, PROJ, 4, NT, H, FUSE>(sp, st); break;
  }
}

// NT: activation terms (2 for fp32 activations, 1 for an exact bf16 input);
// H: K ranges per work item (2 only with 512-column ranges); FUSE: gate/up
// writes h itself (one partial, group 64).
template <int PROJ, int NT, int H, bool FUSE = false>
void launch_split(const SplitParams& sp, hipStream_t st) {
  switch (sp.g.meta_dtype) {
    case OSM_META_F32: launch_split_meta<OSM_META_F32, PROJ, NT, H, FUSE>(sp, st); break;
    case OSM_META_F16: launch_split_meta<OSM_META_F16, PROJ, NT, H, FUSE>(sp, st); break;
    default: launch_split_meta<OSM_META_BF16, PROJ, NT, H, FUSE>(sp, st); break;
  }
}

// A workgroup covers TT consecutive 16-token tiles with the same router rows
// (read once): TT = 2 from 256 tokens, where the grid still holds more than
// two workgroups per compute unit.
constexpr uint32_t kRouterTilesPerGroupFrom = 256;
template <int NS, int NSTEP, int TT>
void launch_router_gemm_steps(dim3 grid, hipStream_t st, const uint16_t* terms, uint32_t T, uint32_t D,
                              const uint16_t* router, const uint16_t* sgv, uint32_t E, float* planes,
                              const float* rnorm, const float* xnorm, float* bplanes) {
  // One-dimensional launch, padded to a multiple of the 8 XCDs.
  const uint32_t items = grid.x * grid.y * grid.z;
  const dim3 launch((items + 7u) / 8u * 8u);
  if (bplanes != nullptr)
    router_gemm_kernel<NS, NSTEP, TT, true><<<launch, kGroupedThreads, 0, st>>>(
        terms, T, D, router, sgv, E, planes, rnorm, xnorm, bplanes, grid.x, grid.y, grid.z);
  else
    router_gemm_kernel<NS, NSTEP, TT, false><<<launch, kGroupedThreads, 0, st>>>(
        terms, T, D, router, sgv, E, planes, rnorm, xnorm, bplanes, grid.x, grid.y, grid.z);
}
template <int NS, int TT>
void launch_router_gemm_tt(uint32_t rcols, dim3 grid, hipStream_t st, const uint16_t* terms, uint32_t T,
                           uint32_t D, const uint16_t* router, const uint16_t* sgv, uint32_t E, float* planes,
                           const float* rnorm, const float* xnorm, float* bplanes) {
  grid.y = (grid.y + TT - 1u) / TT;
  switch (rcols) {
    case 512:
      launch_router_gemm_steps<NS, 16, TT>(grid, st, terms, T, D, router, sgv, E, planes, rnorm, xnorm, bplanes);
      break;
    case 256:
      launch_router_gemm_steps<NS, 8, TT>(grid, st, terms, T, D, router, sgv, E, planes, rnorm, xnorm, bplanes);
      break;
    default:
      launch_router_gemm_steps<NS, 4, TT>(grid, st, terms, T, D, router, sgv, E, planes, rnorm, xnorm, bplanes);
      break;
  }
}
template <int NS>
void launch_router_gemm(uint32_t rcols, dim3 grid, hipStream_t st, const uint16_t* terms, uint32_t T, uint32_t D,
                        const uint16_t* router, const uint16_t* sgv, uint32_t E, float* planes, const float* rnorm,
                        const float* xnorm, float* bplanes) {
  if (T >= kRouterTilesPerGroupFrom)
    launch_router_gemm_tt<NS, 2>(rcols, grid, st, terms, T, D, router, sgv, E, planes, rnorm, xnorm, bplanes);
  else
    launch_router_gemm_tt<NS, 1>(rcols, grid, st, terms, T, D, router, sgv, E, planes, rnorm, xnorm, bplanes);
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

uint32_t osmd_moe_grouped_splits(const osm_expert_geometry* g, uint32_t cols) { return cols / range_cols(*g, cols); }

uint32_t osmd_moe_grouped_router_parts(uint32_t hidden) { return hidden / router_range(hidden); }

int osmd_moe_grouped(const osmd_moe_grouped_args* a, osmd_stream s) {
  const hipStream_t st = static_cast<hipStream_t>(s);
  const osmd_moe_args& m = a->moe;
  const osm_expert_geometry g = m.geom;
  const uint32_t T = m.tokens, D = g.hidden, I = g.inter, G = g.group;
  const uint32_t has_shared = (m.flags & OSMD_MOE_SHARED) ? 1u : 0u;
  const uint32_t nslot = m.top_k + has_shared;
  const uint32_t P = T * nslot;
  // The bucket pass's token index (slot_magic) is exact below 2^24 pairs.
  if (static_cast<uint64_t>(T) * nslot >= (1ull << 24)) return static_cast<int>(hipErrorInvalidValue);
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
  // Up to 16 tokens the per-token router kernel (one wavefront per router
  // row and token) has the shorter latency; beyond, the MFMA router GEMM,
  // whose K-range planes the selection adds (grouped decode at 40 / 56 / 64
  // tokens: 206 / 237 / 252 µs per layer step with the per-token router up
  // to 64 tokens, 198 / 225 / 238 µs with the GEMM from 16). One preparation serves both
  // GEMMs: 3 bf16 terms per activation for the router, of which the expert
  // GEMMs read the first 2 (the group sums are of those 2).
  const bool router_gemm = m.router_dtype == OSM_META_BF16 && (xbf16 || T > kRouterGemmMinTokens);
  if (xbf16 && !router_gemm) {
    // A router of another dtype runs as the per-token kernel, on fp32 input.
    const size_t n = static_cast<size_t>(T) * D;
    widen_bf16_kernel<<<blocks_for(n, 4096), 256, 0, st>>>(static_cast<const uint16_t*>(xin), n, m.x_norm);
    xin = m.x_norm;
    xbf16 = false;
  }
  // A bf16 input is exact as one bf16 term: the router GEMM and the gate/up
  // GEMM then read one term instead of three and two.
  const bool one_term = router_gemm && xbf16;
  const uint32_t x_term_count = router_gemm ? (one_term ? 1u : kRouterSplit) : kActSplit;
  // Error bounds of the GEMM's logits need the router's and the input's
  // 32-column norms.
  const bool gemm_bounds = router_gemm && a->router_norms != nullptr && a->x_norms != nullptr &&
                           a->bound_planes != nullptr;
  float* xnorms = gemm_bounds ? a->x_norms : nullptr;
  const size_t words = static_cast<size_t>(T) * (D / 8u);
  if (router_gemm) {
    if (one_term)
      prepare_kernel<true, 1><<<blocks_for(words, 4096), 256, 0, st>>>(xin, T, D, G, a->x_terms, a->x_sums, xnorms);
    else
      prepare_kernel<false, kRouterSplit><<<blocks_for(words, 4096), 256, 0, st>>>(xin, T, D, G, a->x_terms, a->x_sums,
                                                                                xnorms);
  } else {
    if (xbf16)
      prepare_kernel<true, kActSplit><<<blocks_for(words, 4096), 256, 0, st>>>(xin, T, D, G, a->x_terms, a->x_sums,
                                                                                xnorms);
    else
      prepare_kernel<false, kActSplit><<<blocks_for(words, 4096), 256, 0, st>>>(xin, T, D, G, a->x_terms, a->x_sums,
                                                                                xnorms);
  }
  int r = 0;
  osmd_moe_args ms = m;
  ms.x_bf16 = a->x_bf16 != 0 ? 1u : 0u;  // the exact path reads the input as given
  if (router_gemm) {
    const uint32_t nrows = m.expert_count + has_shared;
    const uint32_t rcols = router_range(D);
    const dim3 grid((nrows + kGroupedWaves * kBlockRows - 1) / (kGroupedWaves * kBlockRows),
                    (T + kTileTokens - 1) / kTileTokens, D / rcols);
    const uint16_t* router = static_cast<const uint16_t*>(m.router);
    const uint16_t* sgv = has_shared ? static_cast<const uint16_t*>(m.shared_gate_vec) : nullptr;
    float* bplanes = gemm_bounds ? a->bound_planes : nullptr;
    if (one_term)
      launch_router_gemm<1>(rcols, grid, st, a->x_terms, T, D, router, sgv, m.expert_count, a->logit_planes,
                            a->router_norms, xnorms, bplanes);
    else
      launch_router_gemm<kRouterSplit>(rcols, grid, st, a->x_terms, T, D, router, sgv, m.expert_count,
                                       a->logit_planes, a->router_norms, xnorms, bplanes);
    ms.logit_planes = a->logit_planes;
    ms.logit_parts = D / rcols;
    ms.bound_planes = gemm_bounds ? a->bound_planes : nullptr;
  } else {
    // The decode router kernel, one token per grid row (fp32 input).
    osmd_moe_args ra = m;
    ra.flags &= ~static_cast<uint32_t>(OSMD_MOE_RMSNORM);  // x is normalised above
    ra.x = static_cast<const float*>(xin);
    r = osmd_moe_router(&ra, s);
    if (r != 0) return r;
  }
  r = osmd_moe_select(&ms, s);
  if (r != 0) return r;
  auto bucket = [&](auto kernel) {
    kernel<<<1, kBucketThreads, 0, st>>>(m.ids, m.weights, has_shared ? m.shared_gate : nullptr, T, m.top_k, nslot,
                                         m.expert_count, m.expert_table, m.shared_expert, m.fallback_blob,
                                         a->pair_pos, a->pair_w, static_cast<Tile*>(a->tiles), tile_rows,
                                         a->tile_count, static_cast<uint32_t>(max_tiles), slot_magic(nslot));
  };
  if (P <= kBucketThreads)
    bucket(bucket_kernel<1>);
  else
    bucket(bucket_kernel<8>);

  SplitParams sp{};
  sp.g = g;
  sp.terms = a->x_terms;
  sp.term_count = x_term_count;
  sp.sums = a->x_sums;
  sp.tile_rows = tile_rows;
  sp.pair_w = a->pair_w;
  sp.tiles = static_cast<const Tile*>(a->tiles);
  sp.P = P;
  sp.max_tiles = static_cast<uint32_t>(max_tiles);
  sp.out = a->gu_part;
  // With 512-column ranges a gate/up work item covers two consecutive
  // ranges and writes one partial for both: half the partials written here
  // and read back by the SwiGLU launch.
  // With one activation term the staged tile is half as large, and four
  // ranges (a 2048-column K whole) fit: one partial per block.
  const uint32_t gu_ranges = osmd_moe_grouped_splits(&g, D);
  const bool gu_pairs = range_cols(g, D) == 512u && gu_ranges % 2u == 0u;
  const bool gu_quads = one_term && gu_pairs && gu_ranges % 4u == 0u;
  const uint32_t gu_h = gu_quads ? 4u : gu_pairs ? 2u : 1u;
  const uint32_t gu_splits = gu_ranges / gu_h;
  set_item_blocks(sp, (I + split_rows<2>() - 1) / split_rows<2>(), gu_splits, item_blocks(static_cast<int>(gu_h)));
  // One partial per row and groups of 64 (a gate/up block's rows): the
  // SwiGLU and h's terms are formed in the gate/up epilogue.
  const bool fuse = one_term && gu_quads && gu_splits == 1u && G == 64u && I % 64u == 0u;
  sp.h_terms = a->h_terms;
  sp.h_sums = a->h_sums;
  if (one_term) {
    if (fuse)
      launch_split<2, 1, 4, true>(sp, st);
    else if (gu_quads)
      launch_split<2, 1, 4>(sp, st);
    else if (gu_pairs)
      launch_split<2, 1, 2>(sp, st);
    else
      launch_split<2, 1, 1>(sp, st);
  } else {
    if (gu_pairs)
      launch_split<2, kActSplit, 2>(sp, st);
    else
      launch_split<2, kActSplit, 1>(sp, st);
  }
  const size_t hwords = static_cast<size_t>(P) * (I / 8u);
  if (!fuse)
    swiglu_terms_kernel<<<blocks_for(hwords, 4096), 256, 0, st>>>(a->gu_part, gu_splits, P, I, G, a->h_terms,
                                                                  a->h_sums);
  sp.terms = a->h_terms;
  sp.term_count = kActSplit;
  sp.sums = a->h_sums;
  sp.out = a->partial;
  const uint32_t dn_splits = osmd_moe_grouped_splits(&g, I);
  set_item_blocks(sp, (D + split_rows<1>() - 1) / split_rows<1>(), dn_splits);
  launch_split<1, kActSplit, 1>(sp, st);
  const float* residual = (m.flags & OSMD_MOE_RESIDUAL) ? static_cast<const float*>(m.x) : nullptr;
  if (D % 4u == 0u && ((reinterpret_cast<uintptr_t>(m.y) | reinterpret_cast<uintptr_t>(residual)) & 15u) == 0u)
    combine4_kernel<<<blocks_for(static_cast<size_t>(T) * (D / 4u), 4096), 256, 0, st>>>(
        a->partial, dn_splits, P, a->pair_pos, T, D, nslot, residual, m.y);
  else
    combine_kernel<<<blocks_for(static_cast<size_t>(T) * D, 4096), 256, 0, st>>>(
        a->partial, dn_splits, P, a->pair_pos, T, D, nslot, residual, m.y);
  return launch_status();
}

}  // extern "C"
