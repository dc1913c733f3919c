// moe_decode.hip -- fused gfx950 kernels for one routed-MoE sublayer decode.
//
// The reference runs this path as 56 blocking dispatches per token-layer with
// routing on the host (src/model/routed_moe.cpp:254-430). Here it is three
// stream-ordered kernels and no host round trip:
//
//   route_kernel    RMSNorm (optional) + router GEMV + shared-gate dot
//                   -> logits, sigmoid shared gate, normalised x.
//   gate_up_kernel  top-k selection (src/cpu/reference_ops.cpp:130-212,
//                   src/model/qwen_router.cpp:11-94), recomputed from the
//                   logits by every routed workgroup so no workgroup waits on
//                   another, proven equal to the reference's from per-logit
//                   error bounds or else recomputed in the reference's order,
//                   then the gate and up q4 GEMVs of every pick and of the
//                   shared expert with SwiGLU fused in the epilogue
//                   (shaders/q4_gemv.comp + shaders/swiglu.comp).
//   down_kernel     down q4 GEMV of every pick and of the shared expert with
//                   the routing weights and the sigmoid shared gate folded in,
//                   plus the optional residual add
//                   (shaders/weighted_accumulate.comp, checkpoint_moe_sublayer.cpp:21-33).
//
// Packed weights stream through 16-byte loads: one load is 4 words = 32
// columns, which never straddles a 32/64/128-column quantisation group, so
// each load needs one scale and one bias. The per-group algebra is the
// reference GEMV's: scale * sum(q * x) + bias * sum(x).
//
// When residency is decided on the host (a capped expert cache), a
// one-workgroup-per-token select kernel runs after route_kernel instead, the
// host reads the ids and writes the slot pointers, and gate_up_kernel reads
// those.
#include "device_common.hpp"

namespace {

using namespace osmk;

constexpr uint32_t kMaxSlots = OSMD_MAX_TOP_K + 1u;

// Timeline build (make timeline -> libosm_hip_timeline.so, OSMD_TIMELINE):
// workgroup 0 of each decode kernel, and the last workgroup, note the
// constant 100 MHz clock (s_memrealtime) at their phases in LDS and copy the
// notes to osmd_timeline when they end (a store at each phase would make the
// kernel's later waits on its vector memory operations wait for it too);
// osmd_timeline_read copies the slots out. Every launch overwrites them, so
// after a graph replay they hold its last layer's. The product build
// compiles all of this to nothing.
#ifdef OSMD_TIMELINE
constexpr int kTimelineSlots = 32;
__device__ unsigned long long osmd_timeline[kTimelineSlots];
__shared__ unsigned long long osmd_timeline_lds[kTimelineSlots];
__device__ __forceinline__ bool timeline_first() { return blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0; }
__device__ __forceinline__ bool timeline_last() {
  return blockIdx.x == gridDim.x - 1u && blockIdx.y == gridDim.y - 1u && blockIdx.z == gridDim.z - 1u;
}
#define OSMD_STAMP(slot, who)                                                                      \
  do {                                                                                             \
    if ((who) && threadIdx.x == 0) osmd_timeline_lds[(slot)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#define OSMD_STAMP_FLUSH(lo, hi, who)                                                \
  do {                                                                               \
    if ((who) && threadIdx.x == 0)                                                   \
      for (int s_ = (lo); s_ < (hi); ++s_) osmd_timeline[s_] = osmd_timeline_lds[s_]; \
  } while (0)
#else
#define OSMD_STAMP(slot, who) ((void)0)
#define OSMD_STAMP_FLUSH(lo, hi, who) ((void)0)
#endif
// Slots: route 0-1 (first workgroup start, end), 2-3 (last workgroup);
// gate/up's workgroup 0 (slot 0, the publisher) 4 start, 5 logits loaded
// and reduced, 6 ranked, 7 certificate decided, 8 selection done, 9 weights
// requested, 10 rows stored, 11 end; down's workgroup 0 12 start, 13 weights
// requested, 14 end; the last workgroup's end: gate/up 15, down 16.

// Blob of slot j for token t: resolved pointers, or one fixed expert (the
// single-expert operator).
struct SlotSource {
  const uint8_t* const* ptrs;  // [B, nslot] or null
  const uint8_t* single;
  uint32_t nslot;
  __device__ __forceinline__ const uint8_t* blob(uint32_t t, uint32_t j) const {
    return ptrs ? ptrs[static_cast<size_t>(t) * nslot + j] : single;
  }
};


// What a routed workgroup needs to select its token's experts: the logits
// and their bounds (or the router GEMM's planes), and, for the exact path,
// the router and the input it was applied to.
struct RouteView {
  const float* logits;                // [B, E]
  const float* bounds;                // [B, E] bound of each logit, or null (no bound: exact path)
  const float* planes;                // null, or `parts` planes [B][E + 1] of partial sums
  const float* bound_planes;          // with planes: [parts][B][E + 1] bound parts, or null
  uint32_t parts, tokens;
  float* logits_out;                  // [B, E]  with planes: the summed logits
  float* gate_out;                    // [B]     with planes: the shared gate
  uint32_t expert_count, top_k, norm_topk_prob, has_shared;
  const uint8_t* const* expert_table;  // [E] or null (picks read `fallback`)
  const uint8_t* shared_expert;
  const uint8_t* fallback;
  uint32_t* ids;                      // [B, k]   published outputs
  float* weights;                     // [B, k]
  float* mass;                        // [B]
  const uint8_t** slot_ptrs;          // [B, nslot]
  uint32_t* stats;                    // null, or the four routing counters
  // The exact path: router [E, D] (router_dtype), the router's input x
  // [B, D] (fp32, or bf16 when x_bf16), RMS-normalised first when rms.
  const void* router;
  uint32_t router_dtype, router_group, hidden;
  const void* x;
  uint32_t x_bf16, rms;
  const float* norm_weight;
  float rms_eps;
};

// Entry i of a slot list (osmd_slot_list_add's packing; i is uniform).
__device__ __forceinline__ uint32_t slot_at(const osmd_slot_list& l, uint32_t i) {
  return static_cast<uint32_t>((i < 12u ? l.lo >> (5u * i) : l.hi >> (5u * (i - 12u))) & 31u);
}

struct GateUpParams {
  osm_expert_geometry g;
  SlotSource src;
  RouteView rv;
  const float* x;  // [B, D]
  float* h;        // [B, nslot, I]
  osmd_slot_list list;  // slots from src (count 0: all nslot, in order; the grid covers list.count)
};

// The down kernel's three forms: the fused sum over every slot (y); the
// partials of the listed slots only (parts); y from the partials of every
// slot, accumulated as the fused form accumulates (combine).
enum DownMode : int { kDownFused = 0, kDownParts = 1, kDownCombine = 2 };

struct DownParams {
  osm_expert_geometry g;
  SlotSource src;
  uint32_t top_k;            // slots [0, top_k) take weights[], the rest shared_gate
  const float* weights;      // [B, top_k] or null (weight 1)
  const float* shared_gate;  // [B] or null (weight 1)
  const uint8_t* fallback;   // read in place of a null slot pointer (weight 0)
  const float* h;            // [B, nslot, I]
  const float* residual;     // [B, D] or null
  float* y;                  // [B, D]
  osmd_slot_list list;       // kDownParts: the slots to run
  float* parts;              // kDownParts (out) / kDownCombine (in): [B][nslot][D][LPR] per-lane partials
};


// ---------------------------------------------------------------------------
// Router elements as loaded, 8 at a time. A wavefront of the router GEMV
// owns one router row (route_block), kept as loaded until the FMA.
constexpr int kRouteWaves = 4;

template <int RD>
struct Raw8 {  // 8 router elements as loaded
  uint4 v[RD == OSM_META_F32 ? 2 : 1];
};
// Affine q8: two words of four bytes and the scale and bias of each word's
// group (a group is a multiple of 4 columns, so a word never straddles one).
template <>
struct Raw8<OSM_ROUTER_AFFINE_Q8> {
  uint2 q;
  float s[2], b[2];
};

// Row r of an affine-q8 matrix of `rows` rows held as one buffer
// [packed rows x D/4][scales rows x D/g][biases rows x D/g]: element c is
// scale * q + bias, the product rounded before the add, as the reference's
// dequantisation computes it (reference_ops.cpp:48-63).
struct Q8Row {
  const uint32_t* q;
  const float* s;
  const float* b;
  uint32_t group;
};
__device__ __forceinline__ Q8Row q8_row(const void* base, uint32_t rows, uint32_t r, uint32_t D, uint32_t group) {
  const uint32_t* q = static_cast<const uint32_t*>(base);
  const uint32_t gpr = D / group;
  const float* s = reinterpret_cast<const float*>(q + static_cast<size_t>(rows) * (D / 4u));
  const float* b = s + static_cast<size_t>(rows) * gpr;
  return Q8Row{q + static_cast<size_t>(r) * (D / 4u), s + static_cast<size_t>(r) * gpr,
               b + static_cast<size_t>(r) * gpr, group};
}
// scale * q + bias with the product rounded first: hipcc would otherwise
// fuse the two into one FMA.
__device__ __forceinline__ float dequant_q8(float s, float q, float b) {
#pragma clang fp contract(off)
  return s * q + b;
}
__device__ __forceinline__ void load_q8x8(const Q8Row& row, uint32_t c, Raw8<OSM_ROUTER_AFFINE_Q8>& r) {
  r.q = ldg8(row.q + c / 4u);
  r.s[0] = ldg<float>(row.s + c / row.group);
  r.b[0] = ldg<float>(row.b + c / row.group);
  r.s[1] = ldg<float>(row.s + (c + 4u) / row.group);
  r.b[1] = ldg<float>(row.b + (c + 4u) / row.group);
}

template <int RD>
__device__ __forceinline__ void load_raw8(const uint8_t* row, uint32_t c, Raw8<RD>& r) {
  if constexpr (RD == OSM_META_F32) {
    r.v[0] = ldg16(row + static_cast<size_t>(c) * 4u);
    r.v[1] = ldg16(row + static_cast<size_t>(c) * 4u + 16u);
  } else {
    r.v[0] = ldg16(row + static_cast<size_t>(c) * 2u);
  }
}

template <int RD>
__device__ __forceinline__ float raw8_get(const Raw8<RD>& r, int j) {
  if constexpr (RD == OSM_ROUTER_AFFINE_Q8) {
    const uint32_t w = j < 4 ? r.q.x : r.q.y;
    const float q = static_cast<float>((w >> (8 * (j % 4))) & 0xFFu);
    return dequant_q8(r.s[j / 4], q, r.b[j / 4]);
  } else if constexpr (RD == OSM_META_F32) {
    const uint4& q = r.v[j / 4];
    const uint32_t w = (j % 4 == 0) ? q.x : (j % 4 == 1) ? q.y : (j % 4 == 2) ? q.z : q.w;
    return __uint_as_float(w);
  } else {
    const uint4& q = r.v[0];
    const uint32_t w = (j / 2 == 0) ? q.x : (j / 2 == 1) ? q.y : (j / 2 == 2) ? q.z : q.w;
    const uint32_t bits = (j % 2 == 0) ? (w & 0xFFFFu) : (w >> 16);
    if constexpr (RD == OSM_META_BF16)
      return bf16_to_f32(bits);
    else
      return f16_to_f32(bits);
  }
}

// ---------------------------------------------------------------------------
// Routing that is the reference's, bit for bit.
//
// The reference ranks experts by softmax probability, the lower id first
// among equal probabilities (reference_ops.cpp:130-212), over logits that it
// sums sequentially in fp32 (reference_ops.cpp:85-93) on the input that
// rms_norm_inplace normalised (reference_ops.cpp:96-128). The device sums in
// other orders, so its logits differ from the reference's by rounding. Every
// device logit l therefore comes with a bound b >= |l - L|, L the
// reference's logit (route_block, the router GEMM), and the selection ranks
// on the device logits only where the bounds prove the reference's order:
//
//  - adjacent picks i, i+1: l_i - l_{i+1} > s (b_i + b_{i+1}), plus kappa
//    when the lower logit has the lower id;
//  - every expert e outside the picks: l_e + s b_e + kappa(e) < l_k - s b_k;
//  - the k-th pick within 80 of the largest logit.
//
// s = 1 + 2^-9 covers a common factor 1 + eta by which the device's
// RMS-normalised input can differ from the reference's (eta <= n u for a
// width n <= 8192 and u = 2^-24, from the two sums of squares) and the
// rounding of the bounds themselves. kappa = 2^-20 + 2^-23 (m - l + 1), m
// the largest logit: a gap in L larger than that keeps the two
// probabilities exp(fl(L - m)) / S at least four ulps apart whatever the
// rounding of the subtraction, the exp (within one ulp) and the division, so
// the reference's probabilities cannot tie where the device's logits do not.
// Within 80 of m no exp underflows.
//
// Otherwise (a near tie, equal device logits, or a missing bound) the
// selection takes the exact path: every expert whose interval can reach the
// picks' lowest lower bound is recomputed in the reference's order, and the
// candidates are ranked by the reference's numerator e = exp(fl(L - m)),
// with the host libm's own bits (osm_libm_expf), ties to the lower id. The
// reference ranks by p = fl(e / S) instead, S its sum of every expert's e
// in id order; p orders as e does, except that two different e can round to
// one p, and then the lower id wins. That can only happen for e_a > e_c
// within 2^-22 e_a (one ulp of the quotient, or 2^-138 where the quotient is
// subnormal). When such a pair is adjacent among the first k + 1 candidates
// with the higher id first, and whenever the k-th candidate is more than 80
// below m (exps near or at underflow), every expert is recomputed: S is then
// summed as the reference sums it and the experts are ranked by fl(e / S),
// ties to the lower id, which is the reference's ranking itself.
//
// The probabilities of the picks (their weights) come from the device
// logits in both paths: exp(l - max) / sum over every expert.
constexpr uint32_t kSelThreads = 256;
constexpr uint32_t kSelWaves = kSelThreads / kWave;
constexpr float kBoundSlack = 1.0f + 0x1p-9f;
constexpr float kUnderflowGap = 80.0f;

// The exact path recomputes logits in the reference's order. The additions
// of one logit form a chain that cannot be split; everything else runs
// beside it. Wavefronts 1-3 produce: per chunk of kExactCols columns, thread
// (candidate r, segment s) loads 16 router elements of candidate r and the
// matching inputs and writes the rounded products w * x into one of two LDS
// buffers. Wavefront 0 adds: lane r adds candidate r's products of the
// previous chunk in column order while the producers fill the other buffer,
// one barrier per chunk.
constexpr uint32_t kExactRows = 16;  // candidates per pass
constexpr uint32_t kExactSegs = (kSelThreads - kWave) / kExactRows;  // producer threads per candidate
constexpr uint32_t kExactCols = kExactSegs * 16u;                     // 192 columns per chunk
constexpr uint32_t kExactStride = kExactCols + 4u;  // LDS row stride: 16-byte aligned rows, adders' reads in distinct banks

// Bins of the device ranking's distance histogram (rank_device).
constexpr uint32_t kHistBins = 64;
constexpr float kHistSpan = 256.0f;

__device__ __forceinline__ float tie_margin(float mx, float l) { return 0x1p-20f + 0x1p-23f * (mx - l + 1.0f); }

// Result of one token's selection, in LDS: ids, device logits and bounds and
// probabilities in pick order, the blob, device logit and bound of every
// expert, and the workgroup's scratch.
template <int PER>
struct Selection {
  uint32_t id[OSMD_MAX_TOP_K];
  float lg[OSMD_MAX_TOP_K];
  float bd[OSMD_MAX_TOP_K];
  float p[OSMD_MAX_TOP_K];
  const uint8_t* blob[kSelThreads * PER];
  float val[kSelThreads * PER];   // device logit of every expert
  float aux[kSelThreads * PER];   // its bound; on the exact path, its e = exp(fl(L - m)) (-1: no candidate)
  float ex[kSelThreads * PER];    // exact path: the reference's logit of a candidate
  float red[3][kSelWaves];
  uint64_t cand[kWave];                       // (key << 32) | ~id of the ranked candidates
  float clg[kWave], cbd[kWave];               // their device logits and bounds
  uint32_t hist[kHistBins];                   // experts per bin of distance from the largest logit
  uint32_t fid[OSMD_MAX_TOP_K + 1];           // exact path: candidates by rank
  float scal[3];                              // exact path: threshold, RMS scale, softmax sum
  uint32_t nneartie, ncand, thr, flags, wcount[kSelWaves];  // nneartie: near ties sent to the full recompute
  uint32_t again;                             // exact path: recompute every expert
  uint16_t cl[kSelThreads * PER];             // exact path: candidate list
  __attribute__((aligned(16))) float xe[2][kExactCols];  // exact path: the inputs of two chunks
  __attribute__((aligned(16))) float prod[2][kExactRows][kExactStride];  // exact path: rounded products of two chunks
};
static_assert(kExactRows * kExactSegs + kWave == kSelThreads, "exact-path chunk mapping");
static_assert(kSelWaves * OSMD_MAX_TOP_K <= kWave, "the fallback's candidates fit the candidate list");

__device__ __forceinline__ void sort_step(uint32_t* k, uint32_t* n, int a, int b) {
  // Descending on (k, n): swap when (k[b], n[b]) > (k[a], n[a]).
  const uint64_t ka = (static_cast<uint64_t>(k[a]) << 32) | n[a];
  const uint64_t kb = (static_cast<uint64_t>(k[b]) << 32) | n[b];
  const bool swap = kb > ka;
  const uint32_t k0 = k[a], n0 = n[a];
  k[a] = swap ? k[b] : k0;
  n[a] = swap ? n[b] : n0;
  k[b] = swap ? k0 : k[b];
  n[b] = swap ? n0 : n[b];
}

template <int PER>
__device__ __forceinline__ void sort_lane(uint32_t* k, uint32_t* n) {
  // Odd-even transposition (PER is 2 or 4).
#pragma unroll
  for (int round = 0; round < PER; ++round) {
#pragma unroll
    for (int j = round & 1; j + 1 < PER; j += 2) sort_step(k, n, j, j + 1);
  }
}

// acc + v[0] + v[1] + ... + v[n-1] in order, each addition rounded to fp32,
// v in LDS (16-byte aligned), n a multiple of 8 and the same in every lane.
// Values go through two register batches of 4 CB: the next batch's reads are
// issued before the current batch's additions, so the chain of additions,
// which cannot be shortened, is what is waited on.
__device__ __forceinline__ float chain_add4(float4 q, float acc) {
#pragma clang fp contract(off)
  acc = acc + q.x;
  acc = acc + q.y;
  acc = acc + q.z;
  acc = acc + q.w;
  return acc;
}
// CB: float4 per batch (8, or 16 where registers allow: the selection
// kernel, which runs one workgroup per token).
template <int CB>
__device__ __forceinline__ void chain_load(const float4* p, float4 (&r)[CB]) {
#pragma unroll
  for (int j = 0; j < CB; ++j) r[j] = p[j];
}
template <int CB>
__device__ __forceinline__ float chain_batch(const float4 (&r)[CB], float acc) {
#pragma unroll
  for (int j = 0; j < CB; ++j) acc = chain_add4(r[j], acc);
  return acc;
}
template <int CB = 8>
__device__ __forceinline__ float chain_sum(const float* v, uint32_t n, float acc) {
  const float4* v4 = reinterpret_cast<const float4*>(v);
  const uint32_t nb = n / (4u * CB);
  float4 a[CB], b[CB];
  if (nb > 0u) chain_load<CB>(v4, a);
  for (uint32_t k = 0; k < nb; k += 2u) {
    const bool b_used = k + 1u < nb;
    if (b_used) chain_load<CB>(v4 + (k + 1u) * CB, b);
    __builtin_amdgcn_sched_barrier(0);
    acc = chain_batch<CB>(a, acc);
    if (!b_used) break;
    if (k + 2u < nb) chain_load<CB>(v4 + (k + 2u) * CB, a);
    __builtin_amdgcn_sched_barrier(0);
    acc = chain_batch<CB>(b, acc);
  }
  for (uint32_t i = nb * 4u * CB; i < n; i += 8u) {
    acc = chain_add4(v4[i / 4u], acc);
    acc = chain_add4(v4[i / 4u + 1u], acc);
  }
  return acc;
}

// x[c] of the router's input, as the reference reads it (0 past the row).
__device__ __forceinline__ float load_x1(const RouteView& rv, uint32_t t, uint32_t c) {
  if (c >= rv.hidden) return 0.0f;
  const size_t o = static_cast<size_t>(t) * rv.hidden + c;
  return rv.x_bf16 ? bf16_to_f32(ldg<uint16_t>(static_cast<const uint16_t*>(rv.x) + o))
                   : ldg<float>(static_cast<const float*>(rv.x) + o);
}
// The same element as loaded (fp32 bits, or a bf16 in the low half), for
// loads issued steps ahead of their use: widening a bf16 right after its
// load would wait for the load there.
__device__ __forceinline__ uint32_t load_x1_bits(const RouteView& rv, uint32_t t, uint32_t c) {
  if (c >= rv.hidden) return 0u;
  const size_t o = static_cast<size_t>(t) * rv.hidden + c;
  return rv.x_bf16 ? static_cast<uint32_t>(ldg<uint16_t>(static_cast<const uint16_t*>(rv.x) + o))
                   : ldg<uint32_t>(static_cast<const float*>(rv.x) + o);
}
__device__ __forceinline__ float x1_value(const RouteView& rv, uint32_t bits) {
  return rv.x_bf16 ? bf16_to_f32(bits) : __uint_as_float(bits);
}

// The reference's RMSNorm scale of token t: the squares summed in order,
// then 1 / sqrt(sum / D + eps), each operation rounded to fp32
// (reference_ops.cpp:113-121). Every thread calls it; x is staged in LDS
// 2 * kExactRows * kExactStride columns at a time for thread 0's chain.
template <int PER>
__device__ float exact_rms_scale(const RouteView& rv, uint32_t t, Selection<PER>& out) {
#pragma clang fp contract(off)
  constexpr uint32_t kCols = 2u * kExactRows * kExactStride;
  float* stage = &out.prod[0][0][0];
  float ss = 0.0f;
  for (uint32_t c0 = 0; c0 < rv.hidden; c0 += kCols) {
    // The squares, each rounded as the reference rounds v * v, in parallel;
    // then thread 0 adds them in order.
    for (uint32_t i = threadIdx.x; i < kCols; i += kSelThreads) {
      const float v = load_x1(rv, t, c0 + i);
      stage[i] = v * v;
    }
    __syncthreads();
    if (threadIdx.x == 0) ss = chain_sum(stage, rv.hidden - c0 < kCols ? rv.hidden - c0 : kCols, ss);
    __syncthreads();
  }
  if (threadIdx.x == 0)
    out.scal[1] = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, static_cast<float>(rv.hidden)) + rv.rms_eps));
  __syncthreads();
  return out.scal[1];
}

// The reference's logits of candidates out.cl[first .. first + nr), nr <=
// kExactRows, for token t: acc + w[c] * x[c] for c = 0 .. D-1, every product
// and sum rounded to fp32 (reference_ops.cpp:85-93), on x scaled as
// rms_norm_inplace does, x * (scale * weight) (reference_ops.cpp:123-126).
// Every thread calls it; candidate r's logit lands in out.ex.
template <int RD, int PER>
__device__ void exact_logits_rd(const RouteView& rv, uint32_t t, Selection<PER>& out, uint32_t first, uint32_t nr,
                                float scale) {
#pragma clang fp contract(off)
  const uint32_t D = rv.hidden, tid = threadIdx.x;
  // Producer (candidate r, columns seg .. seg + 15 of each chunk); the 16
  // candidates of one segment sit in 16 lanes, so their LDS writes land in
  // distinct banks. Producer ptid also stages input column ptid of a chunk.
  const bool producer = tid >= kWave;
  const uint32_t ptid = producer ? tid - kWave : 0u;
  const uint32_t r = ptid % kExactRows, seg = (ptid / kExactRows) * 16u;
  const bool active = producer && r < nr;
  const uint32_t e = r < nr ? out.cl[first + r] : out.cl[first];
  Q8Row qr{};
  const uint8_t* row = nullptr;
  if constexpr (RD == OSM_ROUTER_AFFINE_Q8)
    qr = q8_row(rv.router, rv.expert_count, e, D, rv.router_group);
  else
    row = static_cast<const uint8_t*>(rv.router) + static_cast<size_t>(e) * D * (RD == OSM_META_F32 ? 4u : 2u);
  Raw8<RD> w0{}, w1{};
  auto fetch_w = [&](uint32_t c0) {
    const uint32_t c = c0 + seg;
    if (!active) return;
    if (c < D) {
      if constexpr (RD == OSM_ROUTER_AFFINE_Q8) load_q8x8(qr, c, w0); else load_raw8<RD>(row, c, w0);
    }
    if (c + 8u < D) {
      if constexpr (RD == OSM_ROUTER_AFFINE_Q8) load_q8x8(qr, c + 8u, w1); else load_raw8<RD>(row, c + 8u, w1);
    }
  };
  uint32_t xb = 0u;
  float nwv = 1.0f;
  auto fetch_x = [&](uint32_t c0) {
    if (!producer) return;
    const uint32_t c = c0 + ptid;
    xb = load_x1_bits(rv, t, c);
    nwv = (rv.rms && c < D) ? ldg<float>(rv.norm_weight + c) : 1.0f;
  };
  auto stage_x = [&](uint32_t buf) {
    if (!producer) return;
    const float xv = x1_value(rv, xb);
    out.xe[buf][ptid] = rv.rms ? xv * (scale * nwv) : xv;
  };
  // Step k: the producers write chunk k's products (router elements loaded
  // in step k - 1, inputs staged in step k - 1), stage chunk k + 1's inputs
  // (loaded in step k - 1) and issue the loads of chunk k + 1's router
  // elements and chunk k + 2's inputs; lane r of wavefront 0 adds chunk
  // k - 1. Products past D are written and never added. (Loading the router
  // elements two steps ahead measured no faster: a step is the addition
  // chain plus the barrier.)
  const uint32_t nchunks = (D + kExactCols - 1u) / kExactCols;
  fetch_x(0);
  fetch_w(0);
  stage_x(0);
  fetch_x(kExactCols);
  __syncthreads();
  float acc = 0.0f;
  // The adders' wavefront issues first on its SIMD while it adds (as in
  // exact_logits_deep).
  const bool adder_wave = tid < kWave;
  if (adder_wave) __builtin_amdgcn_s_setprio(2);
  for (uint32_t k = 0; k <= nchunks; ++k) {
    if (active && k < nchunks) {
      float4* dst = reinterpret_cast<float4*>(&out.prod[k & 1u][r][seg]);
      const float4* xs = reinterpret_cast<const float4*>(&out.xe[k & 1u][seg]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 x4 = xs[j];
        const Raw8<RD>& w = j < 2 ? w0 : w1;
        const int o = 4 * (j % 2);
        dst[j] = make_float4(raw8_get<RD>(w, o) * x4.x, raw8_get<RD>(w, o + 1) * x4.y,
                             raw8_get<RD>(w, o + 2) * x4.z, raw8_get<RD>(w, o + 3) * x4.w);
      }
    }
    if (k + 1u < nchunks) {
      stage_x((k + 1u) & 1u);
      fetch_w((k + 1u) * kExactCols);
      fetch_x((k + 2u) * kExactCols);
    }
    if (tid < nr && k > 0u) {
      const uint32_t c0 = (k - 1u) * kExactCols;
      acc = chain_sum(out.prod[(k - 1u) & 1u][tid], D - c0 < kExactCols ? D - c0 : kExactCols, acc);
    }
    __syncthreads();
  }
  if (adder_wave) __builtin_amdgcn_s_setprio(0);
  if (tid < nr) out.ex[out.cl[first + tid]] = acc;
}

// The same logits with the loads two steps ahead: router elements in two
// register sets used on alternate steps, inputs loaded two steps before they
// are staged, and additions in batches of 64. For the selection kernel (one
// workgroup per token, registers to spare): a step is then the addition chain
// rather than the producers' wait for their loads.
template <int RD, int PER>
__device__ void exact_logits_deep(const RouteView& rv, uint32_t t, Selection<PER>& out, uint32_t first, uint32_t nr,
                                  float scale) {
#pragma clang fp contract(off)
  const uint32_t D = rv.hidden, tid = threadIdx.x;
  const bool producer = tid >= kWave;
  const uint32_t ptid = producer ? tid - kWave : 0u;
  const uint32_t r = ptid % kExactRows, seg = (ptid / kExactRows) * 16u;
  const bool active = producer && r < nr;
  const uint32_t e = r < nr ? out.cl[first + r] : out.cl[first];
  Q8Row qr{};
  const uint8_t* row = nullptr;
  if constexpr (RD == OSM_ROUTER_AFFINE_Q8)
    qr = q8_row(rv.router, rv.expert_count, e, D, rv.router_group);
  else
    row = static_cast<const uint8_t*>(rv.router) + static_cast<size_t>(e) * D * (RD == OSM_META_F32 ? 4u : 2u);
  struct W16 {
    Raw8<RD> lo, hi;
  };
  struct X1 {
    uint32_t x;  // as loaded (load_x1_bits)
    float nw;
  };
  auto fetch_w = [&](W16& w, uint32_t chunk) {
    const uint32_t c = chunk * kExactCols + seg;
    if (!active) return;
    if (c < D) {
      if constexpr (RD == OSM_ROUTER_AFFINE_Q8) load_q8x8(qr, c, w.lo); else load_raw8<RD>(row, c, w.lo);
    }
    if (c + 8u < D) {
      if constexpr (RD == OSM_ROUTER_AFFINE_Q8) load_q8x8(qr, c + 8u, w.hi); else load_raw8<RD>(row, c + 8u, w.hi);
    }
  };
  auto fetch_x = [&](X1& v, uint32_t chunk) {
    if (!producer) return;
    const uint32_t c = chunk * kExactCols + ptid;
    v.x = load_x1_bits(rv, t, c);
    v.nw = (rv.rms && c < D) ? ldg<float>(rv.norm_weight + c) : 1.0f;
  };
  auto stage_x = [&](const X1& v, uint32_t buf) {
    if (!producer) return;
    const float xv = x1_value(rv, v.x);
    out.xe[buf][ptid] = rv.rms ? xv * (scale * v.nw) : xv;
  };
  const uint32_t nchunks = (D + kExactCols - 1u) / kExactCols;
  float acc = 0.0f;
  // Step k: products of chunk k from w (loaded in step k - 2), w refilled
  // with chunk k + 2; chunk k + 1's inputs staged from xs (loaded in step
  // k - 2), xs refilled with chunk k + 3; lane r of wavefront 0 adds chunk
  // k - 1.
  auto step = [&](uint32_t k, W16& w, X1& xs) {
    if (active && k < nchunks) {
      float4* dst = reinterpret_cast<float4*>(&out.prod[k & 1u][r][seg]);
      const float4* xe = reinterpret_cast<const float4*>(&out.xe[k & 1u][seg]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 x4 = xe[j];
        const Raw8<RD>& h = j < 2 ? w.lo : w.hi;
        const int o = 4 * (j % 2);
        dst[j] = make_float4(raw8_get<RD>(h, o) * x4.x, raw8_get<RD>(h, o + 1) * x4.y,
                             raw8_get<RD>(h, o + 2) * x4.z, raw8_get<RD>(h, o + 3) * x4.w);
      }
      if (k + 2u < nchunks) fetch_w(w, k + 2u);
    }
    if (k + 1u < nchunks) {
      stage_x(xs, (k + 1u) & 1u);
      if (k + 3u < nchunks) fetch_x(xs, k + 3u);
    }
    if (tid < nr && k > 0u) {
      const uint32_t c0 = (k - 1u) * kExactCols;
      acc = chain_sum<16>(out.prod[(k - 1u) & 1u][tid], D - c0 < kExactCols ? D - c0 : kExactCols, acc);
    }
    __syncthreads();
  };
  W16 wa{}, wb{};
  X1 xa{}, xb{};
  fetch_x(xa, 0);
  fetch_w(wa, 0);
  if (nchunks > 1u) fetch_w(wb, 1);
  stage_x(xa, 0);
  if (nchunks > 1u) fetch_x(xb, 1);
  if (nchunks > 2u) fetch_x(xa, 2);
  __syncthreads();
  // The adders' wavefront issues first on its SIMD while it adds: each
  // addition waits for the one before it, and a wavefront of another
  // workgroup sharing the SIMD would otherwise take the slots in between.
  const bool adder_wave = tid < kWave;
  if (adder_wave) __builtin_amdgcn_s_setprio(2);
  // Even steps stage odd chunks from xb, odd steps even chunks from xa.
  for (uint32_t k = 0; k <= nchunks; k += 2u) {
    step(k, wa, xb);
    if (k + 1u <= nchunks) step(k + 1u, wb, xa);
  }
  if (adder_wave) __builtin_amdgcn_s_setprio(0);
  if (tid < nr) out.ex[out.cl[first + tid]] = acc;
}

template <int PER, bool DEEP>
__device__ void exact_logits(const RouteView& rv, uint32_t t, Selection<PER>& out, uint32_t first, uint32_t nr,
                             float scale) {
  switch (rv.router_dtype) {
    case OSM_META_F32:
      if constexpr (DEEP) exact_logits_deep<OSM_META_F32>(rv, t, out, first, nr, scale);
      else exact_logits_rd<OSM_META_F32>(rv, t, out, first, nr, scale);
      break;
    case OSM_META_F16:
      if constexpr (DEEP) exact_logits_deep<OSM_META_F16>(rv, t, out, first, nr, scale);
      else exact_logits_rd<OSM_META_F16>(rv, t, out, first, nr, scale);
      break;
    case OSM_ROUTER_AFFINE_Q8:
      if constexpr (DEEP) exact_logits_deep<OSM_ROUTER_AFFINE_Q8>(rv, t, out, first, nr, scale);
      else exact_logits_rd<OSM_ROUTER_AFFINE_Q8>(rv, t, out, first, nr, scale);
      break;
    default:
      if constexpr (DEEP) exact_logits_deep<OSM_META_BF16>(rv, t, out, first, nr, scale);
      else exact_logits_rd<OSM_META_BF16>(rv, t, out, first, nr, scale);
      break;
  }
}

// The exact path (every thread of the workgroup; out.id/lg/bd hold the
// device ranking). Rewrites out.id and out.lg; returns whether every expert
// was recomputed. out.nneartie gets the adjacent pairs that sent it to the
// full recompute (near ties with the higher id first).
template <int PER, bool DEEP>
__device__ bool select_exact(const RouteView& rv, uint32_t t, const float (&l)[PER], const float (&b)[PER],
                             Selection<PER>& out, float mx) {
  const uint32_t E = rv.expert_count, k = rv.top_k;
  const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const uint32_t base = tid * PER;
  // The picks' lowest lower bound, by every thread from the ranking in LDS
  // (stable since the certificate's barrier).
  float th = INFINITY;
  for (uint32_t i = 0; i < k; ++i) th = fminf(th, out.lg[i] - kBoundSlack * out.bd[i]);
  const float scale = rv.rms ? exact_rms_scale<PER>(rv, t, out) : 1.0f;
  bool full = false;
  float m = -INFINITY;
  for (;;) {
    // Candidates: a compact list in out.cl, wavefront by wavefront.
    bool member[PER];
    uint32_t mine = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const uint32_t e = base + j;
      // A bound that is not finite admits the expert (NaN comparisons fail).
      member[j] = e < E && (full || !(l[j] + kBoundSlack * b[j] + tie_margin(mx, l[j]) < th));
      mine += member[j] ? 1u : 0u;
    }
    const float incl = wave_incl_scan(static_cast<float>(mine));  // small integers: exact
    if (lane == kWave - 1) out.wcount[wave] = static_cast<uint32_t>(incl);
    __syncthreads();
    uint32_t pos = static_cast<uint32_t>(incl) - mine;
    for (uint32_t w = 0; w < wave; ++w) pos += out.wcount[w];
    const uint32_t nc = out.wcount[0] + out.wcount[1] + out.wcount[2] + out.wcount[3];
    uint32_t cpos[PER];  // list position of each member
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      cpos[j] = pos;
      if (member[j]) out.cl[pos++] = static_cast<uint16_t>(base + j);
    }
    __syncthreads();
    for (uint32_t first = 0; first < nc; first += kExactRows)
      exact_logits<PER, DEEP>(rv, t, out, first, nc - first < kExactRows ? nc - first : kExactRows, scale);
    __syncthreads();
    if (!full && nc <= kWave) {
      // Up to 64 candidates: wavefront 0 ranks them in registers (lane i
      // holds candidate i of the list) with the keys, ranks, near-tie and
      // underflow tests of the general form below, and one barrier instead
      // of five.
      if (tid < kWave) {
        const bool act = lane < nc;
        const uint32_t e = act ? out.cl[lane] : 0u;
        const float x = act ? out.ex[e] : -INFINITY;
        const float mm = wave_max(x);
        const float key = act ? osm_libm_expf(x - mm) : -1.0f;
        if (act) out.aux[e] = key;
        uint32_t rk = 0u;
        for (uint32_t i = 0; i < nc; ++i) {
          const float w = readlane_f(key, static_cast<int>(i));
          const uint32_t ei = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(e), static_cast<int>(i)));
          rk += (w > key || (w == key && ei < e)) ? 1u : 0u;
        }
        if (act && rk <= k) out.fid[rk] = e;
        // This candidate (rank rk) against the one ranked rk + 1.
        const uint32_t n = nc < k + 1u ? nc : k + 1u;
        float ec = 0.0f;
        uint32_t c = 0u;
        for (uint32_t i = 0; i < nc; ++i) {
          const uint32_t ri = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(rk), static_cast<int>(i)));
          if (ri == rk + 1u) {
            ec = readlane_f(key, static_cast<int>(i));
            c = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(e), static_cast<int>(i)));
          }
        }
        const bool near = act && rk + 1u < n && e > c && key != ec && key - ec <= 0x1p-22f * key + 0x1p-138f;
        const uint64_t nb = __ballot(near);
        const uint64_t kb = __ballot(act && rk == k - 1u);  // one lane: nc >= k (the picks are candidates)
        const float xk = readlane_f(x, static_cast<int>(__builtin_ctzll(kb)));
        if (lane == 0u) {
          out.nneartie = static_cast<uint32_t>(__popcll(nb));
          out.again = (nb != 0u || !(xk - mm >= -kUnderflowGap)) ? 1u : 0u;
        }
      }
      __syncthreads();
      if (out.again == 0u) {
        if (tid == 0) out.ncand = nc;
        break;
      }
      full = true;
      __syncthreads();
      continue;
    }
    float lm = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (member[j]) lm = fmaxf(lm, out.ex[base + j]);
    lm = wave_max(lm);
    if (lane == 0) out.red[0][wave] = lm;
    __syncthreads();
    m = fmaxf(fmaxf(out.red[0][0], out.red[0][1]), fmaxf(out.red[0][2], out.red[0][3]));
    // The reference's numerator e = exp(fl(L - m)) (reference_ops.cpp:141-145)
    // with the host libm's bits, by expert in out.aux.
    float key[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      key[j] = member[j] ? osm_libm_expf(out.ex[base + j] - m) : -1.0f;
      if (base + j < E) out.aux[base + j] = key[j];
    }
    if (full) {
      // Every expert is a member: the reference's probabilities, S summed in
      // id order with each addition rounded (reference_ops.cpp:140-144), then
      // p = fl(e / S) (:149-151), which rank the experts.
      __syncthreads();
      if (tid == 0) {
#pragma clang fp contract(off)
        const uint32_t n8 = E & ~7u;
        float s = chain_sum(out.aux, n8, 0.0f);
        for (uint32_t e = n8; e < E; ++e) s = s + out.aux[e];
        out.scal[2] = s;
      }
      __syncthreads();
      const float S = out.scal[2];
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (member[j]) key[j] = __fdiv_rn(key[j], S);
    }
    // Ranking keys in list order in ckey (the products' buffer is free now),
    // so that the ranking reads them without an indirection.
    float* ckey = &out.prod[0][0][0];
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (member[j]) ckey[cpos[j]] = key[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      if (!member[j]) continue;
      const uint32_t e = base + j;
      const float v = key[j];
      uint32_t rk = 0;
#pragma unroll 4
      for (uint32_t i = 0; i < nc; ++i) {
        const float w = ckey[i];
        rk += (w > v || (w == v && out.cl[i] < e)) ? 1u : 0u;
      }
      if (rk <= k) out.fid[rk] = e;
    }
    __syncthreads();
    if (full) {
      if (tid == 0) out.ncand = nc;
      break;
    }
    // Adjacent candidates among the first k + 1 (there are at least k: the
    // device's picks are candidates), one pair per lane: a pair ranked with
    // the higher id first whose e are close enough for their quotients by S
    // to round to one p, where the reference would put the lower id first.
    if (tid < kWave) {
      const uint32_t n = nc < k + 1u ? nc : k + 1u;
      bool near = false;
      if (lane + 1u < n) {
        const uint32_t a = out.fid[lane], c = out.fid[lane + 1u];
        const float ea = out.aux[a], ec = out.aux[c];  // ea >= ec (ranked)
        near = a > c && ea != ec && ea - ec <= 0x1p-22f * ea + 0x1p-138f;
      }
      const uint32_t count = static_cast<uint32_t>(__popcll(__ballot(near)));
      if (lane == 0) out.nneartie = count;
    }
    __syncthreads();
    // Such a pair, or exps near underflow beyond 80 below m: rank every
    // expert by the reference's probabilities.
    const bool again = out.nneartie != 0u || !(out.ex[out.fid[k - 1]] - m >= -kUnderflowGap);
    if (!again) {
      if (tid == 0) out.ncand = nc;
      break;
    }
    full = true;
    __syncthreads();
  }
  if (tid < k) {
    const uint32_t id = out.fid[tid];
    out.id[tid] = id;
    out.lg[tid] = out.val[id];
  }
  __syncthreads();
  return full;
}

// Maximum and minimum over the wavefront, the two reductions interleaved.
__device__ __forceinline__ void wave_max_min(float& mx, float& mn) {
  float a = mx, b = mn;
  a = fmaxf(a, dpp<kDppXor1>(a, a));
  b = fminf(b, dpp<kDppXor1>(b, b));
  a = fmaxf(a, dpp<kDppXor2>(a, a));
  b = fminf(b, dpp<kDppXor2>(b, b));
  a = fmaxf(a, dpp<kDppRowHalfMirror>(a, a));
  b = fminf(b, dpp<kDppRowHalfMirror>(b, b));
  a = fmaxf(a, dpp<kDppRowMirror>(a, a));
  b = fminf(b, dpp<kDppRowMirror>(b, b));
  a = fmaxf(a, dpp<kDppRowBcast15, 0xA>(a, a));
  b = fminf(b, dpp<kDppRowBcast15, 0xA>(b, b));
  a = fmaxf(a, dpp<kDppRowBcast31, 0xC>(a, a));
  b = fminf(b, dpp<kDppRowBcast31, 0xC>(b, b));
  mx = readlane_f(a, 63);
  mn = readlane_f(b, 63);
}

// The device ranking: the k largest (logit, lower id) keys of the workgroup's
// experts into out.id / out.lg / out.bd. Distances from the largest logit
// are bucketed, d = fl(fl(mx - l) * inv) with inv = kHistSpan / (mx - mn),
// into kHistBins bins (the last, which nothing counts, takes everything
// beyond), and the first bin at which the count reaches k bounds the
// candidates: d is monotone in l, so every expert of a later bin has a
// smaller logit than every candidate. At most kWave candidates are ranked
// by one wavefront; otherwise (all logits equal, a non-finite range, a
// distribution too skewed for the bins) each wavefront extracts its own top
// k and wavefront 0 ranks those.
template <int PER>
__device__ __forceinline__ void rank_device(const RouteView& rv, const float (&l)[PER], const float (&b)[PER],
                                            Selection<PER>& out, float mx, float mn) {
  const uint32_t E = rv.expert_count;
  const uint32_t k = rv.top_k;
  const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const uint32_t base = tid * PER;
  const float range = mx - mn;
  const bool binned = range > 0.0f && range < INFINITY;  // workgroup-uniform
  uint32_t bin[PER] = {};
  if (binned) {
    const float inv = kHistSpan / range;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const float d = (mx - l[j]) * inv;  // NaN (a NaN logit) fails the test: last bin
      bin[j] = d < static_cast<float>(kHistBins - 1u) ? static_cast<uint32_t>(d) : kHistBins - 1u;
      if (base + j < E && bin[j] < kHistBins - 1u) atomicAdd(&out.hist[bin[j]], 1u);
    }
  }
  __syncthreads();
  if (wave == 0) {
    const float incl = wave_incl_scan(static_cast<float>(out.hist[lane]));  // counts <= 1024: exact
    const uint64_t reached = __ballot(incl >= static_cast<float>(k));
    const int first = reached ? __ffsll(static_cast<long long>(reached)) - 1 : kWave - 1;
    const float count = readlane_f(incl, first);
    if (lane == 0) {
      out.thr = (binned && reached && count <= static_cast<float>(kWave)) ? static_cast<uint32_t>(first) : ~0u;
      out.ncand = 0;
    }
  }
  __syncthreads();
  const uint32_t thr = out.thr;
  if (thr != ~0u) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const uint32_t e = base + j;
      if (e < E && bin[j] <= thr) {
        const uint32_t pos = atomicAdd(&out.ncand, 1u);
        out.cand[pos] = (static_cast<uint64_t>(ordered_key(l[j])) << 32) | ~e;
        out.clg[pos] = l[j];
        out.cbd[pos] = b[j];
      }
    }
  } else {
    // Fallback: each wavefront's top k by (logit, lower id), one pop per
    // round, lane r keeping round r's result.
    uint32_t key[PER], nid[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      key[j] = base + j < E ? ordered_key(l[j]) : 0u;  // above 0 for every real logit
      nid[j] = ~(base + j);
    }
    sort_lane<PER>(key, nid);
    uint32_t rk = 0u, ri = 0u;
#pragma unroll 1
    for (uint32_t r = 0; r < k; ++r) {
      const uint32_t mk = wave_max_u32(key[0]);
      const int wl = __ffsll(__ballot(key[0] == mk)) - 1;  // never empty: mk is some lane's key
      const uint32_t sid = ~static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(nid[0]), wl));
      rk = lane == r ? mk : rk;
      ri = lane == r ? sid : ri;
      const bool won = static_cast<int>(lane) == wl;  // pop the head
#pragma unroll
      for (int j = 0; j + 1 < PER; ++j) {
        key[j] = won ? key[j + 1] : key[j];
        nid[j] = won ? nid[j + 1] : nid[j];
      }
      key[PER - 1] = won ? 0u : key[PER - 1];
      nid[PER - 1] = won ? 0u : nid[PER - 1];
    }
    if (lane < k) {
      const uint32_t id = ri < E ? ri : E - 1u;  // key-0 entries (fewer than k experts here) stay in the table
      out.cand[wave * k + lane] = (static_cast<uint64_t>(rk) << 32) | ~ri;
      out.clg[wave * k + lane] = out.val[id];
      out.cbd[wave * k + lane] = out.aux[id];
    }
    if (tid == 0) out.ncand = kSelWaves * k;
  }
  __syncthreads();
  // Wavefront 0: each lane ranks one candidate against all of them (LDS
  // broadcast reads); the k best write their place. Fallback candidates of
  // key 0 (fewer than k experts in a wavefront) always have k real ones
  // above them.
  if (wave == 0) {
    const uint32_t nc = out.ncand;
    const uint64_t mine = lane < nc ? out.cand[lane] : 0u;
    uint32_t rank = 0;
#pragma unroll 4
    for (uint32_t c = 0; c < nc; ++c) rank += out.cand[c] > mine ? 1u : 0u;
    if (lane < nc && rank < k) {
      const uint32_t id0 = ~static_cast<uint32_t>(mine);
      out.id[rank] = id0 < E ? id0 : E - 1u;  // a table lookup always stays in the table
      out.lg[rank] = out.clg[lane];
      out.bd[rank] = out.cbd[lane];
    }
  }
  __syncthreads();
}

// Selection from this thread's device logits l[j] and bounds b[j] of experts
// tid*PER + j (entries past E are ignored) and their table pointers. Every
// thread of the workgroup calls it; it ends with a barrier, after which
// out.id and out.flags are complete, and out.p when need_p (workgroup-
// uniform; the softmax denominator and the probabilities are skipped
// otherwise, for workgroups that only read their slot's expert). `count`:
// add this selection to the routing counters now (otherwise
// count_selection does it later).
template <int PER, bool DEEP = false>
__device__ __forceinline__ void select_values(const RouteView& rv, uint32_t t, const float (&l)[PER],
                                              const float (&b)[PER], const uint8_t* const (&tab)[PER],
                                              Selection<PER>& out, bool count, bool need_p = true) {
  const uint32_t E = rv.expert_count;
  const uint32_t k = rv.top_k;
  const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const uint32_t base = tid * PER;
  float mx = -INFINITY, mn = INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (base + j < E) {
      out.blob[base + j] = tab[j];
      out.val[base + j] = l[j];
      out.aux[base + j] = b[j];
      mx = fmaxf(mx, l[j]);
      mn = fminf(mn, l[j]);
    }
  }
  wave_max_min(mx, mn);
  if (lane == 0) {
    out.red[0][wave] = mx;
    out.red[1][wave] = mn;
  }
  if (tid < kHistBins) out.hist[tid] = 0u;
  __syncthreads();
  mx = fmaxf(fmaxf(out.red[0][0], out.red[0][1]), fmaxf(out.red[0][2], out.red[0][3]));
  mn = fminf(fminf(out.red[1][0], out.red[1][1]), fminf(out.red[1][2], out.red[1][3]));
  OSMD_STAMP(5, timeline_first());

  rank_device<PER>(rv, l, b, out, mx, mn);
  OSMD_STAMP(6, timeline_first());

  // The softmax denominator over every expert (reference_ops.cpp:135-151),
  // its four wavefront sums combined in a fixed order.
  float sum = 0.0f;
  if (need_p) {
#pragma unroll
    for (int j = 0; j < PER; ++j) sum += (base + j < E) ? expf(l[j] - mx) : 0.0f;
    sum = wave_sum(sum);
    if (lane == 0) out.red[2][wave] = sum;
  }

  // The certificate: every expert outside the picks below the k-th's lower
  // bound, each adjacent pair of picks far enough apart (one thread per
  // pair), and the k-th pick far from underflow.
  const float lk = out.lg[k - 1];
  const float low = lk - kBoundSlack * out.bd[k - 1];
  const uint64_t kth = (static_cast<uint64_t>(ordered_key(lk)) << 32) | ~out.id[k - 1];
  bool bad = false;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t e = base + j;
    const uint64_t c = (static_cast<uint64_t>(ordered_key(l[j])) << 32) | ~e;
    if (e < E && c < kth && !(l[j] + kBoundSlack * b[j] + tie_margin(mx, l[j]) < low)) bad = true;
  }
  if (tid + 1u < k) {
    const uint32_t i = tid;
    const float need = kBoundSlack * (out.bd[i] + out.bd[i + 1]) +
                       (out.id[i] > out.id[i + 1] ? tie_margin(mx, out.lg[i + 1]) : 0.0f);
    if (!(out.lg[i] - out.lg[i + 1] > need)) bad = true;
  }
  if (tid == 0 && !(lk - mx >= -kUnderflowGap)) bad = true;
  bad = __syncthreads_or(bad) != 0;
  OSMD_STAMP(7, timeline_first());
  if (need_p) sum = ((out.red[2][0] + out.red[2][1]) + out.red[2][2]) + out.red[2][3];
  bool full = false;
  if (bad) full = select_exact<PER, DEEP>(rv, t, l, b, out, mx);
  if (need_p && tid < k) out.p[tid] = expf(out.lg[tid] - mx) / sum;
  if (tid == 0) out.flags = (bad ? 1u : 0u) | (full ? 2u : 0u);
  if (count && tid == 0 && rv.stats != nullptr) {
    atomicAdd(rv.stats + 0, 1u);
    if (bad) atomicAdd(rv.stats + 1, 1u);
    if (full) atomicAdd(rv.stats + 2, 1u);
    if (bad && out.nneartie != 0u) atomicAdd(rv.stats + 3, out.nneartie);
  }
  __syncthreads();
}

// The routing counters of a selection made with count = false
// (thread 0, after the selection).
template <int PER>
__device__ __forceinline__ void count_selection(const RouteView& rv, const Selection<PER>& s) {
  if (rv.stats == nullptr) return;
  const bool bad = (s.flags & 1u) != 0u;
  atomicAdd(rv.stats + 0, 1u);
  if (bad) atomicAdd(rv.stats + 1, 1u);
  if (s.flags & 2u) atomicAdd(rv.stats + 2, 1u);
  if (bad && s.nneartie != 0u) atomicAdd(rv.stats + 3, s.nneartie);
}

// Router GEMM planes summed with every load in flight first (up to 8 K
// ranges: hidden 4096 at 512-column ranges; more take a loop).
constexpr uint32_t kMaxPlanes = 8;

// Loads token t's logits and their bounds (and table pointers) and selects;
// every thread of the workgroup calls it.
// PLANES = false: the logits are final (the per-token router's), so the
// router GEMM's plane sums are not compiled in and the loads below are the
// first thing the workgroup issues.
template <int PER, bool DEEP = false, bool PLANES = true>
__device__ __forceinline__ void select_block(const RouteView& rv, uint32_t t, Selection<PER>& out, bool count,
                                             bool need_p = true) {
  const uint32_t E = rv.expert_count;
  const uint32_t D = rv.hidden;
  const float* lg = rv.logits + static_cast<size_t>(t) * E;
  const uint32_t base = threadIdx.x * PER;
  float p[PER], bnd[PER];
  const uint8_t* tab[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t e = (base + j < E) ? base + j : E - 1u;  // clamped: every load in bounds
    if (PLANES && rv.planes != nullptr) {
      // Partial sums of the router GEMM's K ranges, added in plane order.
      // Range r of R columns starts at the running sum P_r, so its prefix
      // sums are bounded by R |P_r| plus the plane's own part.
      const size_t ps = static_cast<size_t>(rv.tokens) * (E + 1u);
      const size_t o = static_cast<size_t>(t) * (E + 1u) + e;
      const float* pl = rv.planes + o;
      const bool bounded = rv.bound_planes != nullptr;
      const float cols = static_cast<float>(D / rv.parts);
      float v, rs = 0.0f;
      if (rv.parts <= kMaxPlanes) {
        // Every plane's loads issued before the first addition.
        float pv[kMaxPlanes], rb[kMaxPlanes];
#pragma unroll
        for (uint32_t part = 0; part < kMaxPlanes; ++part) {
          if (part < rv.parts) {
            pv[part] = pl[part * ps];
            rb[part] = bounded ? rv.bound_planes[part * ps + o] : 0.0f;
          }
        }
        v = pv[0];
        rs = rb[0];
#pragma unroll
        for (uint32_t part = 1; part < kMaxPlanes; ++part) {
          if (part < rv.parts) {
            rs += rb[part] + cols * fabsf(v);
            v += pv[part];
          }
        }
      } else {
        v = pl[0];
        if (bounded) rs = rv.bound_planes[o];
        for (uint32_t part = 1; part < rv.parts; ++part) {
          if (bounded) rs += rv.bound_planes[part * ps + o] + cols * fabsf(v);
          v += pl[part * ps];
        }
      }
      p[j] = v;
      // Per plane: the GEMM's bound part (router_gemm_bound_coef), plus R
      // |P_r| for the prefix sums of range r, which start at P_r.
      bnd[j] = bounded ? kBoundSlack * 0x1p-24f * rs : INFINITY;
      if (base + j < E) rv.logits_out[static_cast<size_t>(t) * E + e] = v;
    } else {
      p[j] = lg[e];
      bnd[j] = rv.bounds != nullptr ? rv.bounds[static_cast<size_t>(t) * E + e] : INFINITY;
    }
    tab[j] = rv.expert_table ? rv.expert_table[e] : nullptr;
  }
  if (PLANES && rv.planes != nullptr && rv.has_shared && threadIdx.x == 0) {
    const size_t ps = static_cast<size_t>(rv.tokens) * (E + 1u);
    const float* pl = rv.planes + static_cast<size_t>(t) * (E + 1u) + E;
    float g = pl[0];
    for (uint32_t part = 1; part < rv.parts; ++part) g += pl[part * ps];
    rv.gate_out[t] = 1.0f / (1.0f + expf(-g));  // reference_ops.cpp:214-216
  }
  select_values<PER, DEEP>(rv, t, p, bnd, tab, out, count, need_p);
}

template <int PER>
__device__ __forceinline__ const uint8_t* pick_blob(const RouteView& rv, const Selection<PER>& s,
                                                    uint32_t r) {
  const uint8_t* b = rv.expert_table ? s.blob[s.id[r]] : nullptr;
  return b ? b : rv.fallback;
}

// Writes the selection of token t: ids and weights in pick order, the
// selected mass summed in pick order and the optional renormalisation
// (qwen_router.cpp:72-91), and each slot's blob (shared expert last).
// Lanes 0 .. k of wavefront 0 take part, one pick each; the mass is added in
// pick order from their values.
template <int PER>
__device__ __forceinline__ void publish_selection(const RouteView& rv, uint32_t t, uint32_t tid,
                                                  const Selection<PER>& s) {
  if (tid >= kWave) return;
  const uint32_t k = rv.top_k;
  const uint32_t nslot = k + rv.has_shared;
  const float pr = tid < k ? s.p[tid] : 0.0f;
  float mass = 0.0f;
  for (uint32_t r = 0; r < k; ++r) mass = mass + readlane_f(pr, static_cast<int>(r));
  if (tid < k) {
    rv.ids[static_cast<size_t>(t) * k + tid] = s.id[tid];
    rv.weights[static_cast<size_t>(t) * k + tid] = rv.norm_topk_prob ? pr / mass : pr;
    rv.slot_ptrs[static_cast<size_t>(t) * nslot + tid] = pick_blob(rv, s, tid);
  } else if (tid == k && nslot > k) {
    rv.slot_ptrs[static_cast<size_t>(t) * nslot + k] = rv.shared_expert;
  }
  if (tid == 0) rv.mass[t] = mass;
}

template <int PER>
__global__ __launch_bounds__(kSelThreads) void select_kernel(RouteView rv) {
  __shared__ Selection<PER> sel;
  select_block<PER, true>(rv, blockIdx.x, sel, true);
  publish_selection(rv, blockIdx.x, threadIdx.x, sel);
}

// ---------------------------------------------------------------------------
// Router GEMV. A wavefront owns one router row; lane l reads 32 consecutive
// elements per pass of 2048 (route_block), kept as loaded until the FMA.

// Token t's input, RMS-normalised when the flags ask for it
// (reference_ops.cpp:96-128), into xs in LDS (column c at xs_index(c)); write_norm also stores it to
// x_norm. Every workgroup that needs x normalises its own copy: the values
// are the same bits everywhere. 256 threads, hidden <= 8192.
// xs holds column c at xs_index(c): every 32 columns are followed by 4
// unused floats, so lanes that read 32 consecutive columns each (16 bytes
// at a time) spread over the LDS banks.
__device__ __forceinline__ uint32_t xs_index(uint32_t c) { return c + (c / 32u) * 4u; }
__host__ __device__ constexpr size_t route_lds_bytes(uint32_t hidden) {
  return (static_cast<size_t>(hidden) + (hidden / 32u) * 4u) * sizeof(float);
}

__device__ __forceinline__ void stage_x(const osmd_moe_args& a, uint32_t t, float* xs, bool write_norm) {
  __shared__ float red[kRouteWaves];
  const uint32_t D = a.geom.hidden;
  const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const float4* x4 = reinterpret_cast<const float4*>(a.x + static_cast<size_t>(t) * D);
  const uint32_t n4 = D / 4u;
  constexpr int kX4PerThread = 8;
  float4 xv[kX4PerThread];
#pragma unroll
  for (int u = 0; u < kX4PerThread; ++u) {
    const uint32_t i = tid + u * 256u;
    xv[u] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (a.flags & OSMD_MOE_RMSNORM) {
    // The norm weights are loaded with x, before the reduction: loaded after
    // it, each load waited behind the previous chunk's x_norm store (vector
    // memory operations are counted in order).
    const float4* w4 = reinterpret_cast<const float4*>(a.norm_weight);
    float4 nwv[kX4PerThread];
#pragma unroll
    for (int u = 0; u < kX4PerThread; ++u) {
      const uint32_t i = tid + u * 256u;
      nwv[u] = i < n4 ? w4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < kX4PerThread; ++u)
      ss += xv[u].x * xv[u].x + xv[u].y * xv[u].y + xv[u].z * xv[u].z + xv[u].w * xv[u].w;
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < kRouteWaves; ++w2) tot += red[w2];
    const float scale = 1.0f / sqrtf(tot / static_cast<float>(D) + a.rms_eps);
#pragma unroll
    for (int u = 0; u < kX4PerThread; ++u) {
      const uint32_t i = tid + u * 256u;
      if (i < n4) {
        const float4 nw = nwv[u];
        xv[u].x = xv[u].x * (scale * nw.x);
        xv[u].y = xv[u].y * (scale * nw.y);
        xv[u].z = xv[u].z * (scale * nw.z);
        xv[u].w = xv[u].w * (scale * nw.w);
      }
    }
  }
  float4* xn4 = reinterpret_cast<float4*>(a.x_norm + static_cast<size_t>(t) * D);
#pragma unroll
  for (int u = 0; u < kX4PerThread; ++u) {
    const uint32_t i = tid + u * 256u;
    if (i < n4) {
      *reinterpret_cast<float4*>(xs + xs_index(4u * i)) = xv[u];
      if (write_norm) xn4[i] = xv[u];
    }
  }
  __syncthreads();
}

// Router rows blk*4 .. blk*4+3 of token t (row E is the shared-expert gate
// vector): logits, or the sigmoid shared gate (reference_ops.cpp:214-216).
// A wavefront owns one row. Lane l covers columns 2048 v + 32 l .. +32 for
// each pass v (RCH / 4 passes of four 8-element loads, hidden <= 512 RCH).
// The dot product runs in fp64: every product of a router element (at most
// 24 significant bits) and an fp32 input is exact there, and the sums'
// rounding is far below fp32's.
//
// Each logit also gets its bound (when a.logit_bounds is set). With u =
// 2^-24 and p_c = w_c x_c:
//  - the reference sums acc = acc + p_c in column order, rounding each
//    product and sum, so its error is at most u (sum_c |p_c| + sum_c |S_c|),
//    S_c its partial sums; |S_c| <= |P_c| + (a second-order term), P_c the
//    exact prefix sums;
//  - this kernel's logit is the fp64 sum rounded once to fp32: within
//    u |l| of the exact sum, plus the fp64 sums' own error, below
//    2^-40 sum_c |p_c|;
//  - an RMS-normalised input differs from the reference's by a common factor
//    (handled by the selection) and per element by at most 4 u.
// sum_c |P_c| over a lane's 32 columns of a pass is at most 32 |start| plus
// the sum of |its own running sums|, start the exclusive prefix of the lane
// totals (one wavefront scan per pass, plus the totals of the passes
// before). The bound written is
// (1 + 2^-9) u (sum |P_c| + (2 + 4 [RMSNorm] + n^2 u) sum |p_c| + |l|), n
// the width; the slack covers the bound's own rounding and the fp32 running
// sums it is computed from.
template <int RD, int RCH>
__device__ __forceinline__ void route_block(const osmd_moe_args& a, uint32_t t, uint32_t blk, float* xs) {
  static_assert(RCH % 4 == 0, "four loads per pass");
  const uint32_t D = a.geom.hidden;
  const uint32_t E = a.expert_count;
  const uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const uint32_t nrows = E + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  const uint32_t row = blk * kRouteWaves + wave;
  constexpr size_t esz = (RD == OSM_META_F32) ? 4u : 2u;
  auto col = [&](int u) { return static_cast<uint32_t>(u / 4) * 2048u + lane * 32u + static_cast<uint32_t>(u % 4) * 8u; };
  // The row is issued before x, so both are in flight together.
  Raw8<RD> w[RCH];
  if (row < nrows) {
    if constexpr (RD == OSM_ROUTER_AFFINE_Q8) {
      const Q8Row qr = row < E ? q8_row(a.router, E, row, D, a.router_group)
                               : q8_row(a.shared_gate_vec, 1u, 0u, D, a.router_group);
#pragma unroll
      for (int u = 0; u < RCH; ++u)
        if (col(u) < D) load_q8x8(qr, col(u), w[u]);
    } else {
      const uint8_t* wrow = row < E ? static_cast<const uint8_t*>(a.router) + static_cast<size_t>(row) * D * esz
                                    : static_cast<const uint8_t*>(a.shared_gate_vec);
#pragma unroll
      for (int u = 0; u < RCH; ++u)
        if (col(u) < D) load_raw8<RD>(wrow, col(u), w[u]);
    }
  }
  stage_x(a, t, xs, blk == 0);
  if (row < nrows) {
    const bool bound = row < E && a.logit_bounds != nullptr;
    float aa = 0.0f, rsum = 0.0f, carry = 0.0f;
    double accd = 0.0;
#pragma unroll
    for (int v = 0; v < RCH / 4; ++v) {
      if (static_cast<uint32_t>(v) * 2048u >= D) break;  // wavefront-uniform
      double pd = 0.0;  // the lane's running sum over its columns of this pass
      float qa = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int u = v * 4 + q;
        const uint32_t c = col(u);
        if (c < D) {
          const float* xp = xs + xs_index(c);
          const float st = static_cast<float>(pd);
          double csd = 0.0;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float wv = raw8_get<RD>(w[u], j), xv = xp[j];
            csd = fma(static_cast<double>(wv), static_cast<double>(xv), csd);
            aa = fmaf(fabsf(wv), fabsf(xv), aa);
            qa += fabsf(st + static_cast<float>(csd));
          }
          pd += csd;
        }
      }
      if (bound) {
        const float lf = static_cast<float>(pd);
        const float incl = wave_incl_scan(lf);
        rsum += 32.0f * fabsf(carry + (incl - lf)) + qa;
        carry += readlane_f(incl, 63);
      }
      accd += pd;
    }
    const float n = static_cast<float>(D);
    const float c1 = ((a.flags & OSMD_MOE_RMSNORM) ? 6.0f : 2.0f) + n * n * 0x1p-24f;
    float part = rsum + c1 * aa;
    wave_sum_fd(part, accd);
    const float acc = static_cast<float>(accd);
    if (lane == 0) {
      if (row < E) {
        a.logits[static_cast<size_t>(t) * E + row] = acc;
        if (bound) a.logit_bounds[static_cast<size_t>(t) * E + row] = kBoundSlack * 0x1p-24f * (part + fabsf(acc));
      } else {
        a.shared_gate[t] = 1.0f / (1.0f + expf(-acc));
      }
    }
  }
}

template <int RD>
__global__ __launch_bounds__(256) void route_kernel(osmd_moe_args a) {
  extern __shared__ __align__(16) float xs[];  // normalised input of this token, at xs_index(column)
  OSMD_STAMP(0, timeline_first());
  OSMD_STAMP(2, timeline_last());
  route_block<RD, 16>(a, blockIdx.y, blockIdx.x, xs);
  OSMD_STAMP(1, timeline_first());
  OSMD_STAMP(3, timeline_last());
  OSMD_STAMP_FLUSH(0, 2, timeline_first());
  OSMD_STAMP_FLUSH(2, 4, timeline_last());
}

// ---------------------------------------------------------------------------
// gate/up + SwiGLU. Each wavefront owns ROWS consecutive rows of one
// slot; lane l reads 16-byte chunks l, l+64, ... of each row, so a wavefront
// load is 1 KB of contiguous packed weights. The lane's slice of x (and its
// sum) stays in registers for all rows. PER > 0: routed slots select their
// expert from the logits first (PER = experts per lane of the selection).
// One token takes three rows per wavefront (12 per workgroup, 43 workgroups
// per slot at intermediate 512): more workgroups share the VALU-bound dot
// products that follow the weight loads (batch-1 µs per token-layer for
// 8 / 6 / 4 / 3 / 2 rows: 20.95 / 20.66 / 20.52 / 20.33 / 20.76). Several
// tokens take eight: every workgroup repeats the selection of its token, and
// at 4 and 16 tokens three rows measured 14% and 20% slower than eight.
constexpr int kGuWaves = 4;
constexpr int kGuRowsOneToken = 3;
constexpr int kGuRowsBatched = 8;

// Lane's slices of x (chunks lane, lane+64, ... of 32 floats). Lanes past the
// row end (hidden < 64*32*CPL) read chunk nch-1 again and zero their slice,
// so every load is unconditional and in bounds. x may be global or LDS.
template <int CPL>
__device__ __forceinline__ void load_xr(const float* x, uint32_t nch, uint32_t lane, float (&xr)[CPL][32]) {
#pragma unroll
  for (int ci = 0; ci < CPL; ++ci) {
    const uint32_t c = lane + kWave * ci;
    const bool valid = c < nch;
    const uint32_t cc = valid ? c : nch - 1u;
    const float4* xp = reinterpret_cast<const float4*>(x + cc * 32u);
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float4 f = xp[v];
      xr[ci][4 * v + 0] = valid ? f.x : 0.0f;
      xr[ci][4 * v + 1] = valid ? f.y : 0.0f;
      xr[ci][4 * v + 2] = valid ? f.z : 0.0f;
      xr[ci][4 * v + 3] = valid ? f.w : 0.0f;
    }
  }
}

// Gate and up rows blk*16 .. blk*16+15 of slot j of token t from `blob`,
// SwiGLU'd into h[t, j, row].
// store(index, value): h[t, j, row] at index (t * nslot + j) * I + row.
template <int META, int CPL, int ROWS, typename Store>
__device__ __forceinline__ void gate_up_rows(const GateUpParams& p, uint32_t t, uint32_t j, uint32_t blk,
                                             const uint8_t* blob, float (&xr)[CPL][32], Store&& store) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t D = p.g.hidden, I = p.g.inter, G = p.g.group;
  const uint32_t nch = D / 32u;  // 16-byte chunks per row
  const uint32_t gpr = D / G;    // groups per row
  const osm_expert_offsets off = osm_expert_layout(p.g);
  const uint32_t r0 = (blk * kGuWaves + wave) * ROWS;
  uint4 qg[ROWS][CPL], qu[ROWS][CPL];
  uint32_t sg[ROWS][CPL], bg[ROWS][CPL];
  uint32_t su[ROWS][CPL], bu[ROWS][CPL];
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    const uint32_t r = (r0 + i < I) ? r0 + i : I - 1u;
#pragma unroll
    for (int ci = 0; ci < CPL; ++ci) {
      const uint32_t c = lane + kWave * ci;
      const uint32_t cc = c < nch ? c : nch - 1u;
      const size_t qo = (static_cast<size_t>(r) * nch + cc) * 16u;
      qg[i][ci] = ldg16(blob + off.gate_q + qo);
      qu[i][ci] = ldg16(blob + off.up_q + qo);
      const size_t gi = static_cast<size_t>(r) * gpr + (cc * 32u) / G;
      sg[i][ci] = meta_bits<META>(blob + off.gate_s, gi);
      bg[i][ci] = meta_bits<META>(blob + off.gate_b, gi);
      su[i][ci] = meta_bits<META>(blob + off.up_s, gi);
      bu[i][ci] = meta_bits<META>(blob + off.up_b, gi);
    }
  }
  OSMD_STAMP(9, timeline_first());
  // The lane's slices of x (and their sums), loaded while the weights are in flight.
  load_xr<CPL>(p.x + static_cast<size_t>(t) * D, nch, lane, xr);
  float xsum[CPL];
#pragma unroll
  for (int ci = 0; ci < CPL; ++ci) {
    xsum[ci] = 0.0f;
#pragma unroll
    for (int v = 0; v < 32; ++v) xsum[ci] += xr[ci][v];
  }
  float gsum[ROWS], usum[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    float ga = 0.0f, ua = 0.0f;
#pragma unroll
    for (int ci = 0; ci < CPL; ++ci) {
      ga += meta_widen<META>(sg[i][ci]) * nib_dot32(qg[i][ci], xr[ci]) +
            meta_widen<META>(bg[i][ci]) * xsum[ci];
      ua += meta_widen<META>(su[i][ci]) * nib_dot32(qu[i][ci], xr[ci]) +
            meta_widen<META>(bu[i][ci]) * xsum[ci];
    }
    gsum[i] = wave_sum(ga);
    usum[i] = wave_sum(ua);
  }
  // SwiGLU of the wavefront's rows in one pass, lane i for row r0 + i (one
  // exp and division on the wavefront's path instead of one per row).
  if (lane < static_cast<uint32_t>(ROWS)) {
    float g = gsum[0], u = usum[0];
#pragma unroll
    for (int i = 1; i < ROWS; ++i) {
      g = lane == static_cast<uint32_t>(i) ? gsum[i] : g;
      u = lane == static_cast<uint32_t>(i) ? usum[i] : u;
    }
    const uint32_t r = r0 + lane;
    if (r < I) store((static_cast<size_t>(t) * p.src.nslot + j) * I + r, silu_mul(g, u));
  }
}

template <int META, int CPL, int PER, int ROWS>
__global__ __launch_bounds__(256) void gate_up_kernel(GateUpParams p) {
  const uint32_t t = blockIdx.z;
  const uint32_t j = blockIdx.y;
  // x is read with the weights, after the selection, so its slices are not
  // held in registers through it; both loads are in flight together.
  auto rows = [&](const uint8_t* blob) {
    if (blob == nullptr) blob = p.rv.fallback;  // never dereference a null slot
    float xr[CPL][32];
    gate_up_rows<META, CPL, ROWS>(p, t, j, blockIdx.x, blob, xr, [&](size_t i, float v) { p.h[i] = v; });
  };
  if constexpr (PER > 0) {
    // Routed slot: the workgroup selects first. Workgroup (0, 0) publishes
    // the selection and counts it after its own rows, so those stores never
    // delay its weight loads.
    const RouteView& rv = p.rv;
    __shared__ Selection<PER> sel;
    if (j < rv.top_k) {
      // The per-token router's final logits; only the publishing workgroup
      // forms the probabilities.
      const bool publisher = blockIdx.x == 0 && j == 0;
      OSMD_STAMP(4, timeline_first());
      select_block<PER, false, false>(rv, t, sel, false, publisher);
      OSMD_STAMP(8, timeline_first());
      rows(pick_blob(rv, sel, j));
      OSMD_STAMP(10, timeline_first());
      if (publisher) {
        publish_selection(rv, t, threadIdx.x, sel);
        if (threadIdx.x == 0) count_selection(rv, sel);
      }
      OSMD_STAMP(11, timeline_first());
      OSMD_STAMP_FLUSH(4, 12, timeline_first());
    } else {
      rows(rv.shared_expert);
    }
    OSMD_STAMP(15, timeline_last());
    OSMD_STAMP_FLUSH(15, 16, timeline_last());
  } else {
    // Host-driven slots: every slot in order, or the listed ones.
    const uint32_t js = p.list.count ? slot_at(p.list, j) : j;
    const uint8_t* blob = p.src.blob(t, js);
    float xr[CPL][32];
    gate_up_rows<META, CPL, ROWS>(p, t, js, blockIdx.x, blob ? blob : p.rv.fallback, xr,
                                  [&](size_t i, float v) { p.h[i] = v; });
  }
}

// ---------------------------------------------------------------------------
// down + weighted accumulate (+ residual). LPR lanes cover one output row
// (I/32 chunks). A workgroup is four wavefronts: two row groups of 64/LPR
// rows, each covered twice, by the even and by the odd slots, so a launch has
// about one wavefront per SIMD at hidden 2048. Every slot's h sits in LDS
// with its per-chunk sums; the weighted sum over picks and the shared expert
// is a fixed-order register accumulation per row plus one LDS combine of the
// two slot halves -- no atomics and no separate accumulate launches.
//
// LDS chunks of 32 floats are laid out kChunkStride floats apart, so the
// 16-byte reads of the LPR lanes of a row land in different banks.
constexpr int kDownThreads = 256;
constexpr uint32_t kChunkStride = 36;

template <int LPR>
constexpr uint32_t down_rows_per_block() {
  return 2u * (kWave / LPR);
}

size_t down_lds_bytes(uint32_t inter, uint32_t nslot, uint32_t rows_per_block) {
  const size_t chunks = static_cast<size_t>(nslot) * (inter / 32u);
  return (chunks * (kChunkStride + 1u) + 2u * rows_per_block) * sizeof(float);
}


// down + weighted accumulate for rows blk * rows_per_block ... of token t.
// MODE kDownParts writes each listed slot's per-lane partial instead; MODE
// kDownCombine reads every slot's partial back in place of computing it and
// then accumulates exactly as kDownFused does.
template <int META, int LPR, int MAXS, int MODE>
__device__ __forceinline__ void down_block(const DownParams& p, uint32_t t, uint32_t blk, float* hs) {
  constexpr uint32_t kRowsPerGroup = kWave / LPR;
  constexpr uint32_t kRowsPerBlock = down_rows_per_block<LPR>();
  constexpr int kSlotsPerWave = (MAXS + 1) / 2;
  const uint32_t D = p.g.hidden, I = p.g.inter, G = p.g.group;
  const uint32_t nslot = p.src.nslot;
  // The slots this launch covers, by cover index: every slot in order, or
  // the list.
  const uint32_t ncover = MODE == kDownParts ? p.list.count : nslot;
  const uint32_t nchd = I / 32u;
  const uint32_t gpr = I / G;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid % kWave;
  const uint32_t wave = tid / kWave;
  const uint32_t rg = wave & 1u;    // row group
  // Cover indices half, half + 2, ...: wavefront-uniform, so the slot
  // pointers and weights below are scalar loads issued together.
  const uint32_t half = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(wave >> 1)));
  const uint32_t c = lane % LPR;
  const uint32_t row_local = rg * kRowsPerGroup + lane / LPR;
  const uint32_t row = blk * kRowsPerBlock + row_local;
  const bool active = row < D && c < nchd;
  const uint32_t rr = row < D ? row : D - 1u;
  const uint32_t cc = c < nchd ? c : nchd - 1u;
  const osm_expert_offsets off = osm_expert_layout(p.g);
  float* hsum = hs + static_cast<size_t>(nslot) * nchd * kChunkStride;
  float* halves = hsum + static_cast<size_t>(nslot) * nchd;
  // Per-lane partial of slot j at this lane's row and chunk.
  auto part_at = [&](uint32_t j) {
    return ((static_cast<size_t>(t) * nslot + j) * D + rr) * LPR + c;
  };

  const float4* h4 = reinterpret_cast<const float4*>(p.h + static_cast<size_t>(t) * nslot * I);
  const uint32_t n4 = nslot * I / 4u;  // a multiple of 8 (I % 32 == 0)
  constexpr int kH4PerThread = 8;
  float4 hv[kH4PerThread];
  // Every lane issues all kH4PerThread loads, an index past the end reading
  // the last element: with no branch around them, a wait for a load issued
  // earlier counts exactly these behind it. Such a value is never stored:
  // the 8 lanes of a chunk are all in range or all past it (n4 % 8 == 0).
  auto load_h = [&](uint32_t pass) {
#pragma unroll
    for (int u = 0; u < kH4PerThread; ++u) {
      const uint32_t f = (pass * kH4PerThread + u) * kDownThreads + tid;
      hv[u] = h4[f < n4 ? f : n4 - 1u];
    }
  };
  if constexpr (MODE != kDownCombine) load_h(0);
  // This wavefront's slots. Their pointers and weights sit at wavefront-
  // uniform addresses, so they are scalar loads, which complete on their own
  // counter: waiting for them does not wait for h's vector loads issued
  // before them. The packed chunk and metadata of each slot are then loaded
  // with no branch between them. Slots past nslot and null pointers read a
  // valid blob with weight 0 (the combine reads no pointer: every slot it
  // adds was resident).
  const uint8_t* bp[kSlotsPerWave];
  float w[kSlotsPerWave];
  uint32_t js[kSlotsPerWave];
#pragma unroll
  for (int i = 0; i < kSlotsPerWave; ++i) {
    const uint32_t ci = half + 2u * i;
    const uint32_t j = ci < ncover ? (MODE == kDownParts ? slot_at(p.list, ci) : ci) : nslot;
    const uint32_t jj = j < nslot ? j : 0u;
    bp[i] = MODE == kDownCombine ? p.fallback : p.src.blob(t, jj);
    const float* ws = jj < p.top_k ? (p.weights ? p.weights + static_cast<size_t>(t) * p.top_k + jj : nullptr)
                                   : (p.shared_gate ? p.shared_gate + t : nullptr);
    w[i] = ws ? *ws : 1.0f;
    js[i] = jj;
    if (j >= nslot || (MODE != kDownCombine && bp[i] == nullptr)) w[i] = 0.0f;
    if (bp[i] == nullptr) bp[i] = p.fallback;
  }
  uint4 q[kSlotsPerWave];
  uint32_t sb[kSlotsPerWave], bb[kSlotsPerWave];
  float pin[kSlotsPerWave];
  const size_t qo = (static_cast<size_t>(rr) * nchd + cc) * 16u;
  const size_t gi = static_cast<size_t>(rr) * gpr + (cc * 32u) / G;
#pragma unroll
  for (int i = 0; i < kSlotsPerWave; ++i) {
    if constexpr (MODE == kDownCombine) {
      pin[i] = (active && half + 2u * i < nslot) ? p.parts[part_at(js[i])] : 0.0f;
    } else {
      q[i] = ldg16(bp[i] + off.down_q + qo);
      sb[i] = meta_bits<META>(bp[i] + off.down_s, gi);
      bb[i] = meta_bits<META>(bp[i] + off.down_b, gi);
    }
  }
  OSMD_STAMP(13, MODE == kDownFused && timeline_first());

  if constexpr (MODE != kDownCombine) {
    // Stage h and its per-chunk sums: 8 consecutive threads hold one 32-float
    // chunk, summed with DPP within the lane group. The first batch is staged
    // while the weights are in flight (only its own loads are waited for);
    // h of more than kH4PerThread * 1024 floats takes further passes.
    auto stage = [&](uint32_t pass) {
#pragma unroll
      for (int u = 0; u < kH4PerThread; ++u) {
        const uint32_t f = (pass * kH4PerThread + u) * kDownThreads + tid;
        const float s4 = row_sum<8>((hv[u].x + hv[u].y) + (hv[u].z + hv[u].w));
        if (f < n4) {
          const uint32_t chunk = f / 8u;  // slot * nchd + chunk in the slot
          *reinterpret_cast<float4*>(hs + chunk * kChunkStride + (f % 8u) * 4u) = hv[u];
          if ((tid & 7u) == 0u) hsum[chunk] = s4;
        }
      }
    };
    stage(0);
    for (uint32_t pass = 1; pass * kH4PerThread * kDownThreads < n4; ++pass) {
      load_h(pass);
      stage(pass);
    }
    __syncthreads();
  }

  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < kSlotsPerWave; ++i) {
    float part;
    if constexpr (MODE == kDownCombine) {
      part = pin[i];
    } else {
      const uint32_t chunk = js[i] * nchd + cc;
      part = meta_widen<META>(sb[i]) * nib_dot32(q[i], hs + chunk * kChunkStride) +
             meta_widen<META>(bb[i]) * hsum[chunk];
    }
    if constexpr (MODE == kDownParts) {
      if (active && half + 2u * i < ncover) p.parts[part_at(js[i])] = part;
    } else {
      acc = fmaf(w[i], part, acc);
    }
    // Keep each slot's LDS reads next to their use.
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (MODE == kDownParts) return;
  if (!active) acc = 0.0f;
  if constexpr (LPR <= 16)
    acc = row_sum<LPR>(acc);
  else
    acc = group_sum(acc, LPR);
  if (c == 0) halves[half * kRowsPerBlock + row_local] = acc;
  __syncthreads();
  if (tid < kRowsPerBlock) {
    const uint32_t orow = blk * kRowsPerBlock + tid;
    if (orow < D) {
      const float v = halves[tid] + halves[kRowsPerBlock + tid];
      const size_t o = static_cast<size_t>(t) * D + orow;
      p.y[o] = p.residual ? p.residual[o] + v : v;
    }
  }
}

template <int META, int LPR, int MAXS, int MODE>
__global__ __launch_bounds__(kDownThreads) void down_kernel(DownParams p) {
  extern __shared__ __align__(16) float hs[];  // chunks, then chunk sums, then [2][rows] halves
  OSMD_STAMP(12, MODE == kDownFused && timeline_first());
  down_block<META, LPR, MAXS, MODE>(p, blockIdx.y, blockIdx.x, hs);
  OSMD_STAMP(14, MODE == kDownFused && timeline_first());
  OSMD_STAMP(16, MODE == kDownFused && timeline_last());
  OSMD_STAMP_FLUSH(12, 15, MODE == kDownFused && timeline_first());
  OSMD_STAMP_FLUSH(16, 17, MODE == kDownFused && timeline_last());
}


// ---------------------------------------------------------------------------
// Host-side launchers.

int pow2_at_least(uint32_t v) {
  int p = 1;
  while (static_cast<uint32_t>(p) < v) p <<= 1;
  return p;
}

template <int META, int CPL>
int launch_gate_up_cpl(const GateUpParams& gp, uint32_t tokens, int per, hipStream_t st) {
  const bool one = tokens == 1u;
  const uint32_t rows_per_block = kGuWaves * (one ? kGuRowsOneToken : kGuRowsBatched);
  const dim3 grid((gp.g.inter + rows_per_block - 1) / rows_per_block, gp.list.count ? gp.list.count : gp.src.nslot,
                  tokens);
  switch (per) {
    case 0:
      if (one) gate_up_kernel<META, CPL, 0, kGuRowsOneToken><<<grid, 256, 0, st>>>(gp);
      else gate_up_kernel<META, CPL, 0, kGuRowsBatched><<<grid, 256, 0, st>>>(gp);
      break;
    case 2:
      if (one) gate_up_kernel<META, CPL, 2, kGuRowsOneToken><<<grid, 256, 0, st>>>(gp);
      else gate_up_kernel<META, CPL, 2, kGuRowsBatched><<<grid, 256, 0, st>>>(gp);
      break;
    default:
      if (one) gate_up_kernel<META, CPL, 4, kGuRowsOneToken><<<grid, 256, 0, st>>>(gp);
      else gate_up_kernel<META, CPL, 4, kGuRowsBatched><<<grid, 256, 0, st>>>(gp);
      break;
  }
  return launch_status();
}

template <int META>
int launch_gate_up_meta(const GateUpParams& gp, uint32_t tokens, int per, hipStream_t st) {
  const uint32_t nch = gp.g.hidden / 32u;
  if (nch <= 64u) return launch_gate_up_cpl<META, 1>(gp, tokens, per, st);
  if (nch <= 128u) return launch_gate_up_cpl<META, 2>(gp, tokens, per, st);
  return launch_gate_up_cpl<META, 4>(gp, tokens, per, st);
}

// per: 0 = slots from gp.src; otherwise the selection's experts per lane.
int launch_gate_up(const GateUpParams& gp, uint32_t tokens, int per, hipStream_t st) {
  switch (gp.g.meta_dtype) {
    case OSM_META_F32: return launch_gate_up_meta<OSM_META_F32>(gp, tokens, per, st);
    case OSM_META_F16: return launch_gate_up_meta<OSM_META_F16>(gp, tokens, per, st);
    default: return launch_gate_up_meta<OSM_META_BF16>(gp, tokens, per, st);
  }
}

// The slots per wavefront follow the slot count (the list's for kDownParts):
// the combine of nslot slots therefore runs the fused form's loop for
// nslot, which is what makes its sums the same.
template <int META, int LPR, int MODE>
int launch_down_lpr(const DownParams& dp, uint32_t tokens, hipStream_t st) {
  constexpr uint32_t rows_per_block = down_rows_per_block<LPR>();
  const dim3 grid((dp.g.hidden + rows_per_block - 1) / rows_per_block, tokens);
  const size_t lds = down_lds_bytes(dp.g.inter, dp.src.nslot, rows_per_block);
  const uint32_t n = MODE == kDownParts ? dp.list.count : dp.src.nslot;
  if (n <= 2u)
    down_kernel<META, LPR, 2, MODE><<<grid, kDownThreads, lds, st>>>(dp);
  else if (n <= 4u)
    down_kernel<META, LPR, 4, MODE><<<grid, kDownThreads, lds, st>>>(dp);
  else if (n <= 8u)
    down_kernel<META, LPR, 8, MODE><<<grid, kDownThreads, lds, st>>>(dp);
  else if (n <= 12u)
    down_kernel<META, LPR, 12, MODE><<<grid, kDownThreads, lds, st>>>(dp);
  else
    down_kernel<META, LPR, kMaxSlots + 1, MODE><<<grid, kDownThreads, lds, st>>>(dp);
  return launch_status();
}

template <int META, int MODE>
int launch_down_meta(const DownParams& dp, uint32_t tokens, hipStream_t st) {
  switch (pow2_at_least(dp.g.inter / 32u)) {
    case 1: return launch_down_lpr<META, 1, MODE>(dp, tokens, st);
    case 2: return launch_down_lpr<META, 2, MODE>(dp, tokens, st);
    case 4: return launch_down_lpr<META, 4, MODE>(dp, tokens, st);
    case 8: return launch_down_lpr<META, 8, MODE>(dp, tokens, st);
    case 16: return launch_down_lpr<META, 16, MODE>(dp, tokens, st);
    case 32: return launch_down_lpr<META, 32, MODE>(dp, tokens, st);
    default: return launch_down_lpr<META, 64, MODE>(dp, tokens, st);
  }
}

template <int MODE>
int launch_down_mode(const DownParams& dp, uint32_t tokens, hipStream_t st) {
  switch (dp.g.meta_dtype) {
    case OSM_META_F32: return launch_down_meta<OSM_META_F32, MODE>(dp, tokens, st);
    case OSM_META_F16: return launch_down_meta<OSM_META_F16, MODE>(dp, tokens, st);
    default: return launch_down_meta<OSM_META_BF16, MODE>(dp, tokens, st);
  }
}

int launch_down(const DownParams& dp, uint32_t tokens, hipStream_t st) {
  return launch_down_mode<kDownFused>(dp, tokens, st);
}

// Lanes per output row of the down kernel (the partials' last dimension).
uint32_t down_lanes_per_row(uint32_t inter) { return static_cast<uint32_t>(pow2_at_least(inter / 32u)); }

// Experts per lane of a selection: 2 up to 512 experts, 4 beyond. One width
// for every expert count in a range keeps the order of the wavefront sums of
// the softmax the same in every kernel that selects (the per-token kernels
// and the select kernel), so they publish the same bits.
int selection_per(uint32_t experts) { return experts <= 2u * kSelThreads ? 2 : 4; }

template <int RD>
int launch_route_rd(const osmd_moe_args& a, hipStream_t st) {
  const uint32_t nrows = a.expert_count + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  const dim3 grid((nrows + kRouteWaves - 1) / kRouteWaves, a.tokens);
  route_kernel<RD><<<grid, 256, route_lds_bytes(a.geom.hidden), st>>>(a);
  return launch_status();
}

RouteView route_view(const osmd_moe_args& a) {
  RouteView rv;
  rv.logits = a.logits;
  rv.planes = a.logit_planes;
  rv.parts = a.logit_parts;
  rv.tokens = a.tokens;
  rv.logits_out = a.logits;
  rv.gate_out = a.shared_gate;
  rv.expert_count = a.expert_count;
  rv.top_k = a.top_k;
  rv.norm_topk_prob = a.norm_topk_prob;
  rv.has_shared = (a.flags & OSMD_MOE_SHARED) ? 1u : 0u;
  rv.expert_table = a.expert_table;
  rv.shared_expert = a.shared_expert;
  rv.fallback = a.fallback_blob;
  rv.ids = a.ids;
  rv.weights = a.weights;
  rv.mass = a.mass;
  rv.slot_ptrs = a.slot_ptrs;
  rv.bounds = a.logit_bounds;
  rv.bound_planes = a.bound_planes;
  rv.stats = a.route_stats;
  rv.router = a.router;
  rv.router_dtype = a.router_dtype;
  rv.router_group = a.router_group;
  rv.hidden = a.geom.hidden;
  rv.x = a.x;
  rv.x_bf16 = a.x_bf16;
  rv.rms = (a.flags & OSMD_MOE_RMSNORM) ? 1u : 0u;
  rv.norm_weight = a.norm_weight;
  rv.rms_eps = a.rms_eps;
  return rv;
}

int launch_select(const osmd_moe_args& a, hipStream_t st) {
  const RouteView rv = route_view(a);
  switch (selection_per(a.expert_count)) {
    case 2: select_kernel<2><<<a.tokens, kSelThreads, 0, st>>>(rv); break;
    default: select_kernel<4><<<a.tokens, kSelThreads, 0, st>>>(rv); break;
  }
  return launch_status();
}

GateUpParams gate_up_params(const osmd_moe_args& a) {
  const uint32_t nslot = a.top_k + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  GateUpParams gp{};
  gp.g = a.geom;
  gp.src = SlotSource{a.slot_ptrs, nullptr, nslot};
  gp.rv = route_view(a);
  gp.x = a.x_norm;
  gp.h = a.h;
  return gp;
}

DownParams down_params(const osmd_moe_args& a) {
  const uint32_t nslot = a.top_k + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  DownParams dp{};
  dp.g = a.geom;
  dp.src = SlotSource{a.slot_ptrs, nullptr, nslot};
  dp.top_k = a.top_k;
  dp.weights = a.weights;
  dp.shared_gate = a.shared_gate;
  dp.fallback = a.fallback_blob;
  dp.h = a.h;
  dp.residual = (a.flags & OSMD_MOE_RESIDUAL) ? a.x : nullptr;
  dp.y = a.y;
  return dp;
}

}  // namespace

extern "C" {

size_t osmd_moe_down_lds_bytes(uint32_t inter, uint32_t nslot) {
  const uint32_t lpr = static_cast<uint32_t>(pow2_at_least(inter / 32u));
  const uint32_t rows = 2u * (lpr >= static_cast<uint32_t>(kWave) ? 1u : kWave / lpr);
  return down_lds_bytes(inter, nslot, rows);
}

int osmd_moe_router(const osmd_moe_args* a, osmd_stream s) {
  const hipStream_t st = static_cast<hipStream_t>(s);
  switch (a->router_dtype) {
    case OSM_META_F32: return launch_route_rd<OSM_META_F32>(*a, st);
    case OSM_META_F16: return launch_route_rd<OSM_META_F16>(*a, st);
    case OSM_ROUTER_AFFINE_Q8: return launch_route_rd<OSM_ROUTER_AFFINE_Q8>(*a, st);
    default: return launch_route_rd<OSM_META_BF16>(*a, st);
  }
}

int osmd_moe_select(const osmd_moe_args* a, osmd_stream s) {
  return launch_select(*a, static_cast<hipStream_t>(s));
}

int osmd_moe_route(const osmd_moe_args* a, osmd_stream s) {
  const int r = osmd_moe_router(a, s);
  return r != 0 ? r : launch_select(*a, static_cast<hipStream_t>(s));
}

int osmd_moe_gate_up(const osmd_moe_args* a, osmd_stream s) {
  const int per = a->expert_table ? selection_per(a->expert_count) : 0;
  // gate/up's own selection reads final logits (the per-token router's);
  // router GEMM planes go through the select kernel.
  if (per > 0 && a->logit_planes != nullptr) return static_cast<int>(hipErrorInvalidValue);
  return launch_gate_up(gate_up_params(*a), a->tokens, per, static_cast<hipStream_t>(s));
}

int osmd_moe_down(const osmd_moe_args* a, osmd_stream s) {
  return launch_down(down_params(*a), a->tokens, static_cast<hipStream_t>(s));
}

int osmd_moe_experts(const osmd_moe_args* a, osmd_stream s) {
  const int r = osmd_moe_gate_up(a, s);
  return r != 0 ? r : osmd_moe_down(a, s);
}

size_t osmd_moe_parts_bytes(const osm_expert_geometry* g, uint32_t nslot, uint32_t tokens) {
  return static_cast<size_t>(tokens) * nslot * g->hidden * down_lanes_per_row(g->inter) * sizeof(float);
}

int osmd_moe_experts_parts(const osmd_moe_args* a, osmd_slot_list slots, float* parts, osmd_stream s) {
  const uint32_t nslot = a->top_k + ((a->flags & OSMD_MOE_SHARED) ? 1u : 0u);
  if (slots.count == 0u || slots.count > nslot || parts == nullptr || a->expert_table != nullptr)
    return static_cast<int>(hipErrorInvalidValue);
  for (uint32_t i = 0; i < slots.count; ++i) {
    const uint32_t j = static_cast<uint32_t>((i < 12u ? slots.lo >> (5u * i) : slots.hi >> (5u * (i - 12u))) & 31u);
    if (j >= nslot) return static_cast<int>(hipErrorInvalidValue);
  }
  const hipStream_t st = static_cast<hipStream_t>(s);
  GateUpParams gp = gate_up_params(*a);
  gp.list = slots;
  gp.src.nslot = nslot;
  int r = launch_gate_up(gp, a->tokens, 0, st);
  if (r != 0) return r;
  DownParams dp = down_params(*a);
  dp.list = slots;
  dp.parts = parts;
  return launch_down_mode<kDownParts>(dp, a->tokens, st);
}

int osmd_moe_combine(const osmd_moe_args* a, const float* parts, osmd_stream s) {
  if (parts == nullptr) return static_cast<int>(hipErrorInvalidValue);
  DownParams dp = down_params(*a);
  dp.parts = const_cast<float*>(parts);
  return launch_down_mode<kDownCombine>(dp, a->tokens, static_cast<hipStream_t>(s));
}

// From this many tokens on, the per-token decode selects in its own launch
// (one workgroup per token) and gate/up reads the published slot pointers:
// below, the launch costs more than the selection that every routed gate/up
// workgroup repeats (µs per layer step, Qwen3-Next shape, integrated /
// separate: 2 tokens 24.9 / 27.4, 8 tokens 54.6 / 55.8, 16 tokens 91-95 /
// 87.1, 32 tokens 162 / 145). The selection code is the same, so are the bits.
constexpr uint32_t kSeparateSelectMinTokens = 12;

int osmd_moe_decode(const osmd_moe_args* a, osmd_stream s) {
  if (a->expert_table && a->tokens >= kSeparateSelectMinTokens) {
    const int r = osmd_moe_route(a, s);
    if (r != 0) return r;
    osmd_moe_args b = *a;
    b.expert_table = nullptr;  // gate/up reads the slot pointers the selection published
    return osmd_moe_experts(&b, s);
  }
  // Otherwise, with a complete expert table the selection runs inside gate_up.
  const int r = a->expert_table ? osmd_moe_router(a, s) : osmd_moe_route(a, s);
  return r != 0 ? r : osmd_moe_experts(a, s);
}


#ifdef OSMD_TIMELINE
// The timeline slots (timeline build only): n <= 32 values of the 100 MHz
// clock, 0 for a slot no launch wrote since the library loaded.
int osmd_timeline_read(unsigned long long* out, uint32_t n) {
  if (out == nullptr || n > static_cast<uint32_t>(kTimelineSlots)) return static_cast<int>(hipErrorInvalidValue);
  return static_cast<int>(hipMemcpyFromSymbol(out, HIP_SYMBOL(osmd_timeline), n * sizeof(unsigned long long)));
}
#endif

int osmd_expert_forward(const uint8_t* blob, osm_expert_geometry g, const float* x, float* h,
                        float* out, osmd_stream s) {
  const hipStream_t st = static_cast<hipStream_t>(s);
  GateUpParams gp{};
  gp.g = g;
  gp.src = SlotSource{nullptr, blob, 1u};
  gp.rv.fallback = blob;
  gp.x = x;
  gp.h = h;
  int r = launch_gate_up(gp, 1u, 0, st);
  if (r != 0) return r;
  DownParams dp{};
  dp.g = g;
  dp.src = gp.src;
  dp.top_k = 1u;
  dp.weights = nullptr;
  dp.shared_gate = nullptr;
  dp.fallback = blob;
  dp.h = h;
  dp.residual = nullptr;
  dp.y = out;
  return launch_down(dp, 1u, st);
}

}  // extern "C"
