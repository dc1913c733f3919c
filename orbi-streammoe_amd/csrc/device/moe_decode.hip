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
//                   logits by one wavefront of every routed workgroup so no
//                   workgroup waits on another, then the gate and up q4 GEMVs
//                   of every pick and of the shared expert with SwiGLU fused
//                   in the epilogue (shaders/q4_gemv.comp + shaders/swiglu.comp).
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
// one-wavefront select kernel runs after route_kernel instead, the host reads
// the ids and writes the slot pointers, and gate_up_kernel reads those.
#include "device_common.hpp"

namespace {

using namespace osmk;

constexpr uint32_t kMaxSlots = OSMD_MAX_TOP_K + 1u;

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

// What a routed wavefront needs to select its expert from the logits.
struct RouteView {
  const float* logits;                // [B, E]
  const float* planes;                // null, or `parts` planes [B][E + 1] of partial sums
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
};

struct GateUpParams {
  osm_expert_geometry g;
  SlotSource src;
  RouteView rv;
  const float* x;  // [B, D]
  float* h;        // [B, nslot, I]
};

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
};

// Top-k selection on one 256-thread workgroup. Thread i owns experts
// [i*PER, i*PER+PER). Probabilities are the reference's: exp(logit - max) /
// sum over all experts (reference_ops.cpp:130-160); the max and the sum
// combine the four wavefronts' reductions in a fixed order. The order is the
// reference's too: probability descending, lower expert id first among
// equals (reference_ops.cpp:170-196: strict > on insertion, stable sort by
// probability). A probability is >= 0, so its bits order like its value; the
// key is (bits + 1, ~id), unique per expert, and 0 for experts past E and
// popped entries (below every real expert, even one whose probability is
// +0). Each wavefront takes the top-k of its 64 * PER experts in k rounds
// (the largest lane head over the wavefront, the lowest lane holding it:
// lanes own ascending id ranges, so that is the lowest id). The 4k
// candidates are then ranked in one pass: as (key << 32) | ~id they are
// unique and order exactly as probability descending, id ascending, so a
// candidate's place is the number of candidates above it. With a table,
// each thread parks its experts' blob pointers in LDS, so a pick's blob
// costs no dependent global load.
constexpr uint32_t kSelThreads = 256;
constexpr uint32_t kSelWaves = kSelThreads / kWave;

// Result of one token's selection, in LDS: ids and probabilities in pick
// order, the blob of every expert, and the workgroup's reduction scratch.
template <int PER>
struct Selection {
  uint32_t id[OSMD_MAX_TOP_K];
  float p[OSMD_MAX_TOP_K];
  const uint8_t* blob[kSelThreads * PER];
  float red[2][kSelWaves];
  uint64_t cand[kSelWaves * OSMD_MAX_TOP_K];  // (key << 32) | ~id, wavefront-major
};

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

// Selection from this thread's logits p[j] of experts tid*PER + j (entries
// past E are ignored) and their table pointers. Every thread of the
// workgroup calls it; it ends with a barrier, after which out is complete.
template <int PER>
__device__ __forceinline__ void select_values(const RouteView& rv, float (&p)[PER],
                                              const uint8_t* const (&tab)[PER], Selection<PER>& out,
                                              uint64_t* mark = nullptr) {
  const uint32_t E = rv.expert_count;
  const uint32_t k = rv.top_k;
  const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const uint32_t base = tid * PER;
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (base + j >= E) p[j] = -INFINITY;
    mx = fmaxf(mx, p[j]);
  }
  mx = wave_max(mx);
  if (lane == 0) out.red[0][wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(out.red[0][0], out.red[0][1]), fmaxf(out.red[0][2], out.red[0][3]));
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    p[j] = (base + j < E) ? expf(p[j] - mx) : 0.0f;
    sum += p[j];
  }
  sum = wave_sum(sum);
  if (lane == 0) out.red[1][wave] = sum;
  __syncthreads();
  sum = ((out.red[1][0] + out.red[1][1]) + out.red[1][2]) + out.red[1][3];
  if (mark != nullptr && threadIdx.x == 0) mark[5] = static_cast<uint64_t>(wall_clock64());
  uint32_t key[PER], nid[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    key[j] = (base + j < E) ? __float_as_uint(p[j] / sum) + 1u : 0u;
    nid[j] = ~(base + j);
    if (base + j < E) out.blob[base + j] = tab[j];
  }
  sort_lane<PER>(key, nid);

  // This wavefront's top-k. Each round is branch-free (the pop is a select
  // on every lane) and lane r keeps round r's result, written out after the
  // last round. The loop stays rolled: one body, fetched once, instead of
  // k copies that each start with instruction-cache misses (the selection
  // runs on one workgroup, so its code is cold).
  uint32_t rk = 0u, ri = 0u;
#pragma unroll 1
  for (uint32_t r = 0; r < k; ++r) {
    {
      const uint32_t m = wave_max_u32(key[0]);
      const int wl = __ffsll(__ballot(key[0] == m)) - 1;  // never empty: m is some lane's key
      const uint32_t sid = ~static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(nid[0]), wl));
      rk = lane == r ? m : rk;
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
  }
  if (lane < k) out.cand[wave * k + lane] = (static_cast<uint64_t>(rk) << 32) | ~ri;
  __syncthreads();
  if (mark != nullptr && threadIdx.x == 0) mark[6] = static_cast<uint64_t>(wall_clock64());

  // Wavefront 0: each lane ranks one candidate against all of them (LDS
  // broadcast reads); the k best write their place. Candidates of key 0
  // (fewer than k experts in a wavefront) always have k real ones above.
  if (wave == 0) {
    const uint32_t nc = kSelWaves * k;
    const uint64_t mine = lane < nc ? out.cand[lane] : 0u;
    uint32_t rank = 0;
#pragma unroll 4
    for (uint32_t c = 0; c < nc; ++c) rank += out.cand[c] > mine ? 1u : 0u;
    if (lane < nc && rank < k) {
      const uint32_t id = ~static_cast<uint32_t>(mine);
      out.id[rank] = id < E ? id : E - 1u;  // a blob lookup always stays in the table
      out.p[rank] = __uint_as_float(static_cast<uint32_t>(mine >> 32) - 1u);
    }
  }
  __syncthreads();
}

// Loads token t's logits (and table pointers) and selects; every thread of
// the workgroup calls it.
template <int PER>
__device__ __forceinline__ void select_block(const RouteView& rv, uint32_t t, Selection<PER>& out) {
  const uint32_t E = rv.expert_count;
  const float* lg = rv.logits + static_cast<size_t>(t) * E;
  const uint32_t base = threadIdx.x * PER;
  float p[PER];
  const uint8_t* tab[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t e = (base + j < E) ? base + j : E - 1u;  // clamped: every load in bounds
    if (rv.planes != nullptr) {
      // Partial sums of the router GEMM's K ranges, added in plane order.
      const size_t ps = static_cast<size_t>(rv.tokens) * (E + 1u);
      const float* pl = rv.planes + static_cast<size_t>(t) * (E + 1u) + e;
      float v = pl[0];
      for (uint32_t part = 1; part < rv.parts; ++part) v += pl[part * ps];
      p[j] = v;
      if (base + j < E) rv.logits_out[static_cast<size_t>(t) * E + e] = v;
    } else {
      p[j] = lg[e];
    }
    tab[j] = rv.expert_table ? rv.expert_table[e] : nullptr;
  }
  if (rv.planes != nullptr && rv.has_shared && threadIdx.x == 0) {
    const size_t ps = static_cast<size_t>(rv.tokens) * (E + 1u);
    const float* pl = rv.planes + static_cast<size_t>(t) * (E + 1u) + E;
    float g = pl[0];
    for (uint32_t part = 1; part < rv.parts; ++part) g += pl[part * ps];
    rv.gate_out[t] = 1.0f / (1.0f + expf(-g));  // reference_ops.cpp:214-216
  }
  select_values<PER>(rv, p, tab, out);
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
// Threads tid <= k of the workgroup take part.
template <int PER>
__device__ __forceinline__ void publish_selection(const RouteView& rv, uint32_t t, uint32_t tid,
                                                  const Selection<PER>& s) {
  const uint32_t k = rv.top_k;
  const uint32_t nslot = k + rv.has_shared;
  if (tid == 0) {
    float mass = 0.0f;
    for (uint32_t r = 0; r < k; ++r) mass = mass + s.p[r];
    for (uint32_t r = 0; r < k; ++r) {
      rv.ids[static_cast<size_t>(t) * k + r] = s.id[r];
      rv.weights[static_cast<size_t>(t) * k + r] = rv.norm_topk_prob ? s.p[r] / mass : s.p[r];
    }
    rv.mass[t] = mass;
  }
  if (tid < k)
    rv.slot_ptrs[static_cast<size_t>(t) * nslot + tid] = pick_blob(rv, s, tid);
  else if (tid == k && nslot > k)
    rv.slot_ptrs[static_cast<size_t>(t) * nslot + k] = rv.shared_expert;
}

template <int PER>
__global__ __launch_bounds__(kSelThreads) void select_kernel(RouteView rv) {
  __shared__ Selection<PER> sel;
  select_block<PER>(rv, blockIdx.x, sel);
  publish_selection(rv, blockIdx.x, threadIdx.x, sel);
}

// ---------------------------------------------------------------------------
// Router GEMV. A wavefront owns one router row; lane l reads elements
// l*8 + 512u .. +8 (u = 0, 1, ...), kept as loaded until the FMA.
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

// Token t's input, RMS-normalised when the flags ask for it
// (reference_ops.cpp:96-128), into xs[D] in LDS; write_norm also stores it to
// x_norm. Every workgroup that needs x normalises its own copy: the values
// are the same bits everywhere. 256 threads, hidden <= 8192.
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
    const float4* w4 = reinterpret_cast<const float4*>(a.norm_weight);
#pragma unroll
    for (int u = 0; u < kX4PerThread; ++u) {
      const uint32_t i = tid + u * 256u;
      if (i < n4) {
        const float4 nw = w4[i];
        xv[u].x = xv[u].x * (scale * nw.x);
        xv[u].y = xv[u].y * (scale * nw.y);
        xv[u].z = xv[u].z * (scale * nw.z);
        xv[u].w = xv[u].w * (scale * nw.w);
      }
    }
  }
  float4* xs4 = reinterpret_cast<float4*>(xs);
  float4* xn4 = reinterpret_cast<float4*>(a.x_norm + static_cast<size_t>(t) * D);
#pragma unroll
  for (int u = 0; u < kX4PerThread; ++u) {
    const uint32_t i = tid + u * 256u;
    if (i < n4) {
      xs4[i] = xv[u];
      if (write_norm) xn4[i] = xv[u];
    }
  }
  __syncthreads();
}

// Router rows blk*4 .. blk*4+3 of token t (row E is the shared-expert gate
// vector): logits, or the sigmoid shared gate (reference_ops.cpp:214-216).
// RCH loads of 8 elements per lane cover hidden <= 512 * RCH.
// also(row, value) runs on lane 0 after each row's store (row E: the gate).
template <int RD, int RCH, typename Also>
__device__ __forceinline__ void route_block(const osmd_moe_args& a, uint32_t t, uint32_t blk, float* xs,
                                            Also&& also) {
  const uint32_t D = a.geom.hidden;
  const uint32_t E = a.expert_count;
  const uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const uint32_t nrows = E + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  const uint32_t row = blk * kRouteWaves + wave;
  constexpr size_t esz = (RD == OSM_META_F32) ? 4u : 2u;
  // The row is issued before x, so both are in flight together.
  Raw8<RD> w[RCH];
  if (row < nrows) {
    if constexpr (RD == OSM_ROUTER_AFFINE_Q8) {
      const Q8Row qr = row < E ? q8_row(a.router, E, row, D, a.router_group)
                               : q8_row(a.shared_gate_vec, 1u, 0u, D, a.router_group);
#pragma unroll
      for (int u = 0; u < RCH; ++u) {
        const uint32_t c = lane * 8u + u * 8u * kWave;
        if (c < D) load_q8x8(qr, c, w[u]);
      }
    } else {
      const uint8_t* wrow = row < E ? static_cast<const uint8_t*>(a.router) + static_cast<size_t>(row) * D * esz
                                    : static_cast<const uint8_t*>(a.shared_gate_vec);
#pragma unroll
      for (int u = 0; u < RCH; ++u) {
        const uint32_t c = lane * 8u + u * 8u * kWave;
        if (c < D) load_raw8<RD>(wrow, c, w[u]);
      }
    }
  }
  stage_x(a, t, xs, blk == 0);
  if (row < nrows) {
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < RCH; ++u) {
      const uint32_t c = lane * 8u + u * 8u * kWave;
      if (c < D) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = fmaf(raw8_get<RD>(w[u], j), xs[c + j], acc);
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      const float v = row < E ? acc : 1.0f / (1.0f + expf(-acc));
      *(row < E ? a.logits + static_cast<size_t>(t) * E + row : a.shared_gate + t) = v;
      also(row, v);
    }
  }
}

template <int RD>
__global__ __launch_bounds__(256) void route_kernel(osmd_moe_args a) {
  extern __shared__ __align__(16) float xs[];  // [D] normalised input of this token
  route_block<RD, 16>(a, blockIdx.y, blockIdx.x, xs, [](uint32_t, float) {});
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
                                             const uint8_t* blob, const float (&xr)[CPL][32], Store&& store) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t D = p.g.hidden, I = p.g.inter, G = p.g.group;
  const uint32_t nch = D / 32u;  // 16-byte chunks per row
  const uint32_t gpr = D / G;    // groups per row
  const osm_expert_offsets off = osm_expert_layout(p.g);
  float xsum[CPL];
#pragma unroll
  for (int ci = 0; ci < CPL; ++ci) {
    xsum[ci] = 0.0f;
#pragma unroll
    for (int v = 0; v < 32; ++v) xsum[ci] += xr[ci][v];
  }

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
    ga = wave_sum(ga);
    ua = wave_sum(ua);
    const uint32_t r = r0 + i;
    if (lane == 0 && r < I) store((static_cast<size_t>(t) * p.src.nslot + j) * I + r, silu_mul(ga, ua));
  }
}

template <int META, int CPL, int PER, int ROWS>
__global__ __launch_bounds__(256) void gate_up_kernel(GateUpParams p) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t t = blockIdx.z;
  const uint32_t j = blockIdx.y;
  const uint32_t D = p.g.hidden;
  float xr[CPL][32];
  load_xr<CPL>(p.x + static_cast<size_t>(t) * D, D / 32u, lane, xr);

  const uint8_t* blob;
  if constexpr (PER > 0) {
    // Routed slot: the workgroup selects with its x slices loaded; block
    // (0, 0) also publishes the selection.
    const RouteView& rv = p.rv;
    __shared__ Selection<PER> sel;
    if (j < rv.top_k) {
      select_block<PER>(rv, t, sel);
      if (blockIdx.x == 0 && j == 0) publish_selection(rv, t, threadIdx.x, sel);
      blob = pick_blob(rv, sel, j);
    } else {
      blob = rv.shared_expert;
    }
  } else {
    blob = p.src.blob(t, j);
  }
  if (blob == nullptr) blob = p.rv.fallback;  // never dereference a null slot
  gate_up_rows<META, CPL, ROWS>(p, t, j, blockIdx.x, blob, xr, [&](size_t i, float v) { p.h[i] = v; });
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

// ---------------------------------------------------------------------------
// Single-launch decode: how its workgroups hand data to each other.
//
// A one-token decode with every expert resident runs as one grid: router
// workgroups (4 router rows each), one selector, gate/up workgroups (the
// shared expert's first), down workgroups. A workgroup waits only on
// workgroups with lower indices, which the dispatcher starts first.
//
// Everything handed from one workgroup to another -- the logits and shared
// gate, the selection, h -- travels as 8-byte elements that carry the launch
// number next to the value, each written with one agent-scope atomic store
// and read with agent-scope atomic loads (coherent across the XCDs' separate
// L2 caches; no L2 write-back or invalidate is involved). A reader re-reads
// an element until its tag is this launch's number: the read is the wait.
// The selector writes one record per slot (tag, expert id, weight), in eight
// copies, so the readers on the XCD that workgroup b runs on (b % 8) share
// one copy. h is 22 KB that every down workgroup reads, too much to re-read
// while waiting: each gate/up workgroup, once its h stores are complete
// (s_waitcnt vmcnt(0) in every wavefront, then a barrier), adds 1 to its
// slot's done counter, and down workgroups poll the slot counters (one lane
// each) before reading h, whose tags they still check. h rotates through
// four buffers (launch number mod 4) and is first read with ordinary loads,
// served by the reader's L2 after one miss per XCD: each 128-byte line of it
// is written whole by one workgroup with write-through stores, so a miss
// fetches it complete, and a line some L2 still holds from four launches
// back carries an old tag and is read again with coherent loads.
//
// Launch numbers come from a per-workgroup counter, read and advanced once
// per launch, so nothing is reset between launches. Every wait gives up after
// kSpinLimit re-reads and sets the sticky error word; the workgroup then
// goes on with what it read.
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr uint32_t kRecordCopies = 8;
constexpr uint32_t kRecordSlots = 16;
constexpr uint32_t kSharedId = 0xFFFFu;  // record id of the shared expert
constexpr uint32_t kHBuffers = 4;        // h buffers, by launch number mod 4

__device__ __forceinline__ void store_tagged(uint64_t* p, uint32_t epoch, float v) {
  __hip_atomic_store(p, (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_tagged(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_current(uint64_t v, uint32_t epoch) {
  return static_cast<uint32_t>(v >> 32) == epoch;
}
__device__ __forceinline__ float tagged_value(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v)); }
// Selection record: tag (low 16 bits of the launch number), expert id, weight.
__device__ __forceinline__ uint64_t record_of(uint32_t epoch, uint32_t id, float w) {
  return (static_cast<uint64_t>(epoch & 0xFFFFu) << 48) | (static_cast<uint64_t>(id & 0xFFFFu) << 32) |
         __float_as_uint(w);
}
__device__ __forceinline__ bool record_current(uint64_t v, uint32_t epoch) {
  return static_cast<uint32_t>(v >> 48) == (epoch & 0xFFFFu);
}

// Byte offsets of the handshake buffer's parts (the error word is at 0).
struct FusedLayout {
  size_t launch, logits, record, done, h, bytes;
};
__host__ __device__ inline size_t round_up128(size_t n) { return (n + 127u) & ~static_cast<size_t>(127u); }
__host__ __device__ inline FusedLayout fused_layout(uint32_t grid, uint32_t experts, uint32_t nslot,
                                                    uint32_t inter) {
  FusedLayout l;
  l.launch = 128u;
  l.logits = l.launch + round_up128(static_cast<size_t>(grid) * 4u);
  l.record = l.logits + round_up128((static_cast<size_t>(experts) + 1u) * 8u);
  l.done = l.record + static_cast<size_t>(kRecordCopies) * kRecordSlots * 8u;
  l.h = l.done + static_cast<size_t>(kRecordSlots) * 128u;  // one counter per slot, 128 bytes apart
  l.bytes = l.h + kHBuffers * round_up128(static_cast<size_t>(nslot) * inter * 8u);
  return l;
}

struct FusedWaits {
  uint32_t* err;
  uint32_t epoch;
  const uint64_t* record;  // this workgroup's copy
  const uint64_t* h;       // this launch's tagged h [nslot][I]
  const uint32_t* done;    // per-slot gate/up done counters, 128 bytes apart
  uint32_t gu_per_slot;    // gate/up workgroups per slot
  uint64_t* mark;          // this workgroup's timeline slots, or null
  const RouteView* rv;
  const uint8_t** s_blob;  // LDS: blob of each slot
  float* s_w;              // LDS: weight of each slot
};

// Optional timeline of a single launch: thread 0 stamps the steady clock into
// slot i of its workgroup's 8 (slot 7: the hardware id of its compute unit).
__device__ __forceinline__ void stamp(uint64_t* mark, int i) {
  if (mark != nullptr && threadIdx.x == 0) mark[i] = static_cast<uint64_t>(wall_clock64());
}

// Whether a wait should stop: out of spins, or another wait already gave up.
__device__ __forceinline__ bool give_up(uint32_t spin, uint32_t* err) {
  if (spin >= kSpinLimit ||
      ((spin & 255u) == 255u && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)) {
    __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  }
  return false;
}

// Lanes r < n of the calling wavefront read record slot r until it is this
// launch's; returns the lane's record.
__device__ __forceinline__ uint64_t read_record(const FusedWaits& fw, uint32_t n) {
  const uint32_t lane = threadIdx.x % kWave;
  uint64_t v = 0;
  for (uint32_t spin = 0;; ++spin) {
    bool ok = true;
    if (lane < n) {
      v = load_tagged(fw.record + lane);
      ok = record_current(v, fw.epoch);
    }
    if (__all(ok)) break;
    if (give_up(spin, fw.err)) break;
    __builtin_amdgcn_s_sleep(2);
  }
  return v;
}

// s_waitcnt immediate with vmcnt = 0 and the other counters not waited on
// (gfx9 encoding: vmcnt [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
constexpr int kWaitVmcnt0 = 0x0F70;

// Lanes c < n of the calling wavefront poll counter c (128 bytes apart from
// `first`) until it reaches `target`; the others wait with them.
__device__ __forceinline__ void wait_counters(const uint32_t* first, uint32_t n, uint32_t target, uint32_t* err) {
  const uint32_t lane = threadIdx.x % kWave;
  for (uint32_t spin = 0;; ++spin) {
    bool ok = true;
    if (lane < n) {
      const uint32_t v = __hip_atomic_load(const_cast<uint32_t*>(first) + lane * 32u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
      ok = static_cast<int32_t>(v - target) >= 0;
    }
    if (__all(ok)) break;
    if (give_up(spin, err)) break;
    __builtin_amdgcn_s_sleep(4);
  }
}

// Blob of a record: the table entry of its expert (the fallback for a null
// entry or an id out of range), or the shared expert.
__device__ __forceinline__ const uint8_t* record_blob(const RouteView& rv, uint64_t rec) {
  const uint32_t id = static_cast<uint32_t>(rec >> 32) & 0xFFFFu;
  if (id == kSharedId) return rv.shared_expert;
  const uint8_t* b = id < rv.expert_count ? rv.expert_table[id] : nullptr;
  return b ? b : rv.fallback;
}

// down + weighted accumulate for rows blk * rows_per_block ... of token t.
// FUSED: the slot pointers and weights are read once the selection is out,
// and h once every gate/up workgroup is done; the down weights are already
// in flight while h is awaited.
template <int META, int LPR, int MAXS, bool FUSED>
__device__ __forceinline__ void down_block(const DownParams& p, uint32_t t, uint32_t blk, float* hs,
                                           const FusedWaits& fw) {
  constexpr uint32_t kRowsPerGroup = kWave / LPR;
  constexpr uint32_t kRowsPerBlock = down_rows_per_block<LPR>();
  constexpr int kSlotsPerWave = (MAXS + 1) / 2;
  const uint32_t D = p.g.hidden, I = p.g.inter, G = p.g.group;
  const uint32_t nslot = p.src.nslot;
  const uint32_t nchd = I / 32u;
  const uint32_t gpr = I / G;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid % kWave;
  const uint32_t wave = tid / kWave;
  const uint32_t rg = wave & 1u;    // row group
  const uint32_t half = wave >> 1;  // slots half, half + 2, ...
  const uint32_t c = lane % LPR;
  const uint32_t row_local = rg * kRowsPerGroup + lane / LPR;
  const uint32_t row = blk * kRowsPerBlock + row_local;
  const bool active = row < D && c < nchd;
  const uint32_t rr = row < D ? row : D - 1u;
  const uint32_t cc = c < nchd ? c : nchd - 1u;
  const osm_expert_offsets off = osm_expert_layout(p.g);
  float* hsum = hs + static_cast<size_t>(nslot) * nchd * kChunkStride;
  float* halves = hsum + static_cast<size_t>(nslot) * nchd;

  const float4* h4 = reinterpret_cast<const float4*>(p.h + static_cast<size_t>(t) * nslot * I);
  const uint32_t n4 = nslot * I / 4u;  // a multiple of 8 (I % 32 == 0)
  constexpr int kH4PerThread = 8;
  float4 hv[kH4PerThread];
  auto load_h = [&](uint32_t pass) {
    if constexpr (FUSED) {
      // h comes from the gate/up workgroups of this launch: an ordinary
      // read first, then coherent re-reads until every element this thread
      // stages carries the launch number.
      for (uint32_t spin = 0;; ++spin) {
        bool ok = true;
#pragma unroll
        for (int u = 0; u < kH4PerThread; ++u) {
          const uint32_t f = (pass * kH4PerThread + u) * kDownThreads + tid;
          if (f < n4) {
            const uint64_t* src = fw.h + static_cast<size_t>(t) * nslot * I + static_cast<size_t>(f) * 4u;
            uint64_t v0, v1, v2, v3;
            if (spin == 0) {
              const uint4 a = *reinterpret_cast<const uint4*>(src);
              const uint4 c = *reinterpret_cast<const uint4*>(src + 2);
              v0 = (static_cast<uint64_t>(a.y) << 32) | a.x;
              v1 = (static_cast<uint64_t>(a.w) << 32) | a.z;
              v2 = (static_cast<uint64_t>(c.y) << 32) | c.x;
              v3 = (static_cast<uint64_t>(c.w) << 32) | c.z;
            } else {
              v0 = load_tagged(src);
              v1 = load_tagged(src + 1);
              v2 = load_tagged(src + 2);
              v3 = load_tagged(src + 3);
            }
            ok = ok && tag_current(v0, fw.epoch) && tag_current(v1, fw.epoch) && tag_current(v2, fw.epoch) &&
                 tag_current(v3, fw.epoch);
            hv[u] = make_float4(tagged_value(v0), tagged_value(v1), tagged_value(v2), tagged_value(v3));
          } else {
            hv[u] = make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
        if (ok || give_up(spin, fw.err)) break;
        if (spin > 0) __builtin_amdgcn_s_sleep(2);
      }
    } else {
#pragma unroll
      for (int u = 0; u < kH4PerThread; ++u) {
        const uint32_t f = (pass * kH4PerThread + u) * kDownThreads + tid;
        hv[u] = f < n4 ? h4[f] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  if constexpr (FUSED) {
    // Each slot's blob and weight from this launch's selection record.
    if (wave == 0) {
      const uint64_t rec = read_record(fw, nslot);
      if (lane < nslot) {
        fw.s_blob[lane] = record_blob(*fw.rv, rec);
        fw.s_w[lane] = __uint_as_float(static_cast<uint32_t>(rec));
      }
    }
    __syncthreads();
    stamp(fw.mark, 1);
  } else {
    load_h(0);  // h does not depend on the slot pointers: its first batch is issued first
  }

  // This wavefront's slots: pointers and weights (uniform loads), then the
  // packed chunk and metadata of each, with no branch between them. Slots
  // past nslot and null pointers read a valid blob with weight 0.
  const uint8_t* bp[kSlotsPerWave];
  float w[kSlotsPerWave];
#pragma unroll
  for (int i = 0; i < kSlotsPerWave; ++i) {
    const uint32_t j = half + 2u * i;
    const uint32_t js = j < nslot ? j : 0u;
    if constexpr (FUSED) {
      bp[i] = fw.s_blob[js];
      w[i] = fw.s_w[js];
    } else {
      bp[i] = p.src.blob(t, js);
      if (js < p.top_k)
        w[i] = p.weights ? p.weights[static_cast<size_t>(t) * p.top_k + js] : 1.0f;
      else
        w[i] = p.shared_gate ? p.shared_gate[t] : 1.0f;
    }
    if (j >= nslot || bp[i] == nullptr) w[i] = 0.0f;
    if (bp[i] == nullptr) bp[i] = p.fallback;
  }
  uint4 q[kSlotsPerWave];
  uint32_t sb[kSlotsPerWave], bb[kSlotsPerWave];
  const size_t qo = (static_cast<size_t>(rr) * nchd + cc) * 16u;
  const size_t gi = static_cast<size_t>(rr) * gpr + (cc * 32u) / G;
#pragma unroll
  for (int i = 0; i < kSlotsPerWave; ++i) {
    q[i] = ldg16(bp[i] + off.down_q + qo);
    sb[i] = meta_bits<META>(bp[i] + off.down_s, gi);
    bb[i] = meta_bits<META>(bp[i] + off.down_b, gi);
  }
  if constexpr (FUSED) {
    stamp(fw.mark, 2);
    if (wave == 0) wait_counters(fw.done, nslot, fw.epoch * fw.gu_per_slot, fw.err);
    __syncthreads();
    load_h(0);
    stamp(fw.mark, 3);
  }

  // Stage h and its per-chunk sums: 8 consecutive threads hold one 32-float
  // chunk, summed with DPP within the lane group.
  for (uint32_t pass = 0;; ++pass) {
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
    if ((pass + 1) * kH4PerThread * kDownThreads >= n4) break;
    load_h(pass + 1);
  }
  __syncthreads();

  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < kSlotsPerWave; ++i) {
    const uint32_t j = half + 2u * i;
    const uint32_t js = j < nslot ? j : 0u;
    const uint32_t chunk = js * nchd + cc;
    const float part = meta_widen<META>(sb[i]) * nib_dot32(q[i], hs + chunk * kChunkStride) +
                       meta_widen<META>(bb[i]) * hsum[chunk];
    acc += w[i] * part;
    // Keep each slot's LDS reads next to their use.
    __builtin_amdgcn_sched_barrier(0);
  }
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
  if constexpr (FUSED) stamp(fw.mark, 4);
}

template <int META, int LPR, int MAXS>
__global__ __launch_bounds__(kDownThreads) void down_kernel(DownParams p) {
  extern __shared__ __align__(16) float hs[];  // chunks, then chunk sums, then [2][rows] halves
  down_block<META, LPR, MAXS, false>(p, blockIdx.y, blockIdx.x, hs, FusedWaits{});
}

// ---------------------------------------------------------------------------
// The single-launch decode kernel (one token, every expert resident). Blocks
// [0, nr) route, then ngu gate/up blocks (the shared expert's first), then
// the down blocks. Each phase runs the code of the three-kernel decode above,
// so both give the same bits.
constexpr int kFusedRouteLoads = 4;  // hidden <= 2048
constexpr int kFusedMaxSlots = 12;
constexpr int kFusedPer = 2;  // experts <= 512

struct FusedParams {
  osmd_moe_args a;
  GateUpParams gp;
  DownParams dp;
  uint32_t* sync;   // handshake buffer (fused_layout)
  uint64_t* trace;  // [grid][8] timeline, or null
  uint32_t nr, ngu, gu_blocks_per_slot, grid;
};

template <int RD, int META, int LPR>
__global__ __launch_bounds__(256) void fused_decode_kernel(FusedParams f) {
  extern __shared__ __align__(16) float lds[];  // x of the token, or the down staging
  __shared__ uint32_t s_epoch;
  __shared__ Selection<kFusedPer> sel;
  __shared__ const uint8_t* s_blob[kFusedMaxSlots];
  __shared__ float s_w[kFusedMaxSlots];
  const uint32_t b = blockIdx.x;
  const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  uint8_t* base = reinterpret_cast<uint8_t*>(f.sync);
  const FusedLayout lay = fused_layout(f.grid, f.a.expert_count, f.gp.src.nslot, f.a.geom.inter);
  uint32_t* err = f.sync;
  uint32_t* launch = reinterpret_cast<uint32_t*>(base + lay.launch);
  uint64_t* tl = reinterpret_cast<uint64_t*>(base + lay.logits);  // tagged logits, then the gate
  uint64_t* rec = reinterpret_cast<uint64_t*>(base + lay.record);
  uint64_t* th = reinterpret_cast<uint64_t*>(base + lay.h);  // then + (e % 4) buffers, below
  uint32_t* done = reinterpret_cast<uint32_t*>(base + lay.done);
  uint64_t* mark = f.trace ? f.trace + static_cast<size_t>(b) * 8u : nullptr;
  stamp(mark, 0);
  if (mark != nullptr && tid == 0) mark[7] = __smid();
  // This launch's number, from the workgroup's own launch counter.
  if (tid == 0) {
    const uint32_t e = __hip_atomic_load(launch + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    __hip_atomic_store(launch + b, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_epoch = e;
  }
  const RouteView& rv = f.gp.rv;
  const uint32_t k = f.a.top_k, E = f.a.expert_count;
  const uint32_t nslot = f.gp.src.nslot;

  if (b < f.nr) {
    // Router rows; stage_x's barrier makes s_epoch visible before the stores.
    route_block<RD, kFusedRouteLoads>(f.a, 0u, b, lds,
                                      [&](uint32_t row, float v) { store_tagged(tl + row, s_epoch, v); });
    stamp(mark, 1);
    return;
  }
  __syncthreads();
  const uint32_t e = s_epoch;
  th += static_cast<size_t>(e % kHBuffers) * (round_up128(static_cast<size_t>(nslot) * f.a.geom.inter * 8u) / 8u);
  if (b == f.nr) {
    // The selector: every thread reads its experts' tagged logits (thread 0
    // also the gate) until the whole workgroup has this launch's, selects,
    // and threads r < nslot write the records.
    const uint32_t bs = tid * kFusedPer;
    float pv[kFusedPer];
    const uint8_t* tab[kFusedPer];
#pragma unroll
    for (int j = 0; j < kFusedPer; ++j) {
      tab[j] = rv.expert_table[(bs + j < E) ? bs + j : E - 1u];
      // Loaded here, while the logits are still being computed: left alone,
      // the compiler issues these loads after the wait below.
      asm volatile("" : : "v"(tab[j]));
    }
    const bool has_shared = nslot > k;
    for (uint32_t spin = 0;; ++spin) {
      bool ok = true;
#pragma unroll
      for (int j = 0; j < kFusedPer; ++j) {
        const uint64_t v = load_tagged(tl + ((bs + j < E) ? bs + j : E - 1u));
        ok = ok && tag_current(v, e);
        pv[j] = tagged_value(v);
      }
      if (has_shared && tid == 0) {
        const uint64_t v = load_tagged(tl + E);
        ok = ok && tag_current(v, e);
        s_w[0] = tagged_value(v);
      }
      // Both exits are decided for the whole workgroup (the loop holds barriers).
      if (__syncthreads_and(ok)) break;
      if (__syncthreads_or(tid == 0 && give_up(spin, err))) break;
      __builtin_amdgcn_s_sleep(2);
    }
    const float gate = s_w[0];
    stamp(mark, 1);
    select_values<kFusedPer>(rv, pv, tab, sel, mark);
    stamp(mark, 2);
    // Records: weights as the per-token kernels publish them (p / mass in
    // pick order when renormalised), the shared expert last with its gate.
    if (tid < nslot) {
      float mass = 0.0f;
      for (uint32_t r = 0; r < k; ++r) mass = mass + sel.p[r];
      const uint64_t my = tid < k ? record_of(e, sel.id[tid], rv.norm_topk_prob ? sel.p[tid] / mass : sel.p[tid])
                                  : record_of(e, kSharedId, gate);
#pragma unroll
      for (uint32_t c = 0; c < kRecordCopies; ++c)
        __hip_atomic_store(rec + c * kRecordSlots + tid, my, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    stamp(mark, 3);
    publish_selection(rv, 0u, tid, sel);  // ids, weights, mass, slot pointers for the host
    stamp(mark, 4);
    return;
  }
  FusedWaits fw{err, e, rec + (b % kRecordCopies) * kRecordSlots, th, done, f.gu_blocks_per_slot, mark, &rv,
                s_blob, s_w};
  const uint32_t g = b - f.nr - 1u;
  if (g < f.ngu) {
    const uint32_t si = g / f.gu_blocks_per_slot, blk = g % f.gu_blocks_per_slot;
    const uint32_t j = (f.a.flags & OSMD_MOE_SHARED) ? (si == 0 ? k : si - 1u) : si;
    stage_x(f.a, 0u, lds, false);
    stamp(mark, 1);
    float xr[1][32];
    load_xr<1>(lds, f.a.geom.hidden / 32u, lane, xr);
    const uint8_t* blob;
    if (j < k) {
      if (wave == 0) {
        FusedWaits one = fw;
        one.record += j;
        const uint64_t r = read_record(one, 1u);
        if (lane == 0) s_blob[0] = record_blob(rv, r);
      }
      __syncthreads();
      blob = s_blob[0];
    } else {
      blob = f.a.shared_expert;
    }
    if (blob == nullptr) blob = f.a.fallback_blob;
    stamp(mark, 2);
    gate_up_rows<META, 1, kGuRowsOneToken>(f.gp, 0u, j, blk, blob, xr,
                                           [&](size_t i, float v) { store_tagged(th + i, e, v); });
    stamp(mark, 3);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // this wavefront's h stores are complete
    __syncthreads();
    if (tid == 0) __hip_atomic_fetch_add(done + j * 32u, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    stamp(mark, 4);
    return;
  }
  down_block<META, LPR, kFusedMaxSlots, true>(f.dp, 0u, g - f.ngu, lds, fw);
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
  const dim3 grid((gp.g.inter + rows_per_block - 1) / rows_per_block, gp.src.nslot, tokens);
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

template <int META, int LPR>
int launch_down_lpr(const DownParams& dp, uint32_t tokens, hipStream_t st) {
  constexpr uint32_t rows_per_block = down_rows_per_block<LPR>();
  const dim3 grid((dp.g.hidden + rows_per_block - 1) / rows_per_block, tokens);
  const size_t lds = down_lds_bytes(dp.g.inter, dp.src.nslot, rows_per_block);
  const uint32_t n = dp.src.nslot;
  if (n <= 2u)
    down_kernel<META, LPR, 2><<<grid, kDownThreads, lds, st>>>(dp);
  else if (n <= 4u)
    down_kernel<META, LPR, 4><<<grid, kDownThreads, lds, st>>>(dp);
  else if (n <= 8u)
    down_kernel<META, LPR, 8><<<grid, kDownThreads, lds, st>>>(dp);
  else if (n <= 12u)
    down_kernel<META, LPR, 12><<<grid, kDownThreads, lds, st>>>(dp);
  else
    down_kernel<META, LPR, kMaxSlots + 1><<<grid, kDownThreads, lds, st>>>(dp);
  return launch_status();
}

template <int META>
int launch_down_meta(const DownParams& dp, uint32_t tokens, hipStream_t st) {
  switch (pow2_at_least(dp.g.inter / 32u)) {
    case 1: return launch_down_lpr<META, 1>(dp, tokens, st);
    case 2: return launch_down_lpr<META, 2>(dp, tokens, st);
    case 4: return launch_down_lpr<META, 4>(dp, tokens, st);
    case 8: return launch_down_lpr<META, 8>(dp, tokens, st);
    case 16: return launch_down_lpr<META, 16>(dp, tokens, st);
    case 32: return launch_down_lpr<META, 32>(dp, tokens, st);
    default: return launch_down_lpr<META, 64>(dp, tokens, st);
  }
}

int launch_down(const DownParams& dp, uint32_t tokens, hipStream_t st) {
  switch (dp.g.meta_dtype) {
    case OSM_META_F32: return launch_down_meta<OSM_META_F32>(dp, tokens, st);
    case OSM_META_F16: return launch_down_meta<OSM_META_F16>(dp, tokens, st);
    default: return launch_down_meta<OSM_META_BF16>(dp, tokens, st);
  }
}

// Experts per lane of a selection: 8 up to 512 experts, 16 beyond. One width
// for every expert count in a range keeps the order of the wavefront sums of
// the softmax the same in every kernel that selects (the per-token kernels,
// the select kernel, the single launch), so they publish the same bits.
int selection_per(uint32_t experts) { return experts <= 2u * kSelThreads ? 2 : 4; }

template <int RD>
int launch_route_rd(const osmd_moe_args& a, hipStream_t st) {
  const uint32_t nrows = a.expert_count + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  const dim3 grid((nrows + kRouteWaves - 1) / kRouteWaves, a.tokens);
  const size_t lds = static_cast<size_t>(a.geom.hidden) * sizeof(float);
  route_kernel<RD><<<grid, 256, lds, st>>>(a);
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

// Shape of the single-launch grid.
struct FusedShape {
  uint32_t nr, bps, ngu, nd, grid, lpr;
  size_t lds;
};

FusedShape fused_shape(const osmd_moe_args& a) {
  FusedShape f;
  const uint32_t shared = (a.flags & OSMD_MOE_SHARED) ? 1u : 0u;
  const uint32_t nslot = a.top_k + shared;
  const uint32_t D = a.geom.hidden, I = a.geom.inter;
  f.nr = (a.expert_count + shared + kRouteWaves - 1) / kRouteWaves;
  const uint32_t gu_rows = kGuWaves * kGuRowsOneToken;
  f.bps = (I + gu_rows - 1) / gu_rows;
  f.ngu = nslot * f.bps;
  f.lpr = static_cast<uint32_t>(pow2_at_least(I / 32u));
  const uint32_t rows = 2u * (kWave / f.lpr);
  f.nd = (D + rows - 1) / rows;
  f.grid = f.nr + 1u + f.ngu + f.nd;
  const size_t down = down_lds_bytes(I, nslot, rows);
  f.lds = down > D * sizeof(float) ? down : D * sizeof(float);
  return f;
}

bool fused_supported(const osmd_moe_args& a) {
  const uint32_t nslot = a.top_k + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  const uint32_t D = a.geom.hidden, I = a.geom.inter;
  const uint32_t lpr = static_cast<uint32_t>(pow2_at_least(I / 32u));
  return a.tokens == 1u && a.expert_table != nullptr && a.slot_ptrs != nullptr &&
         (a.router_dtype == OSM_META_BF16 || a.router_dtype == OSM_META_F32) && D % 32u == 0u &&
         D <= 512u * kFusedRouteLoads && I % 32u == 0u && (lpr == 4u || lpr == 8u || lpr == 16u) &&
         a.expert_count <= kSelThreads * kFusedPer && nslot <= static_cast<uint32_t>(kFusedMaxSlots) &&
         fused_shape(a).lds <= 65536u;
}

template <int RD, int META>
int launch_fused_meta(const FusedParams& f, const FusedShape& sh, hipStream_t st) {
  switch (sh.lpr) {
    case 4: fused_decode_kernel<RD, META, 4><<<sh.grid, 256, sh.lds, st>>>(f); break;
    case 8: fused_decode_kernel<RD, META, 8><<<sh.grid, 256, sh.lds, st>>>(f); break;
    default: fused_decode_kernel<RD, META, 16><<<sh.grid, 256, sh.lds, st>>>(f); break;
  }
  return launch_status();
}

template <int RD>
int launch_fused_rd(const FusedParams& f, const FusedShape& sh, hipStream_t st) {
  switch (f.a.geom.meta_dtype) {
    case OSM_META_F32: return launch_fused_meta<RD, OSM_META_F32>(f, sh, st);
    case OSM_META_F16: return launch_fused_meta<RD, OSM_META_F16>(f, sh, st);
    default: return launch_fused_meta<RD, OSM_META_BF16>(f, sh, st);
  }
}

GateUpParams gate_up_params(const osmd_moe_args& a) {
  const uint32_t nslot = a.top_k + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  GateUpParams gp;
  gp.g = a.geom;
  gp.src = SlotSource{a.slot_ptrs, nullptr, nslot};
  gp.rv = route_view(a);
  gp.x = a.x_norm;
  gp.h = a.h;
  return gp;
}

DownParams down_params(const osmd_moe_args& a) {
  const uint32_t nslot = a.top_k + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  DownParams dp;
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
  return launch_gate_up(gate_up_params(*a), a->tokens, per, static_cast<hipStream_t>(s));
}

int osmd_moe_down(const osmd_moe_args* a, osmd_stream s) {
  return launch_down(down_params(*a), a->tokens, static_cast<hipStream_t>(s));
}

int osmd_moe_experts(const osmd_moe_args* a, osmd_stream s) {
  const int r = osmd_moe_gate_up(a, s);
  return r != 0 ? r : osmd_moe_down(a, s);
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

int osmd_moe_fused_supported(const osmd_moe_args* a) { return fused_supported(*a) ? 1 : 0; }

size_t osmd_moe_fused_sync_bytes(const osmd_moe_args* a) {
  const uint32_t nslot = a->top_k + ((a->flags & OSMD_MOE_SHARED) ? 1u : 0u);
  return fused_layout(fused_shape(*a).grid, a->expert_count, nslot, a->geom.inter).bytes;
}

size_t osmd_moe_fused_error_offset(void) { return 0u; }

int osmd_moe_fused_shape(const osmd_moe_args* a, uint32_t* out4) {
  const FusedShape sh = fused_shape(*a);
  out4[0] = sh.nr;
  out4[1] = sh.ngu;
  out4[2] = sh.nd;
  out4[3] = sh.grid;
  return 0;
}

int osmd_moe_decode_fused(const osmd_moe_args* a, uint32_t* sync, uint64_t* trace, osmd_stream s) {
  if (!fused_supported(*a) || sync == nullptr) return static_cast<int>(hipErrorInvalidValue);
  const FusedShape sh = fused_shape(*a);
  FusedParams f;
  f.a = *a;
  f.gp = gate_up_params(*a);
  f.dp = down_params(*a);
  f.sync = sync;
  f.trace = trace;
  f.nr = sh.nr;
  f.ngu = sh.ngu;
  f.gu_blocks_per_slot = sh.bps;
  f.grid = sh.grid;
  const hipStream_t st = static_cast<hipStream_t>(s);
  return a->router_dtype == OSM_META_F32 ? launch_fused_rd<OSM_META_F32>(f, sh, st)
                                         : launch_fused_rd<OSM_META_BF16>(f, sh, st);
}

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
