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

// Result of one token's selection, in LDS: ids and probabilities in pick
// order, and the blob of every expert the selecting wavefront looked up.
template <int PER>
struct Selection {
  uint32_t id[OSMD_MAX_TOP_K];
  float p[OSMD_MAX_TOP_K];
  const uint8_t* blob[kWave * PER];
};

// ---------------------------------------------------------------------------
// Top-k selection on one wavefront. Lane l owns experts [l*PER, l*PER+PER).
// Probabilities are the reference's: exp(logit - max) / sum over all experts
// (reference_ops.cpp:130-160). The order is the reference's too: probability
// descending, lower expert id first among equals (reference_ops.cpp:170-196:
// strict > on insertion, stable sort by probability). A probability is >= 0,
// so its bits order like its value; each lane sorts its experts on the key
// (bits, ~id), which is unique, and each round takes the largest head bits
// over the wave and the lowest lane holding them -- lanes own ascending id
// ranges, so that is the lowest id. With a table, the lane's blob pointers
// are loaded together with its logits and parked in LDS, so the pick's blob
// costs no dependent global load.
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
  if constexpr (PER == 8) {
    // Batcher's odd-even merge network: 19 comparators.
    constexpr int net[19][2] = {{0, 1}, {2, 3}, {4, 5}, {6, 7}, {0, 2}, {1, 3}, {4, 6},
                                {5, 7}, {1, 2}, {5, 6}, {0, 4}, {1, 5}, {2, 6}, {3, 7},
                                {2, 4}, {3, 5}, {1, 2}, {3, 4}, {5, 6}};
#pragma unroll
    for (int c = 0; c < 19; ++c) sort_step(k, n, net[c][0], net[c][1]);
  } else {
    // Odd-even transposition for the other widths.
#pragma unroll
    for (int round = 0; round < PER; ++round) {
#pragma unroll
      for (int j = round & 1; j + 1 < PER; j += 2) sort_step(k, n, j, j + 1);
    }
  }
}

template <int PER>
__device__ __forceinline__ void select_wave(const RouteView& rv, uint32_t t, uint32_t lane,
                                            Selection<PER>& out) {
  const uint32_t E = rv.expert_count;
  const uint32_t k = rv.top_k;
  const float* lg = rv.logits + static_cast<size_t>(t) * E;
  const uint32_t base = lane * PER;
  float p[PER];
  const uint8_t* tab[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t e = (base + j < E) ? base + j : E - 1u;  // clamped: every load in bounds
    p[j] = lg[e];
    tab[j] = rv.expert_table ? rv.expert_table[e] : nullptr;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (base + j >= E) p[j] = -INFINITY;
    mx = fmaxf(mx, p[j]);
  }
  mx = wave_max(mx);
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    p[j] = (base + j < E) ? expf(p[j] - mx) : 0.0f;
    sum += p[j];
  }
  sum = wave_sum(sum);
  // key: probability bits + 1, so 0 (experts past E, popped heads) ranks
  // below every real expert, even one whose probability is +0.
  uint32_t key[PER], nid[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    key[j] = (base + j < E) ? __float_as_uint(p[j] / sum) + 1u : 0u;
    nid[j] = ~(base + j);
    if (base + j < E) out.blob[base + j] = tab[j];
  }
  sort_lane<PER>(key, nid);

  // Unrolled: a rolled loop re-packs the loop-carried arrays every round.
#pragma unroll
  for (uint32_t r = 0; r < OSMD_MAX_TOP_K; ++r) {
    if (r < k) {
      const uint32_t m = wave_max_u32(key[0]);
      const unsigned long long ballot = __ballot(key[0] == m);
      const int wl = __ffsll(ballot) - 1;  // never empty: m is some lane's key
      uint32_t sid = ~static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(nid[0]), wl));
      sid = sid < E ? sid : E - 1u;  // a blob lookup always stays in the table
      if (lane == 0) {
        out.id[r] = sid;
        out.p[r] = __uint_as_float(m - 1u);
      }
      if (static_cast<int>(lane) == wl) {  // pop the head
#pragma unroll
        for (int j = 0; j + 1 < PER; ++j) {
          key[j] = key[j + 1];
          nid[j] = nid[j + 1];
        }
        key[PER - 1] = 0u;
        nid[PER - 1] = 0u;
      }
    }
  }
  // LDS writes of one wavefront are visible to its later LDS reads.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
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
template <int PER>
__device__ __forceinline__ void publish_selection(const RouteView& rv, uint32_t t, uint32_t lane,
                                                  const Selection<PER>& s) {
  const uint32_t k = rv.top_k;
  const uint32_t nslot = k + rv.has_shared;
  if (lane == 0) {
    float mass = 0.0f;
    for (uint32_t r = 0; r < k; ++r) mass = mass + s.p[r];
    for (uint32_t r = 0; r < k; ++r) {
      rv.ids[static_cast<size_t>(t) * k + r] = s.id[r];
      rv.weights[static_cast<size_t>(t) * k + r] = rv.norm_topk_prob ? s.p[r] / mass : s.p[r];
    }
    rv.mass[t] = mass;
  }
  if (lane < k)
    rv.slot_ptrs[static_cast<size_t>(t) * nslot + lane] = pick_blob(rv, s, lane);
  else if (lane == k && nslot > k)
    rv.slot_ptrs[static_cast<size_t>(t) * nslot + k] = rv.shared_expert;
}

template <int PER>
__global__ __launch_bounds__(64) void select_kernel(RouteView rv) {
  __shared__ Selection<PER> sel;
  select_wave<PER>(rv, blockIdx.x, threadIdx.x, sel);
  publish_selection(rv, blockIdx.x, threadIdx.x, sel);
}

// ---------------------------------------------------------------------------
// Router GEMV.
constexpr int kRouteWaves = 4;

template <int RD>
__device__ __forceinline__ void load8_row(const uint8_t* row, uint32_t c, float* w) {
  if constexpr (RD == OSM_META_F32) {
    const float4* p = reinterpret_cast<const float4*>(row) + c / 4u;
    const float4 a = p[0], b = p[1];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else {
    const uint4 q = ldg16(row + static_cast<size_t>(c) * 2u);
    const uint32_t v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (RD == OSM_META_BF16) {
        w[2 * i] = bf16_to_f32(v[i] & 0xFFFFu);
        w[2 * i + 1] = bf16_to_f32(v[i] >> 16);
      } else {
        w[2 * i] = f16_to_f32(v[i] & 0xFFFFu);
        w[2 * i + 1] = f16_to_f32(v[i] >> 16);
      }
    }
  }
}

template <int RD>
__global__ __launch_bounds__(256) void route_kernel(osmd_moe_args a) {
  extern __shared__ __align__(16) float xs[];  // [D] normalised input of this token
  __shared__ float red[kRouteWaves];
  const uint32_t t = blockIdx.y;
  const uint32_t D = a.geom.hidden;
  const uint32_t E = a.expert_count;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid % kWave;
  const uint32_t wave = tid / kWave;
  const uint32_t nrows = E + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  const uint32_t row = blockIdx.x * kRouteWaves + wave;
  constexpr size_t esz = (RD == OSM_META_F32) ? 4u : 2u;
  const uint8_t* wrow = row < E ? static_cast<const uint8_t*>(a.router) + static_cast<size_t>(row) * D * esz
                                : static_cast<const uint8_t*>(a.shared_gate_vec);

  // This wavefront's router row (hidden <= 8192 -> <= 16 loads per lane) and
  // all of x, issued together before anything waits.
  constexpr int kRowLoads = 16;
  float w[kRowLoads][8];
  if (row < nrows) {
#pragma unroll
    for (int u = 0; u < kRowLoads; ++u) {
      const uint32_t c = lane * 8u + u * 8u * kWave;
      if (c < D) load8_row<RD>(wrow, c, w[u]);
    }
  }
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
    // RMSNorm of the residual input (reference_ops.cpp:96-128), fused here so
    // every workgroup normalises its own copy instead of a separate launch.
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
      if (blockIdx.x == 0) xn4[i] = xv[u];
    }
  }
  __syncthreads();

  // One router row per wavefront; row E is the shared-expert gate vector.
  if (row < nrows) {
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < kRowLoads; ++u) {
      const uint32_t c = lane * 8u + u * 8u * kWave;
      if (c < D) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = fmaf(w[u][j], xs[c + j], acc);
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      if (row < E)
        a.logits[static_cast<size_t>(t) * E + row] = acc;
      else
        a.shared_gate[t] = 1.0f / (1.0f + expf(-acc));  // reference_ops.cpp:214-216
    }
  }
}

// ---------------------------------------------------------------------------
// gate/up + SwiGLU. Each wavefront owns kGuRowsPerWave consecutive rows of one
// slot; lane l reads 16-byte chunks l, l+64, ... of each row, so a wavefront
// load is 1 KB of contiguous packed weights. The lane's slice of x (and its
// sum) stays in registers for all rows. PER > 0: routed slots select their
// expert from the logits first (PER = experts per lane of the selection).
constexpr int kGuWaves = 4;
constexpr int kGuRowsPerWave = 4;

template <int META, int CPL, int PER>
__global__ __launch_bounds__(256) void gate_up_kernel(GateUpParams p) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t t = blockIdx.z;
  const uint32_t j = blockIdx.y;
  const uint32_t D = p.g.hidden, I = p.g.inter, G = p.g.group;
  const uint32_t nch = D / 32u;  // 16-byte chunks per row
  const uint32_t gpr = D / G;    // groups per row
  const float* x = p.x + static_cast<size_t>(t) * D;

  // Lanes past the row end (hidden < 64*32*CPL) read chunk nch-1 again and
  // zero their x slice, so every load is unconditional and in bounds.
  float xr[CPL][32];
  float xsum[CPL];
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

  const uint8_t* blob;
  if constexpr (PER > 0) {
    // Routed slot: wavefront 0 selects while the others wait with their x
    // slice loaded; block (0, 0) also publishes the selection.
    const RouteView& rv = p.rv;
    __shared__ Selection<PER> sel;
    __shared__ const uint8_t* s_blob;
    if (j < rv.top_k) {
      if (wave == 0) {
        select_wave<PER>(rv, t, lane, sel);
        if (blockIdx.x == 0 && j == 0) publish_selection(rv, t, lane, sel);
        if (lane == 0) s_blob = pick_blob(rv, sel, j);
      }
      __syncthreads();
      blob = s_blob;
    } else {
      blob = rv.shared_expert;
    }
  } else {
    blob = p.src.blob(t, j);
  }
  if (blob == nullptr) blob = p.rv.fallback;  // never dereference a null slot
  const osm_expert_offsets off = osm_expert_layout(p.g);

#pragma unroll
  for (int ci = 0; ci < CPL; ++ci) {
    xsum[ci] = 0.0f;
#pragma unroll
    for (int v = 0; v < 32; ++v) xsum[ci] += xr[ci][v];
  }

  const uint32_t r0 = (blockIdx.x * kGuWaves + wave) * kGuRowsPerWave;
  uint4 qg[kGuRowsPerWave][CPL], qu[kGuRowsPerWave][CPL];
  uint32_t sg[kGuRowsPerWave][CPL], bg[kGuRowsPerWave][CPL];
  uint32_t su[kGuRowsPerWave][CPL], bu[kGuRowsPerWave][CPL];
#pragma unroll
  for (int i = 0; i < kGuRowsPerWave; ++i) {
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
  for (int i = 0; i < kGuRowsPerWave; ++i) {
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
    if (lane == 0 && r < I)
      p.h[(static_cast<size_t>(t) * p.src.nslot + j) * I + r] = silu_mul(ga, ua);
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

template <int META, int LPR, int MAXS>
__global__ __launch_bounds__(kDownThreads) void down_kernel(DownParams p) {
  extern __shared__ __align__(16) float hs[];  // chunks, then chunk sums, then [2][rows] halves
  constexpr uint32_t kRowsPerGroup = kWave / LPR;
  constexpr uint32_t kRowsPerBlock = down_rows_per_block<LPR>();
  constexpr int kSlotsPerWave = (MAXS + 1) / 2;
  const uint32_t t = blockIdx.y;
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
  const uint32_t row = blockIdx.x * kRowsPerBlock + row_local;
  const bool active = row < D && c < nchd;
  const uint32_t rr = row < D ? row : D - 1u;
  const uint32_t cc = c < nchd ? c : nchd - 1u;
  const osm_expert_offsets off = osm_expert_layout(p.g);
  float* hsum = hs + static_cast<size_t>(nslot) * nchd * kChunkStride;
  float* halves = hsum + static_cast<size_t>(nslot) * nchd;

  // h does not depend on the slot pointers: its first batch is issued first.
  const float4* h4 = reinterpret_cast<const float4*>(p.h + static_cast<size_t>(t) * nslot * I);
  const uint32_t n4 = nslot * I / 4u;  // a multiple of 8 (I % 32 == 0)
  constexpr int kH4PerThread = 8;
  float4 hv[kH4PerThread];
#pragma unroll
  for (int u = 0; u < kH4PerThread; ++u) {
    const uint32_t f = u * kDownThreads + tid;
    hv[u] = f < n4 ? h4[f] : make_float4(0.f, 0.f, 0.f, 0.f);
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
    bp[i] = p.src.blob(t, js);
    if (js < p.top_k)
      w[i] = p.weights ? p.weights[static_cast<size_t>(t) * p.top_k + js] : 1.0f;
    else
      w[i] = p.shared_gate ? p.shared_gate[t] : 1.0f;
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
#pragma unroll
    for (int u = 0; u < kH4PerThread; ++u) {
      const uint32_t f = ((pass + 1) * kH4PerThread + u) * kDownThreads + tid;
      hv[u] = f < n4 ? h4[f] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
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
    const uint32_t orow = blockIdx.x * kRowsPerBlock + tid;
    if (orow < D) {
      const float v = halves[tid] + halves[kRowsPerBlock + tid];
      const size_t o = static_cast<size_t>(t) * D + orow;
      p.y[o] = p.residual ? p.residual[o] + v : v;
    }
  }
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
  const uint32_t rows_per_block = kGuWaves * kGuRowsPerWave;
  const dim3 grid((gp.g.inter + rows_per_block - 1) / rows_per_block, gp.src.nslot, tokens);
  switch (per) {
    case 0: gate_up_kernel<META, CPL, 0><<<grid, 256, 0, st>>>(gp); break;
    case 1: gate_up_kernel<META, CPL, 1><<<grid, 256, 0, st>>>(gp); break;
    case 2: gate_up_kernel<META, CPL, 2><<<grid, 256, 0, st>>>(gp); break;
    case 4: gate_up_kernel<META, CPL, 4><<<grid, 256, 0, st>>>(gp); break;
    case 8: gate_up_kernel<META, CPL, 8><<<grid, 256, 0, st>>>(gp); break;
    default: gate_up_kernel<META, CPL, 16><<<grid, 256, 0, st>>>(gp); break;
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

int selection_per(uint32_t experts) { return pow2_at_least((experts + kWave - 1) / kWave); }

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
    case 1: select_kernel<1><<<a.tokens, kWave, 0, st>>>(rv); break;
    case 2: select_kernel<2><<<a.tokens, kWave, 0, st>>>(rv); break;
    case 4: select_kernel<4><<<a.tokens, kWave, 0, st>>>(rv); break;
    case 8: select_kernel<8><<<a.tokens, kWave, 0, st>>>(rv); break;
    default: select_kernel<16><<<a.tokens, kWave, 0, st>>>(rv); break;
  }
  return launch_status();
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
  const uint32_t nslot = a->top_k + ((a->flags & OSMD_MOE_SHARED) ? 1u : 0u);
  GateUpParams gp;
  gp.g = a->geom;
  gp.src = SlotSource{a->slot_ptrs, nullptr, nslot};
  gp.rv = route_view(*a);
  gp.x = a->x_norm;
  gp.h = a->h;
  const int per = a->expert_table ? selection_per(a->expert_count) : 0;
  return launch_gate_up(gp, a->tokens, per, static_cast<hipStream_t>(s));
}

int osmd_moe_down(const osmd_moe_args* a, osmd_stream s) {
  const uint32_t nslot = a->top_k + ((a->flags & OSMD_MOE_SHARED) ? 1u : 0u);
  DownParams dp;
  dp.g = a->geom;
  dp.src = SlotSource{a->slot_ptrs, nullptr, nslot};
  dp.top_k = a->top_k;
  dp.weights = a->weights;
  dp.shared_gate = a->shared_gate;
  dp.fallback = a->fallback_blob;
  dp.h = a->h;
  dp.residual = (a->flags & OSMD_MOE_RESIDUAL) ? a->x : nullptr;
  dp.y = a->y;
  return launch_down(dp, a->tokens, static_cast<hipStream_t>(s));
}

int osmd_moe_experts(const osmd_moe_args* a, osmd_stream s) {
  const int r = osmd_moe_gate_up(a, s);
  return r != 0 ? r : osmd_moe_down(a, s);
}

int osmd_moe_decode(const osmd_moe_args* a, osmd_stream s) {
  // With a complete expert table the selection runs inside gate_up.
  const int r = a->expert_table ? osmd_moe_router(a, s) : osmd_moe_route(a, s);
  return r != 0 ? r : osmd_moe_experts(a, s);
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
