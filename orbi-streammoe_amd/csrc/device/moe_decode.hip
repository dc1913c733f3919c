// moe_decode.hip -- fused gfx950 kernels for one routed-MoE sublayer decode.
//
// The reference runs this path as 56 blocking dispatches per token-layer with
// routing on the host (src/model/routed_moe.cpp:254-430).
// Here it is three stream-ordered kernels and no host round trip:
//
//   route_kernel    RMSNorm (optional) + router GEMV + shared-gate dot; the
//                   last workgroup to finish runs softmax + top-k selection
//                   (src/cpu/reference_ops.cpp:130-212, src/model/qwen_router.cpp:
//                   11-94) and resolves each pick to its expert blob.
//   gate_up_kernel  gate and up q4 GEMVs of every pick and of the shared
//                   expert, SwiGLU fused in the epilogue
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
#include "device_common.hpp"

namespace {

using namespace osmk;

constexpr uint32_t kMaxSlots = OSMD_MAX_TOP_K + 1u;

// Blob of slot j for token t: resolved pointers when routing ran, else one
// fixed expert (the single-expert operator).
struct SlotSource {
  const uint8_t* const* ptrs;  // [B, nslot] or null
  const uint8_t* single;
  uint32_t nslot;
  __device__ __forceinline__ const uint8_t* blob(uint32_t t, uint32_t j) const {
    return ptrs ? ptrs[static_cast<size_t>(t) * nslot + j] : single;
  }
};

struct GateUpParams {
  osm_expert_geometry g;
  SlotSource src;
  const float* x;  // [B, D]
  float* h;        // [B, nslot, I]
};

struct DownParams {
  osm_expert_geometry g;
  SlotSource src;
  uint32_t top_k;            // slots [0, top_k) take weights[], the rest shared_gate
  const float* weights;      // [B, top_k] or null (weight 1)
  const float* shared_gate;  // [B] or null (weight 1)
  const float* h;            // [B, nslot, I]
  const float* residual;     // [B, D] or null
  float* y;                  // [B, D]
};

// ---------------------------------------------------------------------------
// Router.
constexpr int kRouteWaves = 4;

template <int RD>
__device__ __forceinline__ void load8_row(const uint8_t* row, uint32_t c, float* w) {
  if constexpr (RD == OSM_META_F32) {
    const float4* p = reinterpret_cast<const float4*>(row) + c / 4u;
    const float4 a = p[0], b = p[1];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else {
    const uint4 q = *reinterpret_cast<const uint4*>(row + static_cast<size_t>(c) * 2u);
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

// Softmax + top-k on one wavefront. Lane l owns experts [l*PER, l*PER+PER),
// so "lowest lane holding the maximum, then lowest index within the lane" is
// "lowest expert id" -- the reference's tie rule (reference_ops.cpp:170-196:
// strict > on insertion, stable sort by probability descending).
template <int PER>
__device__ void select_top_k(const osmd_moe_args& a, uint32_t t, uint32_t lane) {
  const uint32_t E = a.expert_count;
  const uint32_t k = a.top_k;
  const uint32_t nslot = k + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  const float* lg = a.logits + static_cast<size_t>(t) * E;
  const uint32_t base = lane * PER;
  float p[PER];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    // Logits come from other workgroups (other XCDs): read them at agent scope.
    p[j] = (base + j < E) ? __hip_atomic_load(lg + base + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                          : -INFINITY;
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
#pragma unroll
  for (int j = 0; j < PER; ++j) p[j] = (base + j < E) ? p[j] / sum : -1.0f;

  uint32_t sel_id[OSMD_MAX_TOP_K];
  float sel_p[OSMD_MAX_TOP_K];
#pragma unroll
  for (uint32_t r = 0; r < OSMD_MAX_TOP_K; ++r) {
    sel_id[r] = 0u;
    sel_p[r] = 0.0f;
    if (r < k) {
      float bp = -1.0f;
      int bj = 0;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        if (p[j] > bp) {
          bp = p[j];
          bj = j;
        }
      }
      const float m = wave_max(bp);
      const unsigned long long ballot = __ballot(bp == m);
      const int wl = __ffsll(ballot) - 1;
      const int wj = __shfl(bj, wl, kWave);
      if (static_cast<int>(lane) == wl) {
#pragma unroll
        for (int j = 0; j < PER; ++j)
          if (j == wj) p[j] = -1.0f;
      }
      sel_id[r] = static_cast<uint32_t>(wl) * PER + static_cast<uint32_t>(wj);
      sel_p[r] = m;
    }
  }
  if (lane == 0) {
    // Selected mass in pick order, then optional renormalisation
    // (qwen_router.cpp:72-91).
    float mass = 0.0f;
#pragma unroll
    for (uint32_t r = 0; r < OSMD_MAX_TOP_K; ++r)
      if (r < k) mass = mass + sel_p[r];
    const bool norm = a.norm_topk_prob != 0u;
#pragma unroll
    for (uint32_t r = 0; r < OSMD_MAX_TOP_K; ++r) {
      if (r < k) {
        a.ids[static_cast<size_t>(t) * k + r] = sel_id[r];
        a.weights[static_cast<size_t>(t) * k + r] = norm ? sel_p[r] / mass : sel_p[r];
      }
    }
    a.mass[t] = mass;
  }
  // Resolve each pick to its blob so later kernels skip the table lookup.
  if (lane < k) {
    uint32_t id = 0u;
#pragma unroll
    for (uint32_t r = 0; r < OSMD_MAX_TOP_K; ++r)
      if (r == lane) id = sel_id[r];
    a.slot_ptrs[static_cast<size_t>(t) * nslot + lane] = a.expert_table ? a.expert_table[id] : nullptr;
  } else if (lane == k && nslot > k) {
    a.slot_ptrs[static_cast<size_t>(t) * nslot + k] = a.shared_expert;
  }
}

template <int RD, int PER>
__global__ __launch_bounds__(256) void route_kernel(osmd_moe_args a) {
  extern __shared__ float xs[];  // [D] normalised input of this token
  __shared__ float red[kRouteWaves];
  __shared__ uint32_t last_s;
  const uint32_t t = blockIdx.y;
  const uint32_t D = a.geom.hidden;
  const uint32_t E = a.expert_count;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid % kWave;
  const uint32_t wave = tid / kWave;
  const float* x = a.x + static_cast<size_t>(t) * D;

  float ss = 0.0f;
  for (uint32_t i = tid; i < D; i += blockDim.x) {
    const float v = x[i];
    xs[i] = v;
    ss += v * v;
  }
  if (a.flags & OSMD_MOE_RMSNORM) {
    // RMSNorm of the residual input (reference_ops.cpp:96-128), fused here so
    // every workgroup normalises its own copy instead of a separate launch.
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kRouteWaves; ++w) tot += red[w];
    const float scale = 1.0f / sqrtf(tot / static_cast<float>(D) + a.rms_eps);
    for (uint32_t i = tid; i < D; i += blockDim.x) xs[i] = xs[i] * (scale * a.norm_weight[i]);
  }
  __syncthreads();
  if (blockIdx.x == 0)
    for (uint32_t i = tid; i < D; i += blockDim.x) a.x_norm[static_cast<size_t>(t) * D + i] = xs[i];

  // One router row per wavefront; row E is the shared-expert gate vector.
  const uint32_t nrows = E + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  const uint32_t row = blockIdx.x * kRouteWaves + wave;
  if (row < nrows) {
    constexpr size_t esz = (RD == OSM_META_F32) ? 4u : 2u;
    const uint8_t* wrow = row < E
                              ? static_cast<const uint8_t*>(a.router) + static_cast<size_t>(row) * D * esz
                              : static_cast<const uint8_t*>(a.shared_gate_vec);
    float acc = 0.0f;
#pragma unroll 4
    for (uint32_t c = lane * 8u; c < D; c += 8u * kWave) {
      float w[8];
      load8_row<RD>(wrow, c, w);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = fmaf(w[j], xs[c + j], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      if (row < E)
        a.logits[static_cast<size_t>(t) * E + row] = acc;
      else
        a.shared_gate[t] = 1.0f / (1.0f + expf(-acc));  // reference_ops.cpp:214-216
    }
  }

  // The last workgroup of this token to finish selects the experts. The
  // ticket wraps back to zero on that last increment, so the counter is
  // ready for the next launch without a separate reset.
  __threadfence();
  __syncthreads();
  if (tid == 0) last_s = (atomicInc(&a.counter[t], gridDim.x - 1u) == gridDim.x - 1u) ? 1u : 0u;
  __syncthreads();
  if (last_s == 0u) return;
  __threadfence();
  if (wave != 0) return;
  select_top_k<PER>(a, t, lane);
}

// ---------------------------------------------------------------------------
// gate/up + SwiGLU. Each wavefront owns kGuRowsPerWave consecutive rows of one
// slot; lane l reads 16-byte chunks l, l+64, ... of each row, so a wavefront
// load is 1 KB of contiguous packed weights. The lane's slice of x (and its
// sum) stays in registers for all rows.
constexpr int kGuWaves = 4;
constexpr int kGuRowsPerWave = 4;

template <int META, int CPL>
__global__ __launch_bounds__(256) void gate_up_kernel(GateUpParams p) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t t = blockIdx.z;
  const uint32_t j = blockIdx.y;
  const uint32_t D = p.g.hidden, I = p.g.inter, G = p.g.group;
  const uint32_t nch = D / 32u;  // 16-byte chunks per row
  const uint32_t gpr = D / G;    // groups per row
  const uint8_t* blob = p.src.blob(t, j);
  const uint32_t r0 = (blockIdx.x * kGuWaves + wave) * kGuRowsPerWave;
  if (blob == nullptr) {  // expert not resident: contributes nothing
    if (lane < kGuRowsPerWave && r0 + lane < I)
      p.h[(static_cast<size_t>(t) * p.src.nslot + j) * I + r0 + lane] = 0.0f;
    return;
  }
  const osm_expert_offsets off = osm_expert_layout(p.g);
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
    xsum[ci] = 0.0f;
#pragma unroll
    for (int v = 0; v < 32; ++v) xsum[ci] += xr[ci][v];
  }

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
// (I/32 chunks); a wavefront covers 64/LPR rows per load. Every slot's h sits
// in LDS together with its per-chunk sums, so the weighted sum over picks and
// the shared expert is one deterministic register accumulation per row --
// no atomics and no separate accumulate launches.
constexpr int kDownWaves = 2;

template <int META, int LPR, int MAXS>
__global__ __launch_bounds__(128) void down_kernel(DownParams p) {
  extern __shared__ float hs[];  // [nslot, I] then [nslot, I/32] chunk sums
  const uint32_t t = blockIdx.y;
  const uint32_t D = p.g.hidden, I = p.g.inter, G = p.g.group;
  const uint32_t nslot = p.src.nslot;
  const uint32_t nchd = I / 32u;
  const uint32_t gpr = I / G;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid % kWave;
  const uint32_t wave = tid / kWave;
  constexpr uint32_t kRowsPerWave = kWave / LPR;
  const uint32_t c = lane % LPR;
  const uint32_t row = (blockIdx.x * kDownWaves + wave) * kRowsPerWave + lane / LPR;
  const bool active = row < D && c < nchd;
  const uint32_t rr = row < D ? row : D - 1u;
  const uint32_t cc = c < nchd ? c : nchd - 1u;
  const osm_expert_offsets off = osm_expert_layout(p.g);

  // Issue every slot's packed chunk and metadata first (clamped, so no
  // divergent branch forces a wait between them), then stage h in LDS while
  // they are in flight. Slots past nslot re-read the last slot with weight 0.
  uint4 q[MAXS];
  uint32_t sb[MAXS], bb[MAXS];
  float w[MAXS];
#pragma unroll
  for (uint32_t j = 0; j < MAXS; ++j) {
    const uint32_t js = j < nslot ? j : nslot - 1u;
    const uint8_t* blob = p.src.blob(t, js);
    q[j] = make_uint4(0u, 0u, 0u, 0u);
    sb[j] = bb[j] = 0u;
    if (blob != nullptr) {
      q[j] = ldg16(blob + off.down_q + (static_cast<size_t>(rr) * nchd + cc) * 16u);
      const size_t gi = static_cast<size_t>(rr) * gpr + (cc * 32u) / G;
      sb[j] = meta_bits<META>(blob + off.down_s, gi);
      bb[j] = meta_bits<META>(blob + off.down_b, gi);
    }
    if (j >= nslot || blob == nullptr)
      w[j] = 0.0f;
    else if (j < p.top_k)
      w[j] = p.weights ? p.weights[static_cast<size_t>(t) * p.top_k + j] : 1.0f;
    else
      w[j] = p.shared_gate ? p.shared_gate[t] : 1.0f;
  }

  const float* h = p.h + static_cast<size_t>(t) * nslot * I;
  for (uint32_t i = tid; i < nslot * I; i += blockDim.x) hs[i] = h[i];
  __syncthreads();
  float* hsum = hs + nslot * I;
  for (uint32_t i = tid; i < nslot * nchd; i += blockDim.x) {
    const float* v = hs + (i / nchd) * I + (i % nchd) * 32u;
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e) s += v[e];
    hsum[i] = s;
  }
  __syncthreads();

  float acc = 0.0f;
#pragma unroll
  for (uint32_t j = 0; j < MAXS; ++j) {
    if (j < nslot) {
      const float part = meta_widen<META>(sb[j]) * nib_dot32(q[j], hs + j * I + cc * 32u) +
                         meta_widen<META>(bb[j]) * hsum[j * nchd + cc];
      acc += w[j] * part;
    }
    // Keep each slot's 32 LDS reads next to their use.
    __builtin_amdgcn_sched_barrier(0);
  }
  if (!active) acc = 0.0f;
#pragma unroll
  for (int m = LPR / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, kWave);
  if (c == 0 && row < D) {
    const size_t o = static_cast<size_t>(t) * D + row;
    p.y[o] = p.residual ? p.residual[o] + acc : acc;
  }
}

// ---------------------------------------------------------------------------
// Host-side launchers.

int pow2_at_least(uint32_t v) {
  int p = 1;
  while (static_cast<uint32_t>(p) < v) p <<= 1;
  return p;
}

template <int META>
int launch_gate_up_meta(const GateUpParams& gp, uint32_t tokens, hipStream_t st) {
  const uint32_t nch = gp.g.hidden / 32u;
  const uint32_t rows_per_block = kGuWaves * kGuRowsPerWave;
  const dim3 grid((gp.g.inter + rows_per_block - 1) / rows_per_block, gp.src.nslot, tokens);
  if (nch <= 64u)
    gate_up_kernel<META, 1><<<grid, 256, 0, st>>>(gp);
  else if (nch <= 128u)
    gate_up_kernel<META, 2><<<grid, 256, 0, st>>>(gp);
  else
    gate_up_kernel<META, 4><<<grid, 256, 0, st>>>(gp);
  return launch_status();
}

int launch_gate_up(const GateUpParams& gp, uint32_t tokens, hipStream_t st) {
  switch (gp.g.meta_dtype) {
    case OSM_META_F32: return launch_gate_up_meta<OSM_META_F32>(gp, tokens, st);
    case OSM_META_F16: return launch_gate_up_meta<OSM_META_F16>(gp, tokens, st);
    default: return launch_gate_up_meta<OSM_META_BF16>(gp, tokens, st);
  }
}

template <int META, int LPR>
int launch_down_lpr(const DownParams& dp, uint32_t tokens, hipStream_t st) {
  constexpr uint32_t rows_per_block = kDownWaves * (kWave / LPR);
  const dim3 grid((dp.g.hidden + rows_per_block - 1) / rows_per_block, tokens);
  const uint32_t nchd = dp.g.inter / 32u;
  const size_t lds = static_cast<size_t>(dp.src.nslot) * (dp.g.inter + nchd) * sizeof(float);
  const uint32_t n = dp.src.nslot;
  if (n <= 1u)
    down_kernel<META, LPR, 1><<<grid, kDownWaves * kWave, lds, st>>>(dp);
  else if (n <= 4u)
    down_kernel<META, LPR, 4><<<grid, kDownWaves * kWave, lds, st>>>(dp);
  else if (n <= 8u)
    down_kernel<META, LPR, 8><<<grid, kDownWaves * kWave, lds, st>>>(dp);
  else if (n <= 12u)
    down_kernel<META, LPR, 12><<<grid, kDownWaves * kWave, lds, st>>>(dp);
  else
    down_kernel<META, LPR, kMaxSlots><<<grid, kDownWaves * kWave, lds, st>>>(dp);
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

template <int RD>
int launch_route_rd(const osmd_moe_args& a, hipStream_t st) {
  const uint32_t nrows = a.expert_count + ((a.flags & OSMD_MOE_SHARED) ? 1u : 0u);
  const dim3 grid((nrows + kRouteWaves - 1) / kRouteWaves, a.tokens);
  const size_t lds = static_cast<size_t>(a.geom.hidden) * sizeof(float);
  switch (pow2_at_least((a.expert_count + kWave - 1) / kWave)) {
    case 1: route_kernel<RD, 1><<<grid, 256, lds, st>>>(a); break;
    case 2: route_kernel<RD, 2><<<grid, 256, lds, st>>>(a); break;
    case 4: route_kernel<RD, 4><<<grid, 256, lds, st>>>(a); break;
    case 8: route_kernel<RD, 8><<<grid, 256, lds, st>>>(a); break;
    default: route_kernel<RD, 16><<<grid, 256, lds, st>>>(a); break;
  }
  return launch_status();
}

}  // namespace

extern "C" {

int osmd_moe_route(const osmd_moe_args* a, osmd_stream s) {
  const hipStream_t st = static_cast<hipStream_t>(s);
  switch (a->router_dtype) {
    case OSM_META_F32: return launch_route_rd<OSM_META_F32>(*a, st);
    case OSM_META_F16: return launch_route_rd<OSM_META_F16>(*a, st);
    default: return launch_route_rd<OSM_META_BF16>(*a, st);
  }
}

int osmd_moe_decode(const osmd_moe_args* a, osmd_stream s) {
  const int r = osmd_moe_route(a, s);
  return r != 0 ? r : osmd_moe_experts(a, s);
}

int osmd_moe_gate_up(const osmd_moe_args* a, osmd_stream s) {
  const uint32_t nslot = a->top_k + ((a->flags & OSMD_MOE_SHARED) ? 1u : 0u);
  GateUpParams gp;
  gp.g = a->geom;
  gp.src = SlotSource{a->slot_ptrs, nullptr, nslot};
  gp.x = a->x_norm;
  gp.h = a->h;
  return launch_gate_up(gp, a->tokens, static_cast<hipStream_t>(s));
}

int osmd_moe_down(const osmd_moe_args* a, osmd_stream s) {
  const uint32_t nslot = a->top_k + ((a->flags & OSMD_MOE_SHARED) ? 1u : 0u);
  DownParams dp;
  dp.g = a->geom;
  dp.src = SlotSource{a->slot_ptrs, nullptr, nslot};
  dp.top_k = a->top_k;
  dp.weights = a->weights;
  dp.shared_gate = a->shared_gate;
  dp.h = a->h;
  dp.residual = (a->flags & OSMD_MOE_RESIDUAL) ? a->x : nullptr;
  dp.y = a->y;
  return launch_down(dp, a->tokens, static_cast<hipStream_t>(s));
}

int osmd_moe_experts(const osmd_moe_args* a, osmd_stream s) {
  const int r = osmd_moe_gate_up(a, s);
  return r != 0 ? r : osmd_moe_down(a, s);
}

int osmd_expert_forward(const uint8_t* blob, osm_expert_geometry g, const float* x, float* h,
                        float* out, osmd_stream s) {
  const hipStream_t st = static_cast<hipStream_t>(s);
  GateUpParams gp;
  gp.g = g;
  gp.src = SlotSource{nullptr, blob, 1u};
  gp.x = x;
  gp.h = h;
  int r = launch_gate_up(gp, 1u, st);
  if (r != 0) return r;
  DownParams dp;
  dp.g = g;
  dp.src = gp.src;
  dp.top_k = 1u;
  dp.weights = nullptr;
  dp.shared_gate = nullptr;
  dp.h = h;
  dp.residual = nullptr;
  dp.y = out;
  return launch_down(dp, 1u, st);
}

}  // extern "C"
