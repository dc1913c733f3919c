// q4_ops.hip -- standalone gfx950 kernels behind the reference's single-op
// surface: affine q4 dequant (shaders/q4_dequant.comp), q4 GEMV
// (shaders/q4_gemv.comp), nibble unpack, SwiGLU (shaders/swiglu.comp),
// weighted accumulate (shaders/weighted_accumulate.comp) and RMSNorm
// (shaders/rmsnorm.comp). These serve arbitrary shapes and any group size;
// the routed-MoE hot path uses the fused kernels in moe_decode.hip.
#include "device_common.hpp"

namespace {

using namespace osmk;

// One thread per packed word; each writes its 8 dequantized columns. The
// value is rounded as the reference rounds it (src/cpu/reference_ops.cpp:57-59):
// scale*q first, then + bias, with no fused multiply-add.
template <int META>
__global__ void q4_dequant_kernel(const uint32_t* __restrict__ packed,
                                  const void* __restrict__ scales,
                                  const void* __restrict__ biases, uint32_t rows,
                                  uint32_t packed_cols, uint32_t group,
                                  float* __restrict__ out) {
#pragma clang fp contract(off)
  const size_t total = static_cast<size_t>(rows) * packed_cols;
  const uint32_t groups = packed_cols * 8u / group;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t wi = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; wi < total;
       wi += stride) {
    const uint32_t r = static_cast<uint32_t>(wi / packed_cols);
    const uint32_t wc = static_cast<uint32_t>(wi - static_cast<size_t>(r) * packed_cols);
    const uint32_t w = packed[wi];
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t col = wc * 8u + j;
      const size_t gi = static_cast<size_t>(r) * groups + col / group;
      const float q = static_cast<float>((w >> (4 * j)) & 0xFu);
      const float prod = meta_at<META>(scales, gi) * q;
      v[j] = prod + meta_at<META>(biases, gi);
    }
    float4* o = reinterpret_cast<float4*>(out + wi * 8u);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// One wavefront per output row, lanes striding over packed words. When a word
// lies inside one group the reference GEMV algebra applies
// (shaders/q4_gemv.comp:42-59): scale * sum(q*x) + bias * sum(x); otherwise
// each nibble is dequantized and multiplied.
template <int META>
__global__ void q4_gemv_kernel(const uint32_t* __restrict__ packed,
                               const void* __restrict__ scales,
                               const void* __restrict__ biases, uint32_t out_dim,
                               uint32_t packed_cols, uint32_t group,
                               const float* __restrict__ x, float* __restrict__ y) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= out_dim) return;
  const uint32_t groups = packed_cols * 8u / group;
  const uint32_t* prow = packed + static_cast<size_t>(row) * packed_cols;
  const size_t gbase = static_cast<size_t>(row) * groups;
  float acc = 0.0f;
  if (group % 8u == 0u) {
    for (uint32_t w = lane; w < packed_cols; w += kWave) {
      const uint32_t col0 = w * 8u;
      const float* xc = x + col0;
      float xs = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) xs += xc[j];
      const size_t gi = gbase + col0 / group;
      acc += meta_at<META>(scales, gi) * nib_dot8(prow[w], xc) + meta_at<META>(biases, gi) * xs;
    }
  } else {
    for (uint32_t w = lane; w < packed_cols; w += kWave) {
      const uint32_t word = prow[w];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t col = w * 8u + j;
        const size_t gi = gbase + col / group;
        const float q = static_cast<float>((word >> (4 * j)) & 0xFu);
        acc += (meta_at<META>(scales, gi) * q + meta_at<META>(biases, gi)) * x[col];
      }
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

__global__ void unpack_kernel(const uint32_t* __restrict__ packed, size_t words,
                              uint8_t* __restrict__ out) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += stride) {
    // Byte j of the 8-byte output is nibble j of the word, low nibble first.
    const uint32_t w = packed[i];
    uint32_t b0 = 0, b1 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      b0 |= ((w >> (4 * j)) & 0xFu) << (8 * j);
      b1 |= ((w >> (4 * j + 16)) & 0xFu) << (8 * j);
    }
    reinterpret_cast<uint2*>(out)[i] = make_uint2(b0, b1);
  }
}

__global__ void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u,
                              float* __restrict__ out, size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = silu_mul(g[i], u[i]);
}

// acc[i] += weight * src[i], rounded as the reference's scalar loop rounds.
__global__ void weighted_accumulate_kernel(const float* __restrict__ src, float weight,
                                           float* __restrict__ acc, size_t n) {
#pragma clang fp contract(off)
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    acc[i] = acc[i] + weight * src[i];
}

// One workgroup per row: block-wide sum of squares, then
// v * (1/sqrt(mean + eps) * w) (reference_ops.cpp:112-127).
__global__ void rms_norm_kernel(const float* __restrict__ in, const float* __restrict__ w,
                                float* __restrict__ out, uint32_t dim, float eps) {
  __shared__ float partial[16];
  __shared__ float scale_s;
  const float* row = in + static_cast<size_t>(blockIdx.x) * dim;
  float* orow = out + static_cast<size_t>(blockIdx.x) * dim;
  float ss = 0.0f;
  for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) ss += row[i] * row[i];
  ss = wave_sum(ss);
  const uint32_t wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) partial[wave] = ss;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.0f;
    for (uint32_t i = 0; i < blockDim.x / kWave; ++i) t += partial[i];
    scale_s = 1.0f / sqrtf(t / static_cast<float>(dim) + eps);
  }
  __syncthreads();
  const float scale = scale_s;
  for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x)
    orow[i] = row[i] * (scale * (w ? w[i] : 1.0f));
}

unsigned grid_for(size_t n, unsigned block) {
  size_t g = (n + block - 1) / block;
  if (g == 0) g = 1;
  if (g > 65535u * 4u) g = 65535u * 4u;
  return static_cast<unsigned>(g);
}

// ---- affine q4 quantizer (src/conversion/single_expert_pilot.cpp:276-358) --
// Pass 1, one thread per (row, group): min, max, scale = range / 15 (1 when
// flat), bias = min, the group's error bound (scale * 0.5001 + 1e-6, or 1e-6
// when flat); flags bit 0 marks a non-finite weight. Pass 2, one
// thread per packed word: q = clamp(round-half-away((v - bias) / scale), 0,
// 15) per nibble (an overflowed range gives NaN, mapped to 0), the
// reconstruction error against the group bound (flags bit 1), and per-block
// error maximum and sum for the statistics. Every operation rounds on its
// own, as the reference's scalar loop does.
constexpr int kQuantThreads = 256;

__global__ void quant_groups_kernel(const float* __restrict__ v, size_t rows, size_t cols, size_t group,
                                    float* __restrict__ scales, float* __restrict__ biases,
                                    float* __restrict__ bounds, uint32_t* __restrict__ flags) {
#pragma clang fp contract(off)
  const size_t groups = cols / group;
  const size_t n = rows * groups;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float* g = v + (i / groups) * cols + (i % groups) * group;
    float lo = INFINITY, hi = -INFINITY;
    bool finite = true;
    for (size_t j = 0; j < group; ++j) {
      const float x = g[j];
      finite = finite && isfinite(x);
      lo = fminf(lo, x);
      hi = fmaxf(hi, x);
    }
    if (!finite) atomicOr(flags, 1u);
    const float range = hi - lo;
    const float scale = range > 0.0f ? range / 15.0f : 1.0f;
    scales[i] = scale;
    biases[i] = lo;
    bounds[i] = range > 0.0f ? scale * 0.5001f + 1e-6f : 1e-6f;
  }
}

__global__ __launch_bounds__(kQuantThreads) void quant_pack_kernel(
    const float* __restrict__ v, size_t rows, size_t cols, size_t group,
    const float* __restrict__ scales, const float* __restrict__ biases,
    const float* __restrict__ bounds, uint32_t* __restrict__ packed,
    float* __restrict__ block_max, double* __restrict__ block_sum, uint32_t* __restrict__ flags) {
#pragma clang fp contract(off)
  __shared__ float smax[kQuantThreads];
  __shared__ double ssum[kQuantThreads];
  const size_t words_per_row = cols / 8u;
  const size_t groups = cols / group;
  const size_t n = rows * words_per_row;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  float worst = 0.0f;
  double total = 0.0;
  bool over = false;
  for (size_t w = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; w < n; w += stride) {
    const size_t row = w / words_per_row;
    const size_t col0 = (w % words_per_row) * 8u;
    uint32_t word = 0u;
    for (uint32_t lane = 0; lane < 8u; ++lane) {
      const size_t col = col0 + lane;
      const size_t gi = row * groups + col / group;
      const float scale = scales[gi];
      const float bias = biases[gi];
      const float x = v[row * cols + col];
      const float t = (x - bias) / scale;
      const int r = isnan(t) ? 0 : static_cast<int>(fminf(fmaxf(roundf(t), -1.0f), 16.0f));
      const uint32_t q = static_cast<uint32_t>(r < 0 ? 0 : (r > 15 ? 15 : r));
      word |= q << (4u * lane);
      const float err = fabsf(scale * static_cast<float>(q) + bias - x);
      over = over || err > bounds[gi];
      worst = fmaxf(worst, err);
      total += static_cast<double>(err);
    }
    packed[w] = word;
  }
  if (over) atomicOr(flags, 2u);
  smax[threadIdx.x] = worst;
  ssum[threadIdx.x] = total;
  __syncthreads();
  for (int h = kQuantThreads / 2; h > 0; h >>= 1) {
    if (static_cast<int>(threadIdx.x) < h) {
      smax[threadIdx.x] = fmaxf(smax[threadIdx.x], smax[threadIdx.x + h]);
      ssum[threadIdx.x] += ssum[threadIdx.x + h];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    block_max[blockIdx.x] = smax[0];
    block_sum[blockIdx.x] = ssum[0];
  }
}

}  // namespace

extern "C" {

int osmd_q4_dequant(const osmd_q4_proj* p, float* out, osmd_stream s) {
  const hipStream_t st = static_cast<hipStream_t>(s);
  const size_t words = static_cast<size_t>(p->out_dim) * p->packed_cols;
  const unsigned grid = grid_for(words, 256);
  switch (p->meta_dtype) {
    case OSM_META_F32:
      q4_dequant_kernel<OSM_META_F32><<<grid, 256, 0, st>>>(p->packed, p->scales, p->biases, p->out_dim, p->packed_cols, p->group, out);
      break;
    case OSM_META_F16:
      q4_dequant_kernel<OSM_META_F16><<<grid, 256, 0, st>>>(p->packed, p->scales, p->biases, p->out_dim, p->packed_cols, p->group, out);
      break;
    default:
      q4_dequant_kernel<OSM_META_BF16><<<grid, 256, 0, st>>>(p->packed, p->scales, p->biases, p->out_dim, p->packed_cols, p->group, out);
      break;
  }
  return launch_status();
}

int osmd_q4_gemv(const osmd_q4_proj* p, const float* x, float* y, osmd_stream s) {
  const hipStream_t st = static_cast<hipStream_t>(s);
  const unsigned grid = (p->out_dim + 3u) / 4u;  // 4 waves (rows) per block
  switch (p->meta_dtype) {
    case OSM_META_F32:
      q4_gemv_kernel<OSM_META_F32><<<grid, 256, 0, st>>>(p->packed, p->scales, p->biases, p->out_dim, p->packed_cols, p->group, x, y);
      break;
    case OSM_META_F16:
      q4_gemv_kernel<OSM_META_F16><<<grid, 256, 0, st>>>(p->packed, p->scales, p->biases, p->out_dim, p->packed_cols, p->group, x, y);
      break;
    default:
      q4_gemv_kernel<OSM_META_BF16><<<grid, 256, 0, st>>>(p->packed, p->scales, p->biases, p->out_dim, p->packed_cols, p->group, x, y);
      break;
  }
  return launch_status();
}

int osmd_unpack_nibbles(const uint32_t* packed, size_t words, uint8_t* out, osmd_stream s) {
  unpack_kernel<<<grid_for(words, 256), 256, 0, static_cast<hipStream_t>(s)>>>(packed, words, out);
  return launch_status();
}

int osmd_swiglu(const float* gate, const float* up, float* out, size_t n, osmd_stream s) {
  swiglu_kernel<<<grid_for(n, 256), 256, 0, static_cast<hipStream_t>(s)>>>(gate, up, out, n);
  return launch_status();
}

int osmd_weighted_accumulate(const float* src, float weight, float* acc, size_t n, osmd_stream s) {
  weighted_accumulate_kernel<<<grid_for(n, 256), 256, 0, static_cast<hipStream_t>(s)>>>(src, weight, acc, n);
  return launch_status();
}

int osmd_rms_norm(const float* in, const float* weight, float* out, uint32_t rows, uint32_t dim,
                  float eps, osmd_stream s) {
  rms_norm_kernel<<<rows, 256, 0, static_cast<hipStream_t>(s)>>>(in, weight, out, dim, eps);
  return launch_status();
}

unsigned osmd_q4_quantize_blocks(size_t rows, size_t cols) {
  const size_t words = rows * (cols / 8u);
  size_t b = (words + kQuantThreads - 1) / kQuantThreads;
  if (b == 0) b = 1;
  if (b > 2048) b = 2048;
  return static_cast<unsigned>(b);
}

int osmd_q4_quantize(const float* values, size_t rows, size_t cols, size_t group, uint32_t* packed,
                     float* scales, float* biases, float* bounds, float* block_max, double* block_sum,
                     uint32_t* flags, osmd_stream s) {
  const hipStream_t st = static_cast<hipStream_t>(s);
  const size_t ngroups = rows * (cols / group);
  size_t gb = (ngroups + 255) / 256;
  if (gb > 4096) gb = 4096;
  quant_groups_kernel<<<static_cast<unsigned>(gb), 256, 0, st>>>(values, rows, cols, group, scales, biases,
                                                                 bounds, flags);
  quant_pack_kernel<<<osmd_q4_quantize_blocks(rows, cols), kQuantThreads, 0, st>>>(
      values, rows, cols, group, scales, biases, bounds, packed, block_max, block_sum, flags);
  return launch_status();
}

}  // extern "C"
