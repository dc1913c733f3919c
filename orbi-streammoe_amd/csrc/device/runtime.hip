// runtime.hip -- device memory, streams and events behind osm_device.h.
#include <hip/hip_runtime.h>

#include <cstring>

#include "device_common.hpp"

namespace {

int rc(hipError_t e) { return e == hipSuccess ? 0 : static_cast<int>(e); }

__global__ void zero_kernel(uint4* __restrict__ dst16, size_t n16,
                            uint8_t* __restrict__ tail, size_t ntail) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
    dst16[i] = make_uint4(0u, 0u, 0u, 0u);
  if (blockIdx.x == 0)
    for (size_t i = threadIdx.x; i < ntail; i += blockDim.x) tail[i] = 0;
}

// Grid-stride copy: each lane moves 16 bytes per step, so a wavefront
// instruction moves 1 KB of contiguous memory.
__global__ void copy16_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n16) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
    dst[i] = src[i];
}

// Checksums of the selection's exp (osm_libm_expf) over a range of float bit
// patterns: block b covers inputs first + b * block ..., and its sum is
// sum_i bits(exp(x_i)) * (2 i + 1) mod 2^64 over its inputs i (an odd
// multiplier, so any single wrong result changes the sum).
__global__ __launch_bounds__(256) void libm_expf_sums_kernel(uint32_t first, uint64_t count, uint32_t block,
                                                             uint64_t* __restrict__ sums) {
  __shared__ uint64_t red[256];
  const uint64_t b0 = static_cast<uint64_t>(blockIdx.x) * block;
  uint64_t s = 0;
  for (uint32_t i = threadIdx.x; i < block && b0 + i < count; i += 256u) {
    const float x = __uint_as_float(first + static_cast<uint32_t>(b0 + i));
    s += static_cast<uint64_t>(__float_as_uint(osm_libm_expf(x))) * (2u * static_cast<uint64_t>(i) + 1u);
  }
  red[threadIdx.x] = s;
  __syncthreads();
  for (uint32_t w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) sums[blockIdx.x] = red[0];
}

}  // namespace

extern "C" {

const char* osmd_error_string(int code) {
  return hipGetErrorString(static_cast<hipError_t>(code));
}

int osmd_device_count(int* count) { return rc(hipGetDeviceCount(count)); }

int osmd_libm_expf_checksums(uint32_t first, uint64_t count, uint32_t block, uint64_t* sums, osmd_stream s) {
  const uint64_t nblocks = (count + block - 1u) / block;
  if (count == 0u || block == 0u || nblocks > 0x7FFFFFFFu) return static_cast<int>(hipErrorInvalidValue);
  libm_expf_sums_kernel<<<static_cast<uint32_t>(nblocks), 256, 0, static_cast<hipStream_t>(s)>>>(first, count, block,
                                                                                                 sums);
  return rc(hipGetLastError());
}
int osmd_set_device(int device) { return rc(hipSetDevice(device)); }

int osmd_device_name(int device, char* buf, size_t n) {
  hipDeviceProp_t prop;
  const int r = rc(hipGetDeviceProperties(&prop, device));
  if (r != 0) return r;
  if (n > 0) {
    // Some drivers leave the marketing name empty; the ISA name then says
    // what the device is.
    const char* name = prop.name[0] != '\0' ? prop.name : prop.gcnArchName;
    std::strncpy(buf, name, n - 1);
    buf[n - 1] = '\0';
  }
  return 0;
}

int osmd_device_mem_info(size_t* free_bytes, size_t* total_bytes) {
  return rc(hipMemGetInfo(free_bytes, total_bytes));
}

int osmd_malloc(void** ptr, size_t bytes) { return rc(hipMalloc(ptr, bytes)); }
int osmd_free(void* ptr) { return ptr ? rc(hipFree(ptr)) : 0; }
int osmd_host_malloc(void** ptr, size_t bytes) {
  return rc(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
}
int osmd_host_free(void* ptr) { return ptr ? rc(hipHostFree(ptr)) : 0; }

int osmd_memcpy_h2d(void* dst, const void* src, size_t bytes, osmd_stream s) {
  return rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(s)));
}
int osmd_memcpy_d2h(void* dst, const void* src, size_t bytes, osmd_stream s) {
  return rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, static_cast<hipStream_t>(s)));
}
int osmd_memcpy_d2d(void* dst, const void* src, size_t bytes, osmd_stream s) {
  return rc(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(s)));
}

int osmd_zero(void* dst, size_t bytes, osmd_stream s) {
  if (bytes == 0) return 0;
  // Split into an aligned 16-byte body and a byte tail.
  const uintptr_t p = reinterpret_cast<uintptr_t>(dst);
  if (p % 16 != 0) {
    zero_kernel<<<1, 256, 0, static_cast<hipStream_t>(s)>>>(nullptr, 0, static_cast<uint8_t*>(dst), bytes);
    return osmk::launch_status();
  }
  const size_t n16 = bytes / 16;
  const size_t ntail = bytes - n16 * 16;
  size_t blocks = (n16 + 255) / 256;
  if (blocks == 0) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  zero_kernel<<<static_cast<unsigned>(blocks), 256, 0, static_cast<hipStream_t>(s)>>>(
      static_cast<uint4*>(dst), n16, static_cast<uint8_t*>(dst) + n16 * 16, ntail);
  return osmk::launch_status();
}

int osmd_copy_d2d(void* dst, const void* src, size_t bytes, osmd_stream s) {
  if (bytes == 0) return 0;
  const uintptr_t a = reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) | bytes;
  if (a % 16 != 0) return osmd_memcpy_d2d(dst, src, bytes, s);
  const size_t n16 = bytes / 16;
  size_t blocks = (n16 + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  copy16_kernel<<<static_cast<unsigned>(blocks), 256, 0, static_cast<hipStream_t>(s)>>>(
      static_cast<const uint4*>(src), static_cast<uint4*>(dst), n16);
  return osmk::launch_status();
}

int osmd_copy_from_pinned(void* dst, const void* src, size_t bytes, unsigned blocks, osmd_stream s) {
  if (bytes == 0) return 0;
  const uintptr_t a = reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) | bytes;
  if (a % 16 != 0 || blocks == 0) return osmd_memcpy_h2d(dst, src, bytes, s);
  const size_t n16 = bytes / 16;
  size_t grid = (n16 + 255) / 256;
  if (grid > blocks) grid = blocks;
  copy16_kernel<<<static_cast<unsigned>(grid), 256, 0, static_cast<hipStream_t>(s)>>>(
      static_cast<const uint4*>(src), static_cast<uint4*>(dst), n16);
  return osmk::launch_status();
}

int osmd_stream_create(osmd_stream* s) {
  hipStream_t h = nullptr;
  // Default priority, non-blocking with respect to the null stream.
  const int r = rc(hipStreamCreateWithFlags(&h, hipStreamNonBlocking));
  *s = h;
  return r;
}
int osmd_stream_device(osmd_stream s, int* device) {
  hipDevice_t d = -1;
  const int r = rc(hipStreamGetDevice(static_cast<hipStream_t>(s), &d));
  *device = static_cast<int>(d);
  return r;
}
int osmd_stream_destroy(osmd_stream s) {
  return s ? rc(hipStreamDestroy(static_cast<hipStream_t>(s))) : 0;
}
int osmd_stream_synchronize(osmd_stream s) {
  return rc(hipStreamSynchronize(static_cast<hipStream_t>(s)));
}
int osmd_event_create(osmd_event* e) {
  hipEvent_t h = nullptr;
  const int r = rc(hipEventCreate(&h));
  *e = h;
  return r;
}
int osmd_event_destroy(osmd_event e) {
  return e ? rc(hipEventDestroy(static_cast<hipEvent_t>(e))) : 0;
}
int osmd_event_record(osmd_event e, osmd_stream s) {
  return rc(hipEventRecord(static_cast<hipEvent_t>(e), static_cast<hipStream_t>(s)));
}
int osmd_event_synchronize(osmd_event e) {
  return rc(hipEventSynchronize(static_cast<hipEvent_t>(e)));
}
int osmd_stream_wait_event(osmd_stream s, osmd_event e) {
  return rc(hipStreamWaitEvent(static_cast<hipStream_t>(s), static_cast<hipEvent_t>(e), 0));
}
int osmd_event_elapsed_ms(osmd_event start, osmd_event stop, float* ms) {
  return rc(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
}
int osmd_device_synchronize(void) { return rc(hipDeviceSynchronize()); }

// Graph capture of one stream: what is enqueued between begin and end is
// recorded instead of run, then instantiated once and replayed with a single
// submission per launch. Thread-local mode: other threads keep using HIP.
int osmd_capture_begin(osmd_stream s) {
  return rc(hipStreamBeginCapture(static_cast<hipStream_t>(s), hipStreamCaptureModeThreadLocal));
}
int osmd_capture_end(osmd_stream s, osmd_graph* out) {
  *out = nullptr;
  hipGraph_t graph = nullptr;
  int r = rc(hipStreamEndCapture(static_cast<hipStream_t>(s), &graph));
  if (r != 0) {
    if (graph) (void)hipGraphDestroy(graph);
    return r;
  }
  hipGraphExec_t exec = nullptr;
  r = rc(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
  (void)hipGraphDestroy(graph);
  if (r == 0) *out = exec;
  return r;
}
int osmd_graph_launch(osmd_graph g, osmd_stream s) {
  return rc(hipGraphLaunch(static_cast<hipGraphExec_t>(g), static_cast<hipStream_t>(s)));
}
int osmd_graph_destroy(osmd_graph g) {
  return g ? rc(hipGraphExecDestroy(static_cast<hipGraphExec_t>(g))) : 0;
}

}  // extern "C"
