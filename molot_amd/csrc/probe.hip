// Streaming read / copy probes of known traffic (see include/molot_amd/probe.h).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "molot_amd/attn_hip.h"
#include "molot_amd/probe.h"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 1024;
constexpr int kUnroll = 8;

// Streaming read: workgroup b reads one contiguous slab of the buffer with
// non-temporal 16-byte loads, kUnroll in flight per thread (the fastest of
// the read patterns measured on MI355X).
__global__ __launch_bounds__(kThreads) void read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                        float* __restrict__ sink) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t lo = (int64_t)blockIdx.x * per;
  const int64_t hi = lo + per < n16 ? lo + per : n16;
  int64_t i = lo + threadIdx.x;
  unsigned acc = 0;
  for (; i + (kUnroll - 1) * kThreads < hi; i += kUnroll * kThreads) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * kThreads);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < hi; i += kThreads) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  __shared__ unsigned red[kThreads / 64];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc ^= __shfl_xor(acc, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned r = 0;
    for (int w = 0; w < kThreads / 64; ++w) r ^= red[w];
    sink[blockIdx.x] = (float)(r & 0xFFFF);
  }
}

__global__ __launch_bounds__(kThreads) void copy_kernel(u32x4* __restrict__ dst,
                                                        const u32x4* __restrict__ src,
                                                        int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = src[i + u * stride];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) dst[i + u * stride] = v[u];
  }
  for (; i < n16; i += stride) dst[i] = src[i];
}

int grid_for(int64_t n16) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  int64_t g = (int64_t)cus;  // one 16-wave workgroup per CU
  const int64_t need = (n16 + kThreads - 1) / kThreads;
  return (int)(g < need ? g : (need > 0 ? need : 1));
}

}  // namespace

extern "C" {

int molot_probe_read(const void* src, int64_t bytes, float* sink, int64_t sink_len,
                     void* stream) {
  if (!src || !sink || bytes <= 0 || (bytes & 15) || ((uintptr_t)src & 15)) return MOLOT_EINVAL;
  const int64_t n16 = bytes / 16;
  const int grid = grid_for(n16);
  if (sink_len < grid) return MOLOT_EINVAL;
  hipLaunchKernelGGL(read_kernel, dim3(grid), dim3(kThreads), 0, (hipStream_t)stream,
                     (const u32x4*)src, n16, sink);
  return (int)hipGetLastError();
}

int molot_probe_copy(void* dst, const void* src, int64_t bytes, void* stream) {
  if (!src || !dst || bytes <= 0 || (bytes & 15) || ((uintptr_t)src & 15) ||
      ((uintptr_t)dst & 15))
    return MOLOT_EINVAL;
  const int64_t n16 = bytes / 16;
  hipLaunchKernelGGL(copy_kernel, dim3(grid_for(n16)), dim3(kThreads), 0, (hipStream_t)stream,
                     (u32x4*)dst, (const u32x4*)src, n16);
  return (int)hipGetLastError();
}

}  // extern "C"
