// HBM bandwidth probes: the "measured peak" that the GEMV's bandwidth is quoted against.
//
// hbm_read: every thread walks the buffer with a grid stride, U 16-byte non-temporal loads in flight, and folds the
// words into one XOR. The fold decides a store that real data never triggers, so the loads cannot be removed and
// nothing else is written. hbm_copy: the same walk, each 16-byte piece stored to the destination.
// Both are plain streaming kernels: no LDS, no barriers, every index < n16 by the loop conditions.
#include <hip/hip_runtime.h>
#include <cstdint>

#include "kernels.hpp"

namespace lowbit {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(256) void hbm_read_kernel(const u32x4_t* __restrict__ p, size_t n16,
                                                       uint32_t* __restrict__ sink) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (U - 1) * stride < n16; i += U * stride) {
    u32x4_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    u32x4_t v = __builtin_nontemporal_load(p + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;   // keeps the loads; any thread that stores writes the same word
}

template <int U>
__global__ __launch_bounds__(256) void hbm_copy_kernel(const u32x4_t* __restrict__ p, u32x4_t* __restrict__ q,
                                                       size_t n16) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + (U - 1) * stride < n16; i += U * stride) {
    u32x4_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) __builtin_nontemporal_store(v[u], q + i + u * stride);
  }
  for (; i < n16; i += stride) __builtin_nontemporal_store(__builtin_nontemporal_load(p + i), q + i);
}

hipError_t hbm_read_launch(const void* src, size_t bytes, uint32_t* sink, int blocks, hipStream_t stream) {
  hbm_read_kernel<4><<<blocks, 256, 0, stream>>>(static_cast<const u32x4_t*>(src), bytes / 16, sink);
  return hipGetLastError();
}

hipError_t hbm_copy_launch(const void* src, void* dst, size_t bytes, int blocks, hipStream_t stream) {
  hbm_copy_kernel<4><<<blocks, 256, 0, stream>>>(static_cast<const u32x4_t*>(src), static_cast<u32x4_t*>(dst),
                                                 bytes / 16);
  return hipGetLastError();
}

}  // namespace lowbit
