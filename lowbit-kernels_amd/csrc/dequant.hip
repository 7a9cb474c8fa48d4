// Dequantize to fp16 W [N, K] (the prefill path's first half, then hipBLASLt), and the device relayout
// canonical -> v3 / MFMA layouts.
//
// Dequant: each thread owns one 16-byte piece of packed weights (32 values of one row, inside one group because
// G % 32 == 0) and writes its 64 output bytes with four 16-byte stores; consecutive threads write consecutive output
// (row-major), so a wave writes 4 KB contiguous. The value is (u - 8) exactly in fp16 (magic-number decode) times
// the fp16 scale with one IEEE rounding: bit-identical to float16((u - 8) * scale) computed in fp64, which is the
// reference rule (csrc/w4_gemv.cu:296-310,393-408; checked bit for bit at bench/gpu_run.py:217-228).
#include "kernels.hpp"

namespace lowbit {

namespace {

// canonical word (nibble b = k0 + b) -> v3 word (slots hold k0, k2, k4, k6, k1, k3, k5, k7)
__device__ __forceinline__ uint32_t canonical_to_v3(uint32_t w) {
  uint32_t e = w & 0x0F0F0F0Fu, o = (w >> 4) & 0x0F0F0F0Fu;
  e = (e | (e >> 4)) & 0x00FF00FFu;
  e = (e | (e >> 8)) & 0x0000FFFFu;
  o = (o | (o >> 4)) & 0x00FF00FFu;
  o = (o | (o >> 8)) & 0x0000FFFFu;
  return e | (o << 16);
}

__device__ __forceinline__ size_t mfma_offset(int n, int c, int q, int N, int K) {
  const int t = n >> 4, r = n & 15, rows = min(16, N - 16 * t);
  return (size_t)t * 8 * K + (size_t)c * rows * 64 + 64 * r + 16 * q;
}

}  // namespace

template <bool kMfma>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w, const f16* __restrict__ s,
                                                      f16* __restrict__ out, int N, int K, int G) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x, per_row = (size_t)K / 32;
  if (idx >= (size_t)N * per_row) return;
  const int n = (int)(idx / per_row), b = (int)(idx % per_row);     // output k = 32 b .. 32 b + 31
  const size_t src = kMfma ? mfma_offset(n, b >> 2, b & 3, N, K) : idx * 16;
  const u32x4 wv = load_stream(w + src);
  const f16 sv = s[(size_t)n * (K / G) + (32 * b) / G];
  const f16x2 sc = {sv, sv};
  u32x4 o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f16x2 p[4];
    decode_word(wv[j], p);
#pragma unroll
    for (int e = 0; e < 4; ++e) p[e] = p[e] * sc;
    if (kMfma) {          // v3 words decode in k order: (k0,k1), (k2,k3), (k4,k5), (k6,k7)
      o[j] = u32x4{as_u32(p[0]), as_u32(p[1]), as_u32(p[2]), as_u32(p[3])};
    } else {              // canonical words decode to (k0,k4), (k1,k5), (k2,k6), (k3,k7)
      const f16x2 a = {p[0][0], p[1][0]}, bb = {p[2][0], p[3][0]}, c = {p[0][1], p[1][1]}, d = {p[2][1], p[3][1]};
      o[j] = u32x4{as_u32(a), as_u32(bb), as_u32(c), as_u32(d)};
    }
  }
  u32x4* dst = reinterpret_cast<u32x4*>(out + (size_t)n * K + 32 * b);
#pragma unroll
  for (int j = 0; j < 4; ++j) dst[j] = o[j];
}

template <bool kMfma>
__global__ __launch_bounds__(256) void relayout_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int N,
                                                       int K) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x, per_row = (size_t)K / 32;
  if (idx >= (size_t)N * per_row) return;
  const int n = (int)(idx / per_row), b = (int)(idx % per_row);
  const u32x4 wv = load16(src + idx * 16);
  const u32x4 v3 = {canonical_to_v3(wv[0]), canonical_to_v3(wv[1]), canonical_to_v3(wv[2]), canonical_to_v3(wv[3])};
  const size_t off = kMfma ? mfma_offset(n, b >> 2, b & 3, N, K) : idx * 16;
  *reinterpret_cast<u32x4*>(dst + off) = v3;
}

hipError_t dequant_launch(const uint8_t* w, const f16* s, f16* out, int N, int K, int G, bool mfma, hipStream_t st) {
  const size_t total = (size_t)N * (K / 32);
  dim3 grid((unsigned)((total + 255) / 256)), block(256);
  if (mfma) return launch(dequant_kernel<true>, grid, block, 0, st, w, s, out, N, K, G);
  return launch(dequant_kernel<false>, grid, block, 0, st, w, s, out, N, K, G);
}

hipError_t relayout_launch(const uint8_t* src, uint8_t* dst, int N, int K, bool mfma, hipStream_t st) {
  const size_t total = (size_t)N * (K / 32);
  dim3 grid((unsigned)((total + 255) / 256)), block(256);
  if (mfma) return launch(relayout_kernel<true>, grid, block, 0, st, src, dst, N, K);
  return launch(relayout_kernel<false>, grid, block, 0, st, src, dst, N, K);
}

}  // namespace lowbit
