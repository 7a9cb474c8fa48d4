// Dequantize to fp16 W [N, K] (the prefill path's first half, then hipBLASLt), and the device relayout
// canonical -> v3 / MFMA layouts.
//
// Dequant: each thread decodes 4 packed words (8 values of one row each, inside one group because G % 32 == 0) and
// writes each as one 16-byte store; consecutive threads own consecutive words, so loads and stores are contiguous
// per instruction. The value is (u - 8) exactly in fp16 (magic-number decode) times
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

// A piece is 8 consecutive outputs of one row: one 4-byte packed word in, 16 bytes out, and piece p of the
// row-major output starts at element 8p. A workgroup owns 1024 consecutive pieces, 4 per thread spaced 256 apart, so
// every load instruction reads and every store instruction writes a contiguous span (1 KB / 4 KB per workgroup).
// All 4 loads of a thread are issued before the first decode.
template <bool kMfma>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w, const f16* __restrict__ s,
                                                      f16* __restrict__ out, int N, int K, int G) {
  const uint32_t per_row = (uint32_t)K / 8, total = (uint32_t)N * per_row, groups = (uint32_t)(K / G);
  const uint32_t p0 = blockIdx.x * 1024u + threadIdx.x;
  uint32_t wv[4];
  f16 sv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t p = p0 + 256u * j;
    wv[j] = 0;
    sv[j] = (f16)0.0f;
    if (p < total) {
      const uint32_t n = p / per_row, kp = p - n * per_row;        // output k = 8 kp .. 8 kp + 7
      // MFMA layout: 16-byte piece (n, chunk kp / 16, quarter (kp / 4) % 4), word kp % 4 holds k in order
      const size_t src = kMfma ? mfma_offset((int)n, (int)(kp >> 4), (int)((kp >> 2) & 3), N, K) + 4 * (kp & 3)
                               : (size_t)p * 4;
      wv[j] = *reinterpret_cast<const uint32_t*>(w + src);
      sv[j] = s[(size_t)n * groups + (8 * kp) / (uint32_t)G];
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t p = p0 + 256u * j;
    if (p >= total) continue;
    const f16x2 sc = {sv[j], sv[j]};
    f16x2 q[4];
    decode_word(wv[j], q);
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = q[e] * sc;
    u32x4 o;
    if (kMfma) {          // v3 words decode in k order: (k0,k1), (k2,k3), (k4,k5), (k6,k7)
      o = u32x4{as_u32(q[0]), as_u32(q[1]), as_u32(q[2]), as_u32(q[3])};
    } else {              // canonical words decode to (k0,k4), (k1,k5), (k2,k6), (k3,k7)
      const f16x2 a = {q[0][0], q[1][0]}, b = {q[2][0], q[3][0]}, c = {q[0][1], q[1][1]}, d = {q[2][1], q[3][1]};
      o = u32x4{as_u32(a), as_u32(b), as_u32(c), as_u32(d)};
    }
    *reinterpret_cast<u32x4*>(out + (size_t)p * 8) = o;
  }
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
  const size_t total = (size_t)N * (K / 8);
  if (total >= (1ull << 32) - 1024) return hipErrorInvalidValue;      // piece indices are 32-bit
  dim3 grid((unsigned)((total + 1023) / 1024)), block(256);
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
