// GPU quantizer: one wave per (row, group). Each lane owns value pairs (2 l, 2 l + 1) + 128 j of the group, so the
// packed byte of a pair is formed in one lane. With no clip grid the result is bit-identical to the canonical
// absmax quantizer (reference lowbit/quant.py:23-35): scale = fp16(amax / 7) with a correctly rounded fp32 division,
// q = clamp(round_half_even(w / fp32(scale)), -8, 7). With a grid it follows the reference's clip search
// (lowbit/ops.py:98-112): per candidate a, scale = fp16(fp32(amax * a) / 7), zero -> 1, squared error summed in
// fp32 (wave-tree order), strictly better replaces the best so ties keep the earlier candidate.
#include "kernels.hpp"

namespace lowbit {

namespace {

template <int kDtype>
__device__ __forceinline__ float load_w(const void* w, size_t i) {
  if (kDtype == 0) return reinterpret_cast<const float*>(w)[i];
  if (kDtype == 1) return (float)reinterpret_cast<const f16*>(w)[i];
  const uint32_t b = reinterpret_cast<const uint16_t*>(w)[i];
  return __builtin_bit_cast(float, b << 16);
}

__device__ __forceinline__ float quantize_one(float v, float scf) {
  return fminf(fmaxf(__builtin_rintf(v / scf), -8.0f), 7.0f);
}

}  // namespace

constexpr int kMaxPairsPerLane = 8;     // groups up to 1024 values

template <int kDtype>
__global__ __launch_bounds__(256) void quantize_kernel(const void* __restrict__ w, uint8_t* __restrict__ packed,
                                                       f16* __restrict__ scales, int N, int K, int G, ClipGrid grid) {
  const int lane = threadIdx.x & 63;
  const size_t group = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int KG = K / G;
  if (group >= (size_t)N * KG) return;
  const size_t n = group / KG, g = group % KG;
  const size_t base = n * K + g * G;
  const int npairs = G / 2;
  float v0[kMaxPairsPerLane], v1[kMaxPairsPerLane];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxPairsPerLane; ++j) {
    const int p = lane + 64 * j;
    v0[j] = v1[j] = 0.f;
    if (p < npairs) {
      v0[j] = load_w<kDtype>(w, base + 2 * p);
      v1[j] = load_w<kDtype>(w, base + 2 * p + 1);
      amax = fmaxf(amax, fmaxf(fabsf(v0[j]), fabsf(v1[j])));
    }
  }
  amax = wave_max(amax);
  const int ncand = grid.n > 0 ? grid.n : 1;
  f16 best_sc = (f16)1.0f;
  float best_err = 0.f;
  for (int ci = 0; ci < ncand; ++ci) {
    const float a = grid.n > 0 ? grid.a[ci] : 1.0f;
    const float num = a != 1.0f ? amax * a : amax;
    f16 sc = (f16)(num / 7.0f);
    if (sc == (f16)0.0f) sc = (f16)1.0f;
    if (grid.n == 0) {
      best_sc = sc;
      break;
    }
    const float scf = (float)sc;
    float err = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxPairsPerLane; ++j) {
      if (lane + 64 * j < npairs) {
        const float e0 = quantize_one(v0[j], scf) * scf - v0[j];
        const float e1 = quantize_one(v1[j], scf) * scf - v1[j];
        err += e0 * e0 + e1 * e1;
      }
    }
    err = wave_sum(err);
    if (ci == 0 || err < best_err) {
      best_err = err;
      best_sc = sc;
    }
  }
  const float scf = (float)best_sc;
#pragma unroll
  for (int j = 0; j < kMaxPairsPerLane; ++j) {
    const int p = lane + 64 * j;
    if (p < npairs) {
      const uint32_t u0 = (uint32_t)(int)(quantize_one(v0[j], scf) + 8.0f);
      const uint32_t u1 = (uint32_t)(int)(quantize_one(v1[j], scf) + 8.0f);
      packed[base / 2 + p] = (uint8_t)(u0 | (u1 << 4));
    }
  }
  if (lane == 0) scales[group] = best_sc;
}

hipError_t quantize_launch(const void* w, int dtype, uint8_t* packed, f16* scales, int N, int K, int G,
                           const ClipGrid& grid, hipStream_t st) {
  const size_t groups = (size_t)N * (K / G);
  dim3 gr((unsigned)((groups + 3) / 4)), block(256);
  switch (dtype) {
    case 0: return launch(quantize_kernel<0>, gr, block, 0, st, w, packed, scales, N, K, G, grid);
    case 1: return launch(quantize_kernel<1>, gr, block, 0, st, w, packed, scales, N, K, G, grid);
    default: return launch(quantize_kernel<2>, gr, block, 0, st, w, packed, scales, N, K, G, grid);
  }
}

}  // namespace lowbit
