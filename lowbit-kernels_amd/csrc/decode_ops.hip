// Decode-step neighbours of the W4A16 projections in a Qwen2 decoder layer, so that one layer is nine launches
// instead of the ~50 the stock PyTorch modules issue per token: RMSNorm, RoPE fused with the KV-cache write, and
// causal GQA attention over the cache. Each follows the arithmetic of the module it replaces (transformers
// Qwen2RMSNorm, apply_rotary_pos_emb + StaticCache.update, scaled_dot_product_attention with a causal mask), with
// the same fp16 roundings where the torch ops round.
#include "kernels.hpp"

namespace lowbit {

namespace {

constexpr int kHeadDim = 128;

__device__ __forceinline__ float block_sum(float v, float* red) {    // all threads of the block get the total
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

}  // namespace

// out[m] = w * fp16(x[m] / sqrt(mean(x[m]^2) + eps)), one block per row (Qwen2RMSNorm: the normalisation in fp32,
// rounded to fp16, then the fp16 product with the weight)
__global__ __launch_bounds__(256) void rmsnorm_kernel(const f16* __restrict__ x, const f16* __restrict__ w,
                                                      f16* __restrict__ out, int H, float eps) {
  __shared__ float red[4];
  const size_t row = (size_t)blockIdx.x * H;
  float ss = 0.f;
  for (int i = threadIdx.x * 8; i < H; i += blockDim.x * 8) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + row + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x2 p = as_f16x2(v[j]);
      ss = fmaf((float)p[0], (float)p[0], ss);
      ss = fmaf((float)p[1], (float)p[1], ss);
    }
  }
  const float r = rsqrtf(block_sum(ss, red) / (float)H + eps);
  for (int i = threadIdx.x * 8; i < H; i += blockDim.x * 8) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + row + i);
    const u32x4 g = *reinterpret_cast<const u32x4*>(w + i);
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x2 p = as_f16x2(v[j]), wj = as_f16x2(g[j]);
      const f16x2 n = {(f16)((float)p[0] * r), (f16)((float)p[1] * r)};
      o[j] = as_u32(f16x2{(f16)((float)wj[0] * (float)n[0]), (f16)((float)wj[1] * (float)n[1])});
    }
    *reinterpret_cast<u32x4*>(out + row + i) = o;
  }
}

// qkv [M][(Hq + 2 Hkv) D] (the fused projection's output, bias included) -> q_out [M][Hq][D] with RoPE; k (with
// RoPE) and v written to k_cache / v_cache [Hkv][L][D] at row positions[m]. One thread per (token, head, dim pair
// (i, i + 64)). RoPE as transformers computes it for fp16 models: angle = fp32(position * inv_freq[i]), cos and sin
// in fp32 rounded to fp16, x * cos + rotate_half(x) * sin with each product and the sum rounded to fp16.
__global__ __launch_bounds__(256) void rope_kv_kernel(const f16* __restrict__ qkv, const int64_t* __restrict__ pos,
                                                      const float* __restrict__ inv_freq, f16* __restrict__ q_out,
                                                      f16* __restrict__ k_cache, f16* __restrict__ v_cache, int M,
                                                      int Hq, int Hkv, int L) {
#pragma clang fp contract(off)                                 // each product rounded to fp16 before the sum, as torch
  const int heads = Hq + 2 * Hkv;
  const int gid = blockIdx.x * blockDim.x + threadIdx.x;
  const int i = gid & 63, h = (gid >> 6) % heads, m = (gid >> 6) / heads;
  if (m >= M) return;
  const int64_t p = pos[m];
  if (p < 0 || p >= L) return;                               // the host checks positions; never write out of bounds
  const f16* src = qkv + ((size_t)m * heads + h) * kHeadDim;
  if (h >= Hq + Hkv) {                                       // v: plain copy into the cache
    f16* dst = v_cache + ((size_t)(h - Hq - Hkv) * L + p) * kHeadDim;
    dst[i] = src[i];
    dst[i + 64] = src[i + 64];
    return;
  }
  const float ang = (float)p * inv_freq[i];
  const f16 c = (f16)cosf(ang), s = (f16)sinf(ang);
  const f16 x1 = src[i], x2 = src[i + 64];
  const f16 o1 = (f16)(x1 * c) + (f16)(-x2 * s);
  const f16 o2 = (f16)(x2 * c) + (f16)(x1 * s);
  f16* dst = h < Hq ? q_out + ((size_t)m * Hq + h) * kHeadDim : k_cache + ((size_t)(h - Hq) * L + p) * kHeadDim;
  dst[i] = o1;
  dst[i + 64] = o2;
}

// Causal GQA attention for M query tokens at positions pos[m] over the cache rows 0 .. pos[m]:
// out[m][h * D + d] = sum_j softmax_j(scale * q[m][h] . k[j]) v[j][d], for the G = Hq / Hkv query heads of KV head hk.
// One block of W waves per (token, KV head). Each wave takes blocks of 64 keys (key w * 64 + 64 W b + lane):
// scores with the lane holding one key, an online softmax per head in fp32, then P V with the lane holding two of
// the 128 output dims. The waves' partial states are merged through LDS at the end.
template <int G>
__global__ __launch_bounds__(1024) void attention_kernel(const f16* __restrict__ q, const f16* __restrict__ k_cache,
                                                         const f16* __restrict__ v_cache,
                                                         const int64_t* __restrict__ pos, f16* __restrict__ out,
                                                         int Hq, int Hkv, int L, float scale) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int m = blockIdx.x / Hkv, hk = blockIdx.x % Hkv;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), W = blockDim.x >> 6;
  const int64_t pm = pos[m];
  const int nkeys = (int)min((int64_t)L, pm + 1);
  // LDS: q [G][D] fp16 | p [W][G][64] fp32 | partial states [W][G] (max, sum) + [W][G][D] fp32
  f16* qs = reinterpret_cast<f16*>(smem);
  float* ps = reinterpret_cast<float*>(smem + G * kHeadDim * 2);
  float* st = ps + W * G * 64;
  float* os = st + W * G * 2;
  for (int i = threadIdx.x; i < G * kHeadDim; i += blockDim.x)
    qs[i] = q[((size_t)m * Hq + hk * G) * kHeadDim + i];
  __syncthreads();

  const f16* kb = k_cache + (size_t)hk * L * kHeadDim;
  const f16* vb = v_cache + (size_t)hk * L * kHeadDim;
  float mx[G], sum[G], o0[G], o1[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    mx[g] = -INFINITY;
    sum[g] = 0.f;
    o0[g] = o1[g] = 0.f;
  }
  for (int base = wave * 64; base < nkeys; base += 64 * W) {
    // scores: lane = key base + lane
    const int j = base + lane;
    float sc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) sc[g] = 0.f;
    if (j < nkeys) {
      const u32x4* kr = reinterpret_cast<const u32x4*>(kb + (size_t)j * kHeadDim);
#pragma unroll 4
      for (int c = 0; c < kHeadDim / 8; ++c) {
        const u32x4 kv = kr[c];
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const u32x4 qv = *reinterpret_cast<const u32x4*>(qs + g * kHeadDim + 8 * c);
#pragma unroll
          for (int e = 0; e < 4; ++e) sc[g] = dot2(as_f16x2(qv[e]), as_f16x2(kv[e]), sc[g]);
        }
      }
    }
    // online softmax over this block of keys, per head
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float s = j < nkeys ? sc[g] * scale : -INFINITY;
      const float bm = wave_max(s);
      const float nm = fmaxf(mx[g], bm);
      const float corr = expf(mx[g] - nm);                   // 0 on the first block (mx = -inf)
      const float pj = j < nkeys ? expf(s - nm) : 0.f;
      sum[g] = sum[g] * corr + wave_sum(pj);
      o0[g] *= corr;
      o1[g] *= corr;
      mx[g] = nm;
      ps[(wave * G + g) * 64 + lane] = pj;
    }
    __builtin_amdgcn_wave_barrier();                         // LDS is in order per wave; keep the compiler's order too
    // P V: lane = output dims 2 lane, 2 lane + 1 (the wave reads back its own probabilities)
    const int nb = min(64, nkeys - base);
    for (int t = 0; t < nb; ++t) {
      const f16x2 vv = *reinterpret_cast<const f16x2*>(vb + (size_t)(base + t) * kHeadDim + 2 * lane);
      const float v0 = (float)vv[0], v1 = (float)vv[1];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pj = ps[(wave * G + g) * 64 + t];
        o0[g] = fmaf(pj, v0, o0[g]);
        o1[g] = fmaf(pj, v1, o1[g]);
      }
    }
    __builtin_amdgcn_wave_barrier();                         // every lane has read ps before the next block rewrites it
  }
  // merge the waves
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (lane == 0) {
      st[(wave * G + g) * 2] = mx[g];
      st[(wave * G + g) * 2 + 1] = sum[g];
    }
    os[((wave * G + g) * kHeadDim) + 2 * lane] = o0[g];
    os[((wave * G + g) * kHeadDim) + 2 * lane + 1] = o1[g];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * kHeadDim; idx += blockDim.x) {
    const int g = idx / kHeadDim, d = idx % kHeadDim;
    float gm = -INFINITY;
    for (int w = 0; w < W; ++w) gm = fmaxf(gm, st[(w * G + g) * 2]);
    float num = 0.f, den = 0.f;
    for (int w = 0; w < W; ++w) {
      const float wm = st[(w * G + g) * 2];
      if (wm == -INFINITY) continue;                           // a wave that saw no key
      const float f = expf(wm - gm);
      num = fmaf(f, os[(w * G + g) * kHeadDim + d], num);
      den = fmaf(f, st[(w * G + g) * 2 + 1], den);
    }
    out[((size_t)m * Hq + hk * G + g) * kHeadDim + d] = (f16)(num / den);
  }
}

hipError_t rmsnorm_launch(const f16* x, const f16* w, f16* out, int M, int H, float eps, hipStream_t st) {
  return launch(rmsnorm_kernel, dim3(M), dim3(256), 0, st, x, w, out, H, eps);
}

hipError_t rope_kv_launch(const f16* qkv, const int64_t* pos, const float* inv_freq, f16* q_out, f16* k_cache,
                          f16* v_cache, int M, int Hq, int Hkv, int L, hipStream_t st) {
  const long threads = (long)M * (Hq + 2 * Hkv) * 64;
  return launch(rope_kv_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, qkv, pos, inv_freq, q_out,
                k_cache, v_cache, M, Hq, Hkv, L);
}

namespace {
template <int G>
hipError_t launch_attention(const f16* q, const f16* k, const f16* v, const int64_t* pos, f16* out, int M, int Hq,
                            int Hkv, int L, int max_keys, float scale, hipStream_t st) {
  int waves = 1;                                              // enough waves to give each about 64 keys
  while (waves < 16 && waves * 64 < max_keys) waves *= 2;
  const size_t lds = (size_t)G * kHeadDim * 2 + (size_t)waves * G * 64 * 4 + (size_t)waves * G * 2 * 4 +
                     (size_t)waves * G * kHeadDim * 4;
  if (lds > 65536) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(attention_kernel<G>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
    if (attr != hipSuccess) return attr;
  }
  return launch(attention_kernel<G>, dim3(M * Hkv), dim3(64 * waves), lds, st, q, k, v, pos, out, Hq, Hkv, L, scale);
}
}  // namespace

hipError_t attention_launch(const f16* q, const f16* k, const f16* v, const int64_t* pos, f16* out, int M, int Hq,
                            int Hkv, int L, int max_keys, float scale, hipStream_t st) {
  switch (Hq / Hkv) {
    case 1: return launch_attention<1>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, st);
    case 2: return launch_attention<2>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, st);
    case 4: return launch_attention<4>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, st);
    case 6: return launch_attention<6>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, st);
    case 7: return launch_attention<7>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, st);
    case 8: return launch_attention<8>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace lowbit
