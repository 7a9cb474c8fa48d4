// Decode-step neighbours of the W4A16 projections in a Qwen2 decoder layer, so that one layer is nine launches
// instead of the ~50 the stock PyTorch modules issue per token: RMSNorm, RoPE fused with the KV-cache write, and
// causal GQA attention over the cache. Each follows the arithmetic of the module it replaces (transformers
// Qwen2RMSNorm, apply_rotary_pos_emb + StaticCache.update, scaled_dot_product_attention with a causal mask), with
// the same fp16 roundings where the torch ops round.
#include <algorithm>

#include "kernels.hpp"

namespace lowbit {

namespace {

constexpr int kHeadDim = kAttnHeadDim;

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
// rounded to fp16, then the fp16 product with the weight). The first kNormPieces 16-byte pieces of x and w per thread
// (H <= 8192 at 256 threads) are loaded once, before the block reduction, and kept in registers for the output: one
// memory round trip instead of two; longer rows reload the rest.
constexpr int kNormPieces = 4;
__global__ __launch_bounds__(256) void rmsnorm_kernel(const f16* __restrict__ x, const f16* __restrict__ w,
                                                      f16* __restrict__ out, int H, float eps) {
  __shared__ float red[4];
  const size_t row = (size_t)blockIdx.x * H;
  const int step = blockDim.x * 8;
  u32x4 xv[kNormPieces], wv[kNormPieces];
#pragma unroll
  for (int c = 0; c < kNormPieces; ++c) {
    const int i = threadIdx.x * 8 + c * step;
    if (i < H) {
      xv[c] = *reinterpret_cast<const u32x4*>(x + row + i);
      wv[c] = *reinterpret_cast<const u32x4*>(w + i);
    }
  }
  float ss = 0.f;
  auto add_squares = [&](const u32x4& v) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x2 p = as_f16x2(v[j]);
      ss = fmaf((float)p[0], (float)p[0], ss);
      ss = fmaf((float)p[1], (float)p[1], ss);
    }
  };
#pragma unroll
  for (int c = 0; c < kNormPieces; ++c)
    if (threadIdx.x * 8 + c * step < H) add_squares(xv[c]);
  for (int i = threadIdx.x * 8 + kNormPieces * step; i < H; i += step) add_squares(*reinterpret_cast<const u32x4*>(x + row + i));
  const float r = rsqrtf(block_sum(ss, red) / (float)H + eps);
  auto store_norm = [&](int i, const u32x4& v, const u32x4& g) {
    *reinterpret_cast<u32x4*>(out + row + i) = rms_apply8(v, g, r);
  };
#pragma unroll
  for (int c = 0; c < kNormPieces; ++c) {
    const int i = threadIdx.x * 8 + c * step;
    if (i < H) store_norm(i, xv[c], wv[c]);
  }
  for (int i = threadIdx.x * 8 + kNormPieces * step; i < H; i += step)
    store_norm(i, *reinterpret_cast<const u32x4*>(x + row + i), *reinterpret_cast<const u32x4*>(w + i));
}

// qkv [M][(Hq + 2 Hkv) D] (the fused projection's output, bias included) -> q_out [M][Hq][D] with RoPE; k (with
// RoPE) and v written to k_cache / v_cache [Hkv][L][D] at row positions[m]. One thread per (token, head, dim pair
// (i, i + 64)), RoPE by rope_pair. permuted: qkv holds each head's rows in the RoPE-permuted order (rope_row), as the
// fused decoder's W4A16 q|k|v projection writes them.
__global__ __launch_bounds__(256) void rope_kv_kernel(const f16* __restrict__ qkv, const int64_t* __restrict__ pos,
                                                      const float* __restrict__ inv_freq, f16* __restrict__ q_out,
                                                      f16* __restrict__ k_cache, f16* __restrict__ v_cache, int M,
                                                      int Hq, int Hkv, int L, bool permuted) {
  const int heads = Hq + 2 * Hkv;
  const int gid = blockIdx.x * blockDim.x + threadIdx.x;
  const int i = gid & 63, h = (gid >> 6) % heads, m = (gid >> 6) / heads;
  if (m >= M) return;
  const int64_t p = pos[m];
  if (p < 0 || p >= L) return;                               // the host checks positions; never write out of bounds
  const f16* src = qkv + ((size_t)m * heads + h) * kHeadDim;
  const int s1 = permuted ? rope_row(i) : i, s2 = permuted ? rope_row(i) + 8 : i + 64;   // dims i and i + 64
  if (h >= Hq + Hkv) {                                       // v: plain copy into the cache
    f16* dst = v_cache + ((size_t)(h - Hq - Hkv) * L + p) * kHeadDim;
    dst[i] = src[s1];
    dst[i + 64] = src[s2];
    return;
  }
  f16 o1, o2;
  rope_pair(src[s1], src[s2], p, inv_freq[i], o1, o2);
  f16* dst = h < Hq ? q_out + ((size_t)m * Hq + h) * kHeadDim : k_cache + ((size_t)(h - Hq) * L + p) * kHeadDim;
  dst[i] = o1;
  dst[i + 64] = o2;
}

// Causal GQA attention for M query tokens at positions pos[m] over the cache rows 0 .. pos[m]:
// out[m][h * D + d] = sum_j softmax_j(scale * q[m][h] . k[j]) v[j][d], KV head h / (Hq / Hkv) for query head h.
// One block of W waves per (token, group of G consecutive query heads of one KV head): G = Hq / Hkv shares every K/V
// read among the heads; G = 1 gives Hq / Hkv times more blocks (decode steps, where M Hkv blocks cannot fill the
// chip). Lane l always owns dims 8 (l % 16) .. + 7 and key row-group l / 16: each 16-byte K and V load of a wave
// reads four whole cache rows, the lane's slice of q stays in registers, a score is a 16-lane DPP sum, and the
// probabilities never leave the lane that multiplies them into V. Waves take blocks of KB keys; the row groups and
// the waves are merged at the end (lane shuffles, then LDS).
// When (token, group) blocks alone cannot fill the chip (a decode step), the keys are also split into P partitions
// of CH keys (grid.y): each block writes its partial (max, sum, unnormalized output) to the workspace and
// attention_combine, launched next, merges the P partials in partition order (merge_partitions). A merge by the last
// block to arrive (agent-coherent partial stores, an arrival counter per (token, group)) measured slower in graph
// decode (3B: 1.139 against 1.124 ms/token): phase stamps put 1.8 us on the arrival count alone, the P blocks of a
// (token, group) incrementing one counter, and 2.6 us on the last block's merge, against ~3 us for the key loop.
// Output dim d of one (block, head) from the P <= kAttnMaxParts partial records (kAttnRec floats) at float index `first`,
// `stride` floats apart: max over partitions, then the rescaled sums in partition order (partitions that saw no key
// hold max = -inf and are skipped; partition 0 always holds key 0). The loops run to the compile-time bound, so all
// the loads are requested before the first is used.
__device__ __forceinline__ float merge_partitions(__amdgpu_buffer_rsrc_t pr, int first, int stride, int P, int d) {
  float pm[kAttnMaxParts], ps[kAttnMaxParts], po[kAttnMaxParts];
#pragma unroll
  for (int p = 0; p < kAttnMaxParts; ++p) {
    const int at = 4 * (first + p * stride);
    const bool live = p < P;
    pm[p] = live ? load_partial(pr, at) : -INFINITY;
    ps[p] = live ? load_partial(pr, at + 4) : 0.f;
    po[p] = live ? load_partial(pr, at + 4 * (4 + d)) : 0.f;
  }
  float gm = -INFINITY;
#pragma unroll
  for (int p = 0; p < kAttnMaxParts; ++p) gm = fmaxf(gm, pm[p]);
  float num = 0.f, den = 0.f;
#pragma unroll
  for (int p = 0; p < kAttnMaxParts; ++p) {
    if (pm[p] == -INFINITY) continue;
    const float f = expf(pm[p] - gm);
    num = fmaf(f, po[p], num);
    den = fmaf(f, ps[p], den);
  }
  return num / den;
}

template <int G, int KB>
__global__ __launch_bounds__(G == 1 && KB == 32 ? 1024 : 512) void attention_kernel(
    const f16* __restrict__ q, const f16* __restrict__ k_cache, const f16* __restrict__ v_cache,
    const int64_t* __restrict__ pos, f16* __restrict__ out, int Hq, int Hkv, int L, float scale, int CH,
    float* __restrict__ part) {
  constexpr int NI = KB / 4;                                 // 16-byte loads per lane and step, per K and per V
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  args_in_sgprs(q, k_cache, v_cache, pos, out, Hq, Hkv, L, CH, part, (int)blockDim.x);
  const int groups = Hq / G, P = gridDim.y, pid = blockIdx.y;
  const int m = blockIdx.x / groups, h0 = (blockIdx.x % groups) * G, hk = h0 / (Hq / Hkv);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), W = blockDim.x >> 6;
  const int rg = lane >> 4, dl = (lane & 15) * 8;          // key row-group, first dim of the lane's slice
  const int64_t pm = pos[m];
  const int nkeys = (int)min((int64_t)L, pm + 1), last = nkeys - 1;
  const int kbeg = pid * CH, kend = pid == P - 1 ? nkeys : min(nkeys, kbeg + CH);   // this block's keys
  u32x4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qv[g] = *reinterpret_cast<const u32x4*>(q + ((size_t)m * Hq + h0 + g) * kHeadDim + dl);
  const f16* kb = k_cache + (size_t)hk * L * kHeadDim + dl;
  const f16* vb = v_cache + (size_t)hk * L * kHeadDim + dl;
  float mx[G], sum[G], o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    mx[g] = -INFINITY;
    sum[g] = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) o[g][d] = 0.f;
  }
  for (int base = kbeg + wave * KB; base < kend; base += KB * W) {
    // step keys base + 4 i + rg, i < NI (rows past the end are clamped and masked)
    u32x4 kq[NI], vq[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) kq[i] = *reinterpret_cast<const u32x4*>(kb + (size_t)min(base + 4 * i + rg, last) * kHeadDim);
#pragma unroll
    for (int i = 0; i < NI; ++i) vq[i] = *reinterpret_cast<const u32x4*>(vb + (size_t)min(base + 4 * i + rg, last) * kHeadDim);
    __builtin_amdgcn_sched_barrier(0);                      // every load requested before the first is used
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s[NI];
      float bm = -INFINITY;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) a = dot2(as_f16x2(qv[g][e]), as_f16x2(kq[i][e]), a);
        a = row_sum(a) * scale;                              // the key's score, in all 16 lanes of the row group
        s[i] = base + 4 * i + rg < kend ? a : -INFINITY;
        bm = fmaxf(bm, s[i]);
      }
      bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64));                // the step's max over all its keys
      const float nm = fmaxf(mx[g], bm);
      const float corr = __expf(mx[g] - nm);                 // 0 on the first step (mx = -inf)
      float ps = 0.f;
#pragma unroll
      for (int d = 0; d < 8; ++d) o[g][d] *= corr;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const float pj = __expf(s[i] - nm);                  // 0 for masked keys
        ps += pj;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f16x2 v2 = as_f16x2(vq[i][e]);
          o[g][2 * e] = fmaf(pj, (float)v2[0], o[g][2 * e]);
          o[g][2 * e + 1] = fmaf(pj, (float)v2[1], o[g][2 * e + 1]);
        }
      }
      ps += __shfl_xor(ps, 16, 64);                           // + the other row groups' keys: the step's total
      ps += __shfl_xor(ps, 32, 64);
      sum[g] = sum[g] * corr + ps;
      mx[g] = nm;
    }
  }
  // merge the four row groups (lanes l, l ^ 16, l ^ 32, l ^ 48 hold the same dims), then the waves through LDS
  float* st = reinterpret_cast<float*>(smem);                // [W][G] (max, sum)
  float* os = st + W * G * 2;                                // [W][G][D]
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      o[g][d] += __shfl_xor(o[g][d], 16, 64);
      o[g][d] += __shfl_xor(o[g][d], 32, 64);
    }
    if (lane == 0) {
      st[(wave * G + g) * 2] = mx[g];
      st[(wave * G + g) * 2 + 1] = sum[g];
    }
    if (rg == 0) {
#pragma unroll
      for (int d = 0; d < 8; ++d) os[(wave * G + g) * kHeadDim + dl + d] = o[g][d];
    }
  }
  __syncthreads();
  // partial of this block: [G][2 + D] floats (max, sum, then the unnormalized output), per (token, group, partition)
  float* mine = part + (size_t)(blockIdx.x * P + pid) * G * kAttnRec;
  for (int idx = threadIdx.x; idx < G * kHeadDim; idx += blockDim.x) {
    const int g = idx / kHeadDim, d = idx % kHeadDim;
    float gm = -INFINITY;
    for (int w = 0; w < W; ++w) gm = fmaxf(gm, st[(w * G + g) * 2]);
    float num = 0.f, den = 0.f;
    for (int w = 0; w < W; ++w) {
      const float wm = st[(w * G + g) * 2];
      if (wm == -INFINITY) continue;                          // a wave that saw no key
      const float f = expf(wm - gm);
      num = fmaf(f, os[(w * G + g) * kHeadDim + d], num);
      den = fmaf(f, st[(w * G + g) * 2 + 1], den);
    }
    if (P == 1) {
      out[((size_t)m * Hq + h0 + g) * kHeadDim + d] = (f16)(num / den);
    } else {
      mine[g * kAttnRec + 4 + d] = num;
      if (d == 0) {
        mine[g * kAttnRec] = gm;
        mine[g * kAttnRec + 1] = den;
      }
    }
  }
}

// out[m][h][d] from the P <= kAttnMaxParts partials of attention_kernel or attention_mfma (merge_partitions), launched
// after it
__global__ __launch_bounds__(256) void attention_combine(const float* __restrict__ part, f16* __restrict__ out,
                                                         int blocks, int G, int P, int Hq) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= blocks * G * kHeadDim) return;
  const int b = idx / (G * kHeadDim), g = (idx / kHeadDim) % G, d = idx % kHeadDim;
  const int groups = Hq / G, m = b / groups, h = (b % groups) * G + g;
  const __amdgpu_buffer_rsrc_t pr = make_rsrc(part, (uint32_t)(blocks * P * G * kAttnRec * 4));
  out[((size_t)m * Hq + h) * kHeadDim + d] =
      (f16)merge_partitions(pr, b * P * G * kAttnRec + g * kAttnRec, G * kAttnRec, P, d);
}

// Causal GQA attention on MFMA for multi-token steps and prompts (same contract as attention_kernel): one wave per
// (KV head, 16 query rows, key partition), the query rows of a KV head numbered row = token * G + head-in-group.
// Per block of 32 keys (v_mfma_f32_16x16x32_f16):
//   S^T = K Q^T: A = 16 keys x 32 dims (lane (r, c): key kb + 8 (r / 4) + r % 4 + 4 t, 16 bytes of its row), B = the
//   wave's 16 query rows x 32 dims (held in registers), two key tiles t x four 32-dim steps; the key order is chosen so
//   that lane (r, c) ends up with the scores of query row r at keys kb + 8 c .. kb + 8 c + 7;
//   online softmax per query row (max and sum over the four lanes r, r + 16, r + 32, r + 48), masked past the row's
//   position; the probabilities, split into an fp16 head and an fp16 remainder (together exact to ~2^-22), are the
//   B operands of the next product (two MFMAs per dim tile, so the weights carry fp32 accuracy as in
//   attention_kernel);
//   O^T += V^T P^T: A = 16 dims x 32 keys of V^T, which the wave writes to its own LDS from its 8 KB of V rows
//   (4 keys x 8 dims per lane, packed into 8-byte rows of V^T) and reads back as 16-byte fragments; eight dim tiles.
// A wave touches only its own LDS, in order, so no barrier is needed. With P > 1 each wave writes the partial (max,
// sum, unnormalized output) of its rows in attention_kernel's layout and attention_combine merges them.
constexpr int kAttnVtPitch = 80;                            // bytes per dim row of the staged V^T (64 + 16 padding)

__global__ __launch_bounds__(64) void attention_mfma(const f16* __restrict__ q, const f16* __restrict__ k_cache,
                                                     const f16* __restrict__ v_cache, const int64_t* __restrict__ pos,
                                                     f16* __restrict__ out, int M, int Hq, int Hkv, int L, float scale,
                                                     float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) uint8_t vt[kHeadDim * kAttnVtPitch];
  args_in_sgprs(q, k_cache, v_cache, pos, out, M, Hq, Hkv, L, part);
  const int G = Hq / Hkv, P = gridDim.y, pid = blockIdx.y;
  const int hk = blockIdx.x % Hkv, tile = blockIdx.x / Hkv;
  const int lane = threadIdx.x, r = lane & 15, c = lane >> 4;
  // this lane's query row (as the B column r)
  const int row = 16 * tile + r, m = row / G, g = row - m * G;
  const bool live = m < M;
  const int pr = live ? (int)min((int64_t)L - 1, pos[m]) : -1;  // last key the row attends
  int wmax = pr;                                               // the wave's last key
  wmax = max(wmax, __shfl_xor(wmax, 1, 64));
  wmax = max(wmax, __shfl_xor(wmax, 2, 64));
  wmax = max(wmax, __shfl_xor(wmax, 4, 64));
  wmax = max(wmax, __shfl_xor(wmax, 8, 64));
  // the P partitions split the keys this wave attends (not the caller's bound on them) in whole 32-key blocks
  const int ch = ((wmax + 1 + P - 1) / P + 31) / 32 * 32;
  const int kbeg = pid * ch, kend = min(wmax + 1, kbeg + ch);
  const __amdgpu_buffer_rsrc_t qr = make_rsrc(q, (uint32_t)M * (uint32_t)Hq * kHeadDim * 2u);
  const int qoff = live ? ((m * Hq + hk * G + g) * kHeadDim + 8 * c) * 2 : kOutOfRange;
  f16x8 qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) qf[ks] = __builtin_bit_cast(f16x8, buffer_load16(qr, qoff + 64 * ks));
  const f16* kh = k_cache + (size_t)hk * L * kHeadDim;
  const f16* vh = v_cache + (size_t)hk * L * kHeadDim;
  const int kr = 8 * (r >> 2) + (r & 3);                      // key of A row r in tile 0 (tile 1: + 4)
  float mx = -INFINITY, lsum = 0.f;
  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // K and V rows are read in whole 32-key blocks, clamped to the wave's last attended key: rows past it may never
  // have been written (NaN or Inf in an uninitialized cache), and a masked key's weight 0 times NaN is still NaN in
  // the P V product
  for (int kb = kbeg; kb < kend; kb += 32) {
    u32x4 kf[2][4], vf[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const f16* krow = kh + (size_t)min(kb + kr + 4 * t, wmax) * kHeadDim + 8 * c;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kf[t][ks] = *reinterpret_cast<const u32x4*>(krow + 32 * ks);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)                               // V rows kb + 4 (lane % 8) + j, dims 8 (lane / 8 + 8 u)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        vf[u][j] = *reinterpret_cast<const u32x4*>(vh + (size_t)min(kb + 4 * (lane & 7) + j, wmax) * kHeadDim +
                                                   8 * ((lane >> 3) + 8 * u));
    f32x4 st[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      st[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        st[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, kf[t][ks]), qf[ks], st[t], 0, 0, 0);
    }
    // V^T rows (dim) x 4 keys per lane into the wave's LDS
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int d0 = 8 * ((lane >> 3) + 8 * u);
#pragma unroll
      for (int e = 0; e < 4; ++e) {                           // dims d0 + 2 e, d0 + 2 e + 1
        const uint32_t a0 = vf[u][0][e], a1 = vf[u][1][e], a2 = vf[u][2][e], a3 = vf[u][3][e];
        // v_perm picks bytes of {a1, a0}: 0x05040100 the low halves (a0, a1), 0x07060302 the high halves
        const uint2 lo = make_uint2(__builtin_amdgcn_perm(a1, a0, 0x05040100u),
                                    __builtin_amdgcn_perm(a3, a2, 0x05040100u));
        const uint2 hi = make_uint2(__builtin_amdgcn_perm(a1, a0, 0x07060302u),
                                    __builtin_amdgcn_perm(a3, a2, 0x07060302u));
        *reinterpret_cast<uint2*>(vt + (d0 + 2 * e) * kAttnVtPitch + 8 * (lane & 7)) = lo;
        *reinterpret_cast<uint2*>(vt + (d0 + 2 * e + 1) * kAttnVtPitch + 8 * (lane & 7)) = hi;
      }
    }
    // scores of row r at keys kb + 8 c + i (i = 4 t + v), masked past the row's position and the partition
    float sc[8], bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = kb + 8 * c + i;
      sc[i] = key <= pr && key < kend ? st[i >> 2][i & 3] * scale : -INFINITY;
      bm = fmaxf(bm, sc[i]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float nm = fmaxf(mx, bm);
    const float corr = nm == -INFINITY ? 1.f : __expf(mx - nm);   // 0 on the first block with a key
    f16x8 ph, pl;                                           // p = ph + pl to ~2^-22: fp32-accurate weights
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float pj = nm == -INFINITY ? 0.f : __expf(sc[i] - nm);
      ps += pj;
      ph[i] = (f16)pj;
      pl[i] = (f16)(pj - (float)ph[i]);
    }
    lsum = lsum * corr + ps;
    mx = nm;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f16x8 va = *reinterpret_cast<const f16x8*>(vt + (16 * dt + r) * kAttnVtPitch + 16 * c);
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph, o[dt] * corr, 0, 0, 0);
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, o[dt], 0, 0, 0);
    }
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (!live) return;
  // lane (r, c) holds O^T[16 dt + 4 c + v][row r]
  if (P == 1) {
    f16* dst = out + ((size_t)m * Hq + hk * G + g) * kHeadDim + 4 * c;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f16x2 lo = {(f16)(o[dt][0] / lsum), (f16)(o[dt][1] / lsum)};
      const f16x2 hi = {(f16)(o[dt][2] / lsum), (f16)(o[dt][3] / lsum)};
      *reinterpret_cast<uint2*>(dst + 16 * dt) = make_uint2(as_u32(lo), as_u32(hi));
    }
    return;
  }
  float* mine = part + (((size_t)(m * Hkv + hk) * P + pid) * G + g) * kAttnRec;
  if (c == 0) {
    mine[0] = mx;
    mine[1] = lsum;
  }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(mine + 4 + 16 * dt + 4 * c) = o[dt];
}

// fp16 GEMV for the (tied) lm_head, M <= 4: y[m][n] = fp16(sum_k x[m][k] W[n][k]), W fp16 [N][K] row-major, fp32
// accumulation. A bandwidth kernel: the workgroup stages x[M][K] in LDS once (one barrier), then each wave streams
// RW weight rows with 16-byte non-temporal loads (lane l takes k = 512 c + 8 l .. + 7 of chunk c, so every load is
// one contiguous 1 KB), kHeadChunks chunks of every row in flight, dot2 against x from LDS, and a wave reduction per
// row. Two rows per wave, four chunks each (MI355X graph, 3 cold copies of the 151936 x 2048 Qwen2.5 head): 94.3 us
// (6.6 TB/s) against 102.3 for 8 rows and two chunks, 99.0 for 4 and two, 96.2 for one row and four; same bits.
constexpr int kHeadChunks = 4;

// The greedy pick's order on (fp16 logit, index) as one 64-bit key, larger = picked, as torch.argmax picks: the larger
// value (-0 equal to +0, a NaN above every number), then the smaller index. Zero is below every key.
__device__ __forceinline__ uint64_t pick_key(uint16_t b, int idx) {
  uint32_t k;
  if ((b & 0x7FFFu) > 0x7C00u) {
    k = 0x10000u;                                            // NaN
  } else {
    if (b == 0x8000u) b = 0;                                 // -0 ties with +0
    k = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);      // fp16 order as unsigned order
  }
  return ((uint64_t)k << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)idx);
}

// PICK (M = 1): each workgroup also writes the key of its largest logit (as stored, fp16) to pick[blockIdx.x], for
// head_pick_kernel
template <int M, int RW, int CH = kHeadChunks, bool PICK = false>
__global__ __launch_bounds__(256) void gemv_f16_kernel(const f16* __restrict__ x, const f16* __restrict__ w,
                                                       f16* __restrict__ y, int N, int K, uint64_t* __restrict__ pick,
                                                       int mrows) {
  static_assert(!PICK || M == 1, "the greedy pick takes one row");
  // M rows compiled in, mrows <= M of them real (x staged and y stored for those; the rest computes on stale LDS)
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  u32x4* xs = reinterpret_cast<u32x4*>(smem);               // [M][K / 8]
  // wave through readfirstlane: the row buffer resource below is then known uniform and stays in scalar registers
  // (from a per-lane value every weight load becomes a waterfall loop)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kp = K >> 3;                                     // 16-byte pieces per row
  for (int i = threadIdx.x; i < mrows * kp; i += blockDim.x) xs[i] = *reinterpret_cast<const u32x4*>(x + 8 * (size_t)i);
  __syncthreads();
  const int n0 = (blockIdx.x * 4 + wave) * RW;
  if (!PICK && n0 >= N) return;                             // (PICK: every wave reaches the barrier below; one past N
                                                             // reads nothing and stores nothing)
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(w + (size_t)min(n0, N) * K, (uint32_t)(max(0, min(RW, N - n0)) * K * 2));
  float acc[RW][M];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
  const int nc = (kp + 63) >> 6;                             // 512-k chunks
  for (int c0 = 0; c0 < nc; c0 += CH) {
    u32x4 wv[CH][RW];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int p = 64 * (c0 + u) + lane;                    // this lane's piece of the chunk
#pragma unroll
      for (int r = 0; r < RW; ++r) wv[u][r] = buffer_load16_nt(wr, p < kp ? 2 * (r * K + 8 * p) : kOutOfRange);
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int p = 64 * (c0 + u) + lane;
      if (p >= kp) break;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const u32x4 xv = xs[m * kp + p];
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[r][m] = dot2(as_f16x2(wv[u][r][e]), as_f16x2(xv[e]), acc[r][m]);
      }
    }
  }
  uint64_t best = 0;
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float v = wave_sum(acc[r][m]);
      if (lane == 0 && n0 + r < N && m < mrows) {
        const f16 h = (f16)v;
        y[(size_t)m * N + n0 + r] = h;
        if constexpr (PICK) {
          const uint64_t kv = pick_key(__builtin_bit_cast(uint16_t, h), n0 + r);
          best = kv > best ? kv : best;
        }
      }
    }
  if constexpr (PICK) {
    __shared__ uint64_t red[4];
    if (lane == 0) red[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
      for (int v = 1; v < 4; ++v) best = red[v] > best ? red[v] : best;
      pick[blockIdx.x] = best;
    }
  }
}

// The greedy pick and its feedback, one workgroup: the largest of the head workgroups' keys (pick[0 .. n)) gives the
// index; tokens[0] = index, positions[0] += 1 (positions may be null), out[*out_count] = index while *out_count <
// out_cap and *out_count + 1 (out_count may be null), and h_out[0 .. H) = embed row index (embed may be null): the next
// step's input, so that a one-token step needs no embedding gather of its own
constexpr int kPickThreads = 1024;
__global__ __launch_bounds__(kPickThreads) void head_pick_kernel(const uint64_t* __restrict__ pick, int n,
                                                                 int64_t* tokens, int64_t* positions, int64_t* out,
                                                                 int out_cap, int* out_count,
                                                                 const f16* __restrict__ embed, int H, f16* h_out) {
  __shared__ uint64_t red[kPickThreads / 64];
  __shared__ int s_idx;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint64_t best = 0;
  for (int i0 = tid; i0 < n; i0 += 8 * kPickThreads) {      // eight loads in flight per thread
    uint64_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = i0 + u * kPickThreads < n ? pick[i0 + u * kPickThreads] : 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) best = v[u] > best ? v[u] : best;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t o = __shfl_xor(best, off, 64);
    best = o > best ? o : best;
  }
  if (lane == 0) red[wave] = best;
  __syncthreads();
  if (tid == 0) {
    for (int v = 1; v < kPickThreads / 64; ++v) best = red[v] > best ? red[v] : best;
    const int idx = (int)(0xFFFFFFFFu - (uint32_t)best);
    s_idx = idx;
    tokens[0] = idx;
    if (positions) positions[0] += 1;
    if (out_count) {
      const unsigned c = (unsigned)*out_count;               // (a count past INT_MAX stays out of range)
      if (c < (unsigned)out_cap) out[c] = idx;
      *out_count = (int)(c + 1u);
    }
  }
  if (embed == nullptr) return;                              // (uniform)
  __syncthreads();
  const u32x4* src = reinterpret_cast<const u32x4*>(embed + (size_t)s_idx * H);
  for (int i = tid; i < (H >> 3); i += kPickThreads) reinterpret_cast<u32x4*>(h_out)[i] = src[i];
}

constexpr int kHeadRows = 2;                                // RW: rows per wave (4 waves a workgroup)

// fp16-weight MFMA GEMV for the head beyond 8 rows (up to 64: MT 16-row activation tiles), where the dot2 kernel above
// turns ALU-bound. Each wave owns one 16-row tile of W, the MFMA's A, straight from global: lane (r, q) takes row r,
// k = 128 c + 32 s + 8 q + 0..7 as k-step s of chunk c, so one load instruction reads 64 contiguous bytes of each of
// 16 rows (kF16wSlots chunks in flight, default cache policy: with non-temporal loads the half-used 128-byte lines
// were fetched twice, 199 against 135 us). The workgroup's four waves share each 128-k chunk of x (B, the same k
// order), staged by all 256 threads into one of two LDS buffers (16-byte pieces XOR-swizzled by row, so a B
// fragment's 16 rows hit different banks) while the previous chunk is consumed, one barrier per chunk; rows past M
// read zeros and are not stored. Lane l holds y[16 mt + l % 16][16 t + 4 (l / 16) + v], v = 0..3. On the 151936 x 2048
// head (3 cold copies): 16 rows 135 us against 204 for hipBLASLt, 32 rows 142 against 146, 48 rows 152 against 144
// (hipBLASLt keeps those), the same as with x staged whole in LDS at 16 rows.
constexpr int kF16wSlots = 4;
template <int MT>
__global__ __launch_bounds__(256) void gemm_f16w_rows_kernel(const f16* __restrict__ x, const f16* __restrict__ w,
                                                             f16* __restrict__ y, int M, int N, int K) {
  constexpr int kRows = 16 * MT, kBuf = kRows * 256;        // one staged chunk of x: kRows rows x 256 bytes
  constexpr int XP = kRows * 16 / 256;                     // 16-byte pieces a thread stages per chunk
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q = lane >> 4, KC = K >> 7;
  const int n0 = 16 * (blockIdx.x * 4 + wave);
  const int rows = max(0, min(16, N - n0));
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(w + (size_t)min(n0, N) * K, (uint32_t)(rows * K * 2));
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)(M * K * 2));
  const int woff = r < rows ? 2 * (r * K + 8 * q) : kOutOfRange;
  auto slot = [](int row, int piece) { return 16 * (16 * row + (piece ^ (row & 15))); };   // byte offset in a buffer
  int xoff[XP], xsl[XP];
#pragma unroll
  for (int u = 0; u < XP; ++u) {                            // piece p = tid + 256 u: row p / 16, piece p % 16
    const int p = tid + 256 * u;
    xoff[u] = (p >> 4) < M ? 2 * ((p >> 4) * K + 8 * (p & 15)) : kOutOfRange;
    xsl[u] = slot(p >> 4, p & 15);
  }
  u32x4 ring[kF16wSlots][4], rx[XP];
  auto issue = [&](int d, int c) {
#pragma unroll
    for (int s = 0; s < 4; ++s) ring[d][s] = buffer_load16(wr, c < KC ? woff + 2 * (128 * c + 32 * s) : kOutOfRange);
  };
  auto load_x = [&](int c) {
#pragma unroll
    for (int u = 0; u < XP; ++u) rx[u] = buffer_load16(xr, c < KC ? xoff[u] + 256 * c : kOutOfRange);
  };
  auto stage_x = [&](int b) {
#pragma unroll
    for (int u = 0; u < XP; ++u) *reinterpret_cast<u32x4*>(smem + b * kBuf + xsl[u]) = rx[u];
  };
  load_x(0);
#pragma unroll
  for (int d = 0; d < kF16wSlots; ++d) issue(d, d);
  stage_x(0);
  __syncthreads();
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < KC; c0 += kF16wSlots) {
#pragma unroll
    for (int d = 0; d < kF16wSlots; ++d) {
      const int c = c0 + d;
      if (c < KC) {                                         // uniform: every wave runs the same chunks
        load_x(c + 1);
        const uint8_t* xb = smem + (c & 1) * kBuf;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const u32x4 b = *reinterpret_cast<const u32x4*>(xb + slot(16 * mt + r, 4 * s + q));
            acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, ring[d][s]),
                                                             __builtin_bit_cast(f16x8, b), acc[mt], 0, 0, 0);
          }
        issue(d, c + kF16wSlots);
        if (c + 1 < KC) stage_x((c + 1) & 1);
        __syncthreads();
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + r, n = n0 + 4 * q;
    if (m < M && n < N) {
      f16* dst = y + (size_t)m * N + n;
      if (n + 4 <= N && (reinterpret_cast<uintptr_t>(dst) & 7) == 0) {
        const f16x2 lo = {(f16)acc[mt][0], (f16)acc[mt][1]}, hi = {(f16)acc[mt][2], (f16)acc[mt][3]};
        *reinterpret_cast<uint2*>(dst) = make_uint2(as_u32(lo), as_u32(hi));
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (n + v < N) dst[v] = (f16)acc[mt][v];
      }
    }
  }
}

hipError_t gemm_f16w_rows_launch(const f16* x, const f16* w, f16* y, int M, int N, int K, hipStream_t st) {
  const dim3 grid((unsigned)((N + 63) / 64)), block(256);
  const int MT = (M + 15) / 16;
  const size_t lds = (size_t)2 * 16 * MT * 256;
  switch (MT) {
    case 1: return launch(gemm_f16w_rows_kernel<1>, grid, block, lds, st, x, w, y, M, N, K);
    case 2: return launch(gemm_f16w_rows_kernel<2>, grid, block, lds, st, x, w, y, M, N, K);
    case 3: return launch(gemm_f16w_rows_kernel<3>, grid, block, lds, st, x, w, y, M, N, K);
    default: return launch(gemm_f16w_rows_kernel<4>, grid, block, lds, st, x, w, y, M, N, K);
  }
}

namespace {
template <int M, int RW, int CH>
hipError_t launch_head(const f16* x, const f16* w, f16* y, int mrows, int N, int K, hipStream_t st) {
  const dim3 grid((unsigned)((N + 4 * RW - 1) / (4 * RW))), block(256);
  return launch(gemv_f16_kernel<M, RW, CH>, grid, block, (size_t)M * K * 2, st, x, w, y, N, K, nullptr, mrows);
}
}  // namespace

hipError_t gemv_f16_launch(const f16* x, const f16* w, f16* y, int M, int N, int K, hipStream_t st) {
  switch (M) {
    case 1: return launch_head<1, kHeadRows, kHeadChunks>(x, w, y, 1, N, K, st);
    case 2: return launch_head<2, kHeadRows, kHeadChunks>(x, w, y, 2, N, K, st);
    case 3: return launch_head<3, kHeadRows, kHeadChunks>(x, w, y, 3, N, K, st);
    case 4: return launch_head<4, kHeadRows, kHeadChunks>(x, w, y, 4, N, K, st);
    // more rows: 8 weight rows per wave, two chunks in flight (the head, 3 cold copies: 8 rows 119.5 us against
    // 126.6 for 4 per wave and 163.7 for 2; hipBLASLt 203.6. 16 rows: 206 us, level with hipBLASLt's 204: the dot2
    // sequence per weight byte grows with the rows and the kernel turns ALU-bound)
    default: {
      const bool x_fits = (size_t)M * K * 2 <= 65536;      // the dot2 kernels stage x whole
      if (M <= 8 && x_fits) return launch_head<8, 8, 2>(x, w, y, M, N, K, st);
      if (K % 128) return x_fits && M <= 16 ? launch_head<16, 8, 2>(x, w, y, M, N, K, st) : hipErrorInvalidValue;
      return gemm_f16w_rows_launch(x, w, y, M, N, K, st);
    }
  }
}

int head_pick_parts(int N) { return (N + 4 * kHeadRows - 1) / (4 * kHeadRows); }

hipError_t head_pick_launch(const f16* x, const f16* w, f16* y, int N, int K, uint64_t* pick, int64_t* tokens,
                            int64_t* positions, int64_t* out, int out_cap, int* out_count, const f16* embed, f16* h_out,
                            hipStream_t st) {
  const int parts = head_pick_parts(N);
  if (hipError_t e = launch(gemv_f16_kernel<1, kHeadRows, kHeadChunks, true>, dim3(parts), dim3(256), (size_t)K * 2, st,
                            x, w, y, N, K, pick, 1))
    return e;
  return launch(head_pick_kernel, dim3(1), dim3(kPickThreads), 0, st, pick, parts, tokens, positions, out, out_cap,
                out_count, embed, K, h_out);
}

hipError_t rmsnorm_launch(const f16* x, const f16* w, f16* out, int M, int H, float eps, hipStream_t st) {
  return launch(rmsnorm_kernel, dim3(M), dim3(256), 0, st, x, w, out, H, eps);
}

// table[m][i] = fp16 (cos, sin) of positions[m] * inv_freq[i] (rope_cos_sin): the RoPE factors of a step, shared by
// every head and layer; the multi-row q|k|v GEMMs read them in their store
__global__ __launch_bounds__(256) void rope_table_kernel(const int64_t* __restrict__ pos, const float* __restrict__ inv_freq,
                                                         uint32_t* __restrict__ table, int M) {
  const int gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= M * 64) return;
  f16 c, s;
  rope_cos_sin(pos[gid >> 6], inv_freq[gid & 63], c, s);
  table[gid] = as_u32(f16x2{c, s});
}

hipError_t rope_table_launch(const int64_t* pos, const float* inv_freq, uint32_t* table, int M, hipStream_t st) {
  return launch(rope_table_kernel, dim3((unsigned)((M * 64 + 255) / 256)), dim3(256), 0, st, pos, inv_freq, table, M);
}

hipError_t rope_kv_launch(const f16* qkv, const int64_t* pos, const float* inv_freq, f16* q_out, f16* k_cache,
                          f16* v_cache, int M, int Hq, int Hkv, int L, bool permuted, hipStream_t st) {
  const long threads = (long)M * (Hq + 2 * Hkv) * 64;
  return launch(rope_kv_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, qkv, pos, inv_freq, q_out,
                k_cache, v_cache, M, Hq, Hkv, L, permuted);
}

namespace {
// combine = false: the partials are left for the caller (their count in *parts; with one partition the kernel writes
// out itself and *parts is 1)
template <int G, int KB>
hipError_t launch_attention(const f16* q, const f16* k, const f16* v, const int64_t* pos, f16* out, int M, int Hq,
                            int Hkv, int L, int max_keys, float scale, void* ws, size_t ws_bytes, hipStream_t st,
                            int max_parts = kAttnMaxParts, bool combine = true, int* parts = nullptr) {
  const int max_waves = (G == 1 && KB == 32) ? 16 : 8;
  const long blocks = (long)M * (Hq / G);
  // key partitions: when the (token, group) blocks cannot fill the chip, split the keys so that about
  // kAttnTargetBlocks blocks run, each with at least kAttnMinKeys keys, within the workspace
  int P = 1;
  if (ws && ws_bytes > kAttnCounterBytes && blocks < kAttnTargetBlocks && max_keys >= kAttnMinSplitKeys) {
    P = (int)std::min<long>({(kAttnTargetBlocks + blocks - 1) / blocks, (max_keys + kAttnMinKeys - 1) / kAttnMinKeys,
                             (long)max_parts});
    const size_t per = (size_t)blocks * G * kAttnRec * sizeof(float);
    P = (int)std::max<size_t>(1, std::min<size_t>((size_t)P, (ws_bytes - kAttnCounterBytes) / per));
  }
  const int CH = ((max_keys + P - 1) / P + KB - 1) / KB * KB;   // keys per partition, whole steps
  P = (max_keys + CH - 1) / CH;
  int waves = 1;                                              // enough waves to give each one step of keys
  while (waves < max_waves && waves * KB < CH) waves *= 2;
  // prefill-sized launches (many blocks) take at most 4 waves per block: merging 8 waves' partial outputs through LDS
  // costs more than the keys they share out (measured: 3B prompt of 512 tokens 58 -> 48 us, 7B 99 -> 70 us)
  if (blocks * P >= kAttnManyBlocks && waves > 4) waves = 4;
  const size_t lds = (size_t)waves * G * 2 * 4 + (size_t)waves * G * kHeadDim * 4;
  float* part = ws ? reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kAttnCounterBytes) : nullptr;
  if (parts) *parts = P;
  hipError_t e = launch(attention_kernel<G, KB>, dim3((unsigned)blocks, P), dim3(64 * waves), lds, st, q, k, v, pos,
                        out, Hq, Hkv, L, scale, CH, part);
  if (e != hipSuccess || P == 1 || !combine) return e;
  const long threads = (long)M * Hq * kHeadDim;
  return launch(attention_combine, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, part, out, (int)blocks, G,
                P, Hq);
}
// multi-token steps and prompts on MFMA: one wave per (KV head, 16 query rows, key partition); partitions while the
// waves number fewer than kAttnMfmaTargetWaves, at most one per kAttnMinKeys of max_keys, within the workspace (each
// wave splits the keys its rows actually attend, so a bound well above the real count costs nothing)
hipError_t launch_attention_mfma(const f16* q, const f16* k, const f16* v, const int64_t* pos, f16* out, int M,
                                 int Hq, int Hkv, int L, int max_keys, float scale, void* ws, size_t ws_bytes,
                                 hipStream_t st) {
  const int G = Hq / Hkv;
  const long waves = (long)((M * G + 15) / 16) * Hkv;
  int P = 1;
  if (ws && ws_bytes > kAttnCounterBytes && waves < kAttnMfmaTargetWaves && max_keys >= 2 * kAttnMinKeys) {
    P = (int)std::min<long>({(kAttnMfmaTargetWaves + waves - 1) / waves, (max_keys + kAttnMinKeys - 1) / kAttnMinKeys,
                             (long)kAttnMaxParts});
    const size_t per = (size_t)M * Hkv * G * kAttnRec * sizeof(float);
    P = (int)std::max<size_t>(1, std::min<size_t>((size_t)P, (ws_bytes - kAttnCounterBytes) / per));
  }
  // the partials after the workspace's first kAttnCounterBytes (unused, kept for the layout)
  float* part = ws ? reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kAttnCounterBytes) : nullptr;
  hipError_t e = launch(attention_mfma, dim3((unsigned)waves, P), dim3(64), 0, st, q, k, v, pos, out, M, Hq, Hkv, L,
                        scale, part);
  if (e != hipSuccess || P == 1) return e;
  const long threads = (long)M * Hq * kHeadDim;
  return launch(attention_combine, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, part, out, M * Hkv, G, P,
                Hq);
}
}  // namespace

hipError_t attention_launch(const f16* q, const f16* k, const f16* v, const int64_t* pos, f16* out, int M, int Hq,
                            int Hkv, int L, int max_keys, float scale, void* ws, size_t ws_bytes, hipStream_t st) {
  if ((long)M * (Hq / Hkv) >= kAttnMfmaMinRows)
    return launch_attention_mfma(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, ws, ws_bytes, st);
  if ((long)M * Hkv < 64)                                     // few tokens: one query head per block, short steps
    return launch_attention<1, 32>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, ws, ws_bytes, st);
  switch (Hq / Hkv) {
    case 1: return launch_attention<1, 64>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, ws, ws_bytes, st);
    case 2: return launch_attention<2, 64>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, ws, ws_bytes, st);
    case 4: return launch_attention<4, 32>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, ws, ws_bytes, st);
    case 6: return launch_attention<6, 32>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, ws, ws_bytes, st);
    case 7: return launch_attention<7, 32>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, ws, ws_bytes, st);
    case 8: return launch_attention<8, 32>(q, k, v, pos, out, M, Hq, Hkv, L, max_keys, scale, ws, ws_bytes, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t attention_partials_launch(const f16* q, const f16* k, const f16* v, const int64_t* pos, f16* out, int Hq,
                                     int Hkv, int L, int max_keys, float scale, void* ws, size_t ws_bytes, int* parts,
                                     hipStream_t st) {
  // one token: the decode kernel with one query head per block (the MFMA kernel takes 32 or more rows per KV head)
  if (Hq / Hkv >= kAttnMfmaMinRows || Hkv >= 64) return hipErrorInvalidValue;
  return launch_attention<1, 32>(q, k, v, pos, out, 1, Hq, Hkv, L, max_keys, scale, ws, ws_bytes, st, kAttnXMaxParts,
                                 false, parts);
}

}  // namespace lowbit
