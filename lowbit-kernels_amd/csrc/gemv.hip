// M <= 8 GEMV kernels (no MFMA): y[M, N] = x[M, K] . dequant(W)[N, K]^T, fp16 in/out, fp32 accumulation.
//
// gemv_mfma_layout: the deployed decode kernel (the role of the reference's gemv_v6, csrc/w4_gemv.cu:327-391), on the
//   MFMA layout. A 16-row tile x 128-k chunk is one contiguous 1 KB block; lane l reads the 16 bytes at 16 l, i.e.
//   row l / 4, k-quarter l % 4 (32 consecutive k), so every wave-load is one fully coalesced 1 KB. Each lane decodes
//   its 32 nibbles to exact fp16 (u - 8) values, multiplies them with x by v_dot2_f32_f16 into an fp32 partial per
//   chunk, scales the partial by the group's fp16 scale (fp32 FMA), and keeps going. At the end the 4 lanes of a row
//   are summed with two quad DPP adds and the waves of the workgroup, which split K, are summed through LDS.
//   R tiles per wave share each x load. Weights are streamed with non-temporal loads.
// gemv_rowmajor: the canonical / v3 layouts (reference v2 / v4 roles, csrc/w4_gemv.cu:60-94,150-207), needed when
//   G or K is not a multiple of 128 and the MFMA layout cannot be used. One wave per R rows; lane l takes the
//   32-k blocks l, l + 64, ...; wave64 DPP + readlane reduction per row.
#include <algorithm>

#include "kernels.hpp"

namespace lowbit {

namespace {

// x[m][k0 .. k0 + 32) as 16 fp16 pairs (four 16-byte loads)
template <int M>
__device__ __forceinline__ void load_x32(const f16* __restrict__ x, int K, int k0, u32x4 (&xv)[M][4]) {
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int j = 0; j < 4; ++j) xv[m][j] = load16(x + (size_t)m * K + k0 + 8 * j);
}

// 32 weights (one 16-byte piece, four v3 words) against x pairs in the same order -> fp32 partial
__device__ __forceinline__ float dot32(const u32x4& wv, const u32x4 (&xv)[4]) {
  float part = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f16x2 p[4];
    decode_word(wv[j], p);
#pragma unroll
    for (int e = 0; e < 4; ++e) part = dot2(p[e], as_f16x2(xv[j][e]), part);
  }
  return part;
}

}  // namespace

// One memory round trip before the first chunk is decoded. The prologue first requests x (the workgroup stages all
// of x[M][K] into LDS) and the workgroup's fp16 scales, then the weight pieces of each wave's first D chunks. Load
// counters retire in order, so staging x waits only for the x and scale loads while the weights are still in flight;
// one barrier later every wave decodes as its weights arrive. Later chunks stream through the same D slots, each
// refilled as soon as it is consumed. Weight loads use one buffer resource per tile: chunks past K and rows past N
// read as zero without a branch, so the compiler waits on exactly the slot it needs. When M K is too large for LDS
// (kLdsX = false) each lane loads its x pairs from global memory and decodes exactly.
// CS > 1 (R = 1) splits each 16-row tile over CS workgroups of 16 / CS rows, so layers with few tiles still occupy
// every CU: a wave-load then covers CS consecutive chunks of the workgroup's rows (lane l: chunk l / (64 / CS)), each
// piece a contiguous 64 * 16 / CS bytes, and the CS partial sums of a row are added across lanes before the waves'.
//
// LR > 0 (M = 1, R = 1, x in LDS): the weight ring lives in LDS instead of registers. Each wave owns LR slots of 1 KB
// and fills them with direct-to-LDS wave-loads (the same 1 KB pieces); at each step it waits for its oldest slot,
// reads its 16 bytes back, refills the slot LR wave-loads ahead at once and only then decodes. So LR - 1 wave-loads
// stay in flight through the decode at no register cost, where a register ring can refill a slot only after its
// registers are decoded. x, the scales and the norm weights also arrive by direct-to-LDS loads, so the compiler issues
// no vector-memory load before the main loop and every wait on the ring is counted by hand (see dma16).
//
// kAttnX (M = 1, register ring, x in LDS, fused): x is an attention step's output, merged here from the records of its
// key partitions (attention_partials_launch) instead of read: thread t < K / 4 loads the records of head t / 32,
// merges dims 4 t .. 4 t + 3 with the arithmetic of the attention's own merge (merge_partitions: the same bits) and
// writes them to LDS; one barrier later the zero-weight sums are taken from LDS. This replaces the attention's merge
// launch and its output round trip (one launch fewer per decoded token and layer).
// kF16 (M = 1, R = 1, register ring, x in LDS): the same kernel over an fp16 weight [N, K] in row-major order, the
// comparator the W4A16 decode is measured against (same tiles, waves, tile splits, prologue, reduction and epilogues;
// only the weight bytes differ). A wave-load is then 16 rows x 32 k (64 contiguous bytes per row): lane (r, q) takes
// k = 32 p + 8 q .. + 7 of row r for sub-load p, 4 dot2 against x; no scales, no zero sums.
template <int M, int R, int D, bool kLdsX, bool kFused = false, int CS = 1, int LR = 0, bool kF16 = false,
          bool kAttnX = false>
__global__ __launch_bounds__(gemv_max_threads(M, R, D)) void gemv_mfma_layout(const f16* __restrict__ x,
                                                                           const uint8_t* __restrict__ w,
                                                                           const f16* __restrict__ s,
                                                                           f16* y, int N, int K, int G,
                                                                           Epilogue epi,
                                                                           const f16* __restrict__ norm_w, float eps) {
  static_assert(CS == 1 || (R == 1 && (CS == 2 || CS == 4)), "a tile splits over 2 or 4 workgroups, one tile each");
  static_assert(LR == 0 || (M == 1 && R == 1 && kLdsX), "the LDS ring serves the one-row, one-tile GEMV");
  static_assert(!kF16 || (M == 1 && R == 1 && LR == 0 && kLdsX), "the fp16-weight mode serves the one-row GEMV");
  static_assert(!kAttnX || (M == 1 && R == 1 && LR == 0 && kLdsX && kFused), "x from attention partials: one row");
  constexpr int RS = 16 / CS;                               // rows of a tile one workgroup owns
  constexpr int XB = M == 1 ? 2 : 1;                        // x blocks (32 k) staged per thread before the ring
  constexpr int kScaleLoads = 4;                            // scales per thread requested before the ring
  // norm_w (M = 1 with x in LDS only; the launcher then gives every block of x a thread): the projection's input is
  // RMSNorm(x) * norm_w, computed here exactly as lowbit_rmsnorm does (fp32 statistics, fp16 roundings)
  const bool norm = !kAttnX && kFused && kLdsX && M == 1 && norm_w != nullptr;   // kFused: epilogue / norm compiled in
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  args_in_sgprs(x, w, s, N, K, G, (int)blockDim.x);
  if constexpr (kFused) args_in_sgprs(epi.aux, norm_w);    // the epilogue's and the norm's argument lines too
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int q = lane & 3, rl = (lane >> 2) & (RS - 1), cs = lane / (4 * RS);   // cs: chunk within a wave-load
  const int sub = CS == 1 ? 0 : (int)blockIdx.x % CS;      // which 16 / CS rows of the tile
  const int r = RS * sub + rl;                              // this lane's row within its 16-row tile
  // KC: wave-loads per 16-row tile (int4: 128-k chunks; fp16: 32-k pieces)
  const int ntiles = (N + 15) >> 4, KC = kF16 ? K >> 5 : K >> 7, KG = K / G, cpg = G >> 7;
  const size_t tile_bytes = kF16 ? (size_t)32 * K : (size_t)8 * K;   // 16 rows x K/2 bytes (fp16: 16 rows x 2K)
  const int t0 = (CS == 1 ? (int)blockIdx.x : (int)blockIdx.x / CS) * R;
  // rows of this workgroup (none for the second half or quarters of a tile cut short by N: such a workgroup reads
  // only zeros and stores nothing). The clamp is computed per lane (v_med3); readfirstlane keeps the scale buffer
  // resource built from it in scalar registers, where a per-lane value would make every scale load a waterfall loop.
  const int n0 = 16 * t0 + RS * sub, nrows = __builtin_amdgcn_readfirstlane(max(0, min(RS * R, N - n0)));
  // LDS: x [M][K] fp16, its zero-weight sums [M][K/32][2] fp32, the scales [nrows][K/G] fp16 (LR > 0: the layout of
  // gemv_ring_lds, then the ring)
  const GemvRingLds RL = gemv_ring_lds(K, KG, RS, nwaves, LR, norm);
  f16* lds_x = reinterpret_cast<f16*>(smem);
  float* lds_xs = reinterpret_cast<float*>(smem + (LR ? RL.xs : kLdsX ? (size_t)M * K * 2 : 0));
  f16* lds_s = reinterpret_cast<f16*>(smem + (LR ? RL.s : kLdsX ? (size_t)M * K * 2 + (size_t)M * (K / 32) * 8 : 0));

  // 1. x and scale requests
  const int nb = M * (K / 32), ns = kF16 ? 0 : nrows * KG;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)(M * K * 2));
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(s + (size_t)n0 * KG, (uint32_t)(ns * 2));
  // kAttnX: x piece t (dims 4 t .. 4 t + 3, head t / 32) from its head's records (max, sum, -, -, output[128]); the
  // loads of this thread's first piece go out before everything else, further pieces (K / 4 > threads) in staging.
  // Partitions past attn_parts and pieces past K / 4 read nothing (max -inf: skipped by the merge).
  float apm[kAttnX ? kAttnXMaxParts : 1], aps[kAttnX ? kAttnXMaxParts : 1];
  f32x4 apo[kAttnX ? kAttnXMaxParts : 1];
  const __amdgpu_buffer_rsrc_t ar =
      make_rsrc(epi.attn_part, kAttnX ? (uint32_t)((K >> 7) * epi.attn_parts * kAttnRec * 4) : 0u);
  auto attn_load = [&](int t) {
    const int P = epi.attn_parts, rec0 = (t >> 5) * P * kAttnRec * 4;
    const bool tl = t < (K >> 2);
#pragma unroll
    for (int p = 0; p < kAttnXMaxParts; ++p) {
      const bool live = tl && p < P;
      const int rec = rec0 + p * kAttnRec * 4;
      const float mv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ar, live ? rec : kOutOfRange, 0, 0));
      aps[p] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ar, live ? rec + 4 : kOutOfRange, 0, 0));
      apo[p] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ar, live ? rec + 16 + 16 * (t & 31) : kOutOfRange,
                                                                            0, 0));
      apm[p] = live ? mv : -INFINITY;
    }
  };
  if constexpr (kAttnX) attn_load((int)threadIdx.x);
  u32x4 xst[XB][4], wst[XB][4];
  if (LR == 0 && kLdsX && !kAttnX) {
#pragma unroll
    for (int u = 0; u < XB; ++u) {
      const int b = (int)threadIdx.x + u * (int)blockDim.x;
      if (b < nb) {                                         // only threads that own a block issue its loads
#pragma unroll
        for (int j = 0; j < 4; ++j) xst[u][j] = buffer_load16(xr, 64 * b + 16 * j);
      }
    }
    if (norm) {
      const __amdgpu_buffer_rsrc_t nr = make_rsrc(norm_w, (uint32_t)(K * 2));
#pragma unroll
      for (int u = 0; u < XB; ++u) {
        const int b = (int)threadIdx.x + u * (int)blockDim.x;
        if (b < nb) {
#pragma unroll
          for (int j = 0; j < 4; ++j) wst[u][j] = buffer_load16(nr, 64 * b + 16 * j);
        }
      }
    }
  }
  // up to kScaleLoads scales per thread, all in flight before the weights (loads complete in issue order, so a
  // thread's later ones, loaded while staging, would each wait for the whole ring)
  uint16_t sst[kScaleLoads];
  if constexpr (LR == 0) {
#pragma unroll
    for (int u = 0; u < kScaleLoads; ++u) {
      const int i = (int)threadIdx.x + u * (int)blockDim.x;
      if (i < ns) sst[u] = buffer_load2_nt(sr, 2 * i);
    }
  }

  // 2. the weight ring
  __amdgpu_buffer_rsrc_t wr[R];
  int woff[R], wstep[R], srow[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int t = min(t0 + i, ntiles - 1);
    const int rows = t0 + i < ntiles ? min(16, N - 16 * t) : 0;
    const bool live = r < rows;
    if constexpr (kF16) {                                  // row r's 64 bytes of sub-load p at 64 p
      wr[i] = make_rsrc(w + t * tile_bytes, (uint32_t)(rows * K * 2));
      woff[i] = live ? 2 * K * r + 16 * q + 64 * cs : kOutOfRange;
      wstep[i] = live ? 64 * CS : 0;
    } else {
      wr[i] = make_rsrc(w + t * tile_bytes, (uint32_t)(rows * (K / 2)));
      woff[i] = live ? 64 * r + 16 * q + cs * rows * 64 : kOutOfRange;
      wstep[i] = live ? CS * rows * 64 : 0;                // bytes from one wave-load's chunks to the next
    }
    srow[i] = live ? (16 * i + rl) * KG : 0;               // this lane's row in the staged scales
  }
  u32x4 ring[LR ? 1 : D][R];
  const uint32_t lds0 = lds_addr(smem), ring0 = lds0 + RL.ring + (uint32_t)wave * (uint32_t)(LR << 10);
  if constexpr (LR > 0) {
    // x, the scales and the norm weights in 1 KB wave-loads, round robin over the waves, then this wave's first LR
    // weight wave-loads; x keeps the default policy (every workgroup reads it), the rest is streamed
    // A 16-byte load that runs past its range reads zeros as a whole, so the scales' range is rounded up to 16
    // bytes (the next rows' scales, never read), clipped at the end of the scale tensor, whose size the planner
    // requires to be a multiple of 16 bytes (N K / G % 8 == 0): every scale of the workgroup arrives, and no load
    // leaves the tensor.
    const int nxp = (2 * K + 1023) >> 10, nsp = (2 * ns + 1023) >> 10, ngp = norm ? nxp : 0;
    const __amdgpu_buffer_rsrc_t srd =
        make_rsrc(s + (size_t)n0 * KG, (uint32_t)min((2 * ns + 15) & ~15, max(0, 2 * (N - n0) * KG)));
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(norm_w, norm ? (uint32_t)(K * 2) : 0u);
    for (int p = wave; p < nxp + nsp + ngp; p += nwaves) {
      if (p < nxp) dma16(xr, (p << 10) + 16 * lane, lds0 + (p << 10));
      else if (p < nxp + nsp) dma16_nt(srd, ((p - nxp) << 10) + 16 * lane, lds0 + RL.s + ((p - nxp) << 10));
      else dma16(gr, ((p - nxp - nsp) << 10) + 16 * lane, lds0 + RL.g + ((p - nxp - nsp) << 10));
    }
#pragma unroll
    for (int d = 0; d < LR; ++d) dma16_nt(wr[0], woff[0] + (wave + nwaves * d) * wstep[0], ring0 + (d << 10));
    lds_wait_barrier<LR>();                                 // everything but the ring has landed, in every wave
  } else {
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
      for (int i = 0; i < R; ++i) ring[d][i] = buffer_load16_nt(wr[i], woff[i] + (wave + nwaves * d) * wstep[i]);
  }
  // one row, one tile: the bias or residual element of the output this thread stores at the end, requested with the
  // first weights so that its round trip is not paid after the main loop (n_out: -1 for threads that store nothing)
  f16 aux_out{};
  if constexpr (kFused && M == 1 && R == 1) {
    const int n_out = nwaves == 1 ? (q == 0 && cs == 0 ? 16 * t0 + r : -1)
                                  : ((int)threadIdx.x < RS ? 16 * t0 + RS * sub + (int)threadIdx.x : -1);
    if ((epi.mode == kEpiBias || epi.mode == kEpiResidual) && n_out >= 0 && n_out < N) aux_out = epi.aux[n_out];
  }

  // 3. stage x with the decode's own dot2 sequence run on zero weights (every nibble 8), over the lo positions
  //    (k % 8 in 0,1,4,5) and the hi positions (2,3,6,7) of each 32-k block: a block of real weights minus these is
  //    2^-24 sum((u - 8) x) (lo) and 2^-20 sum((u - 8) x) (hi), and exactly 0 where the weights are zero.
  const f16x2 z8lo = as_f16x2(0x00080008u), z8hi = as_f16x2(0x00800080u);
  auto stage_block = [&](int b, const u32x4 (&v)[4], bool write_x = true) {
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (write_x) reinterpret_cast<u32x4*>(lds_x)[4 * b + j] = v[j];
      if constexpr (kF16) continue;                         // fp16 weights: no offset to remove
      lo = dot2(z8lo, as_f16x2(v[j][0]), lo);
      hi = dot2(z8hi, as_f16x2(v[j][1]), hi);
      lo = dot2(z8lo, as_f16x2(v[j][2]), lo);
      hi = dot2(z8hi, as_f16x2(v[j][3]), hi);
    }
    if constexpr (!kF16) {
      lds_xs[2 * b] = lo;
      lds_xs[2 * b + 1] = hi;
    }
  };
  if (LR > 0 && norm) {                                    // x and the norm weights from LDS into registers
#pragma unroll
    for (int u = 0; u < XB; ++u) {
      const int b = (int)threadIdx.x + u * (int)blockDim.x;
      if (b < nb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          xst[u][j] = reinterpret_cast<const u32x4*>(lds_x)[4 * b + j];
          wst[u][j] = reinterpret_cast<const u32x4*>(smem + RL.g)[4 * b + j];
        }
      }
    }
  }
  if (norm) {                                               // RMSNorm of the (single) row before staging it
    __shared__ float ss_red[16];
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < XB; ++u) {
      const int b = (int)threadIdx.x + u * (int)blockDim.x;
      if (b < nb) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const f16x2 v = as_f16x2(xst[u][j][e]);
            ss = fmaf((float)v[0], (float)v[0], ss);
            ss = fmaf((float)v[1], (float)v[1], ss);
          }
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) ss_red[wave] = ss;
    if constexpr (LR > 0) lds_barrier();                    // (not __syncthreads: it would drain the ring)
    else __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < nwaves; ++i) tot += ss_red[i];
    const float rn = rsqrtf(tot / (float)K + eps);
#pragma unroll
    for (int u = 0; u < XB; ++u) {
      const int b = (int)threadIdx.x + u * (int)blockDim.x;
      if (b < nb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) xst[u][j] = rms_apply8(xst[u][j], wst[u][j], rn);
      }
    }
  }
  if (kAttnX) {                                            // merge x into LDS, then its zero-weight sums from there
    for (int t = (int)threadIdx.x; t < (K >> 2); t += blockDim.x) {
      if (t != (int)threadIdx.x) attn_load(t);
      float gm = -INFINITY;
#pragma unroll
      for (int p = 0; p < kAttnXMaxParts; ++p) gm = fmaxf(gm, apm[p]);
      float num[4] = {0.f, 0.f, 0.f, 0.f}, den = 0.f;
#pragma unroll
      for (int p = 0; p < kAttnXMaxParts; ++p) {
        if (apm[p] == -INFINITY) continue;                  // a partition that saw no key
        const float f = expf(apm[p] - gm);
#pragma unroll
        for (int e = 0; e < 4; ++e) num[e] = fmaf(f, apo[p][e], num[e]);
        den = fmaf(f, aps[p], den);
      }
      const f16x2 lo = {(f16)(num[0] / den), (f16)(num[1] / den)}, hi = {(f16)(num[2] / den), (f16)(num[3] / den)};
      *reinterpret_cast<uint2*>(lds_x + 4 * t) = make_uint2(as_u32(lo), as_u32(hi));
    }
    __syncthreads();
    if constexpr (!kF16) {
      for (int b = (int)threadIdx.x; b < nb; b += blockDim.x) {
        u32x4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = reinterpret_cast<const u32x4*>(lds_x)[4 * b + j];
        stage_block(b, v, false);
      }
    }
  } else if (LR > 0) {                                     // x is in LDS (normalized in registers when norm)
    if (norm) {
#pragma unroll
      for (int u = 0; u < XB; ++u) {
        const int b = (int)threadIdx.x + u * (int)blockDim.x;
        if (b < nb) stage_block(b, xst[u]);
      }
    } else {
      for (int b = (int)threadIdx.x; b < nb; b += blockDim.x) {
        u32x4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = reinterpret_cast<const u32x4*>(lds_x)[4 * b + j];
        stage_block(b, v, false);
      }
    }
    lds_barrier();
  } else if (kLdsX) {
#pragma unroll
    for (int u = 0; u < XB; ++u) {
      const int b = (int)threadIdx.x + u * (int)blockDim.x;
      if (b < nb) stage_block(b, xst[u]);
    }
    for (int b = (int)threadIdx.x + XB * (int)blockDim.x; b < nb; b += blockDim.x) {   // long x only
      u32x4 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = buffer_load16(xr, 64 * b + 16 * j);
      stage_block(b, v);
    }
  }
  if constexpr (LR == 0) {
#pragma unroll
    for (int u = 0; u < kScaleLoads; ++u) {
      const int i = (int)threadIdx.x + u * (int)blockDim.x;
      if (i < ns) reinterpret_cast<uint16_t*>(lds_s)[i] = sst[u];
    }
    for (int i = (int)threadIdx.x + kScaleLoads * (int)blockDim.x; i < ns; i += blockDim.x)   // > 4 per thread only
      reinterpret_cast<uint16_t*>(lds_s)[i] = buffer_load2_nt(sr, 2 * i);
    __syncthreads();
  }

  float acc[R][M];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[i][m] = 0.f;

  // this wave's wave-loads are c_j = wave + j * nwaves, j < nj (wave-load c holds chunks CS c .. CS c + CS - 1). Groups
  // of D followed by another refill their slot D wave-loads ahead (a refill past the end reads zeros and is never
  // consumed); the last group, up to D wave-loads, drains the ring without refills.
  const int nj = (KC / CS - wave + nwaves - 1) / nwaves;
  const uint32_t gmagic = cpg == 1 ? 0u : (uint32_t)(0xFFFFFFFFu / (uint32_t)cpg) + 1u;   // c / cpg == mulhi(c, gmagic)
  auto consume = [&](const u32x4 (&slot)[R], int cw) {
    if constexpr (kF16) {                                   // sub-load p: k = 32 p + 8 q .. + 7 of the lane's row
      const int p = CS * cw + cs;
      const u32x4 xv = reinterpret_cast<const u32x4*>(lds_x + 32 * p + 8 * q)[0];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[0][0] = dot2(as_f16x2(slot[0][e]), as_f16x2(xv[e]), acc[0][0]);
      return;
    }
    const int c = CS * cw + cs;                             // this lane's chunk
    const int g = cpg == 1 ? c : (int)__umulhi((uint32_t)c, gmagic);
    u32x4 xv[M][4];
    if (kLdsX) {
      float xs[M][2];
#pragma unroll
      for (int m = 0; m < M; ++m) {
#pragma unroll
        for (int j = 0; j < 4; ++j) xv[m][j] = reinterpret_cast<const u32x4*>(lds_x + (size_t)m * K + 128 * c + 32 * q)[j];
        const int blk = m * (K / 32) + 4 * c + q;
        xs[m][0] = lds_xs[2 * blk];
        xs[m][1] = lds_xs[2 * blk + 1];
      }
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const float scale = (float)lds_s[srow[i] + g];
        float lo[M], hi[M];
#pragma unroll
        for (int m = 0; m < M; ++m) lo[m] = hi[m] = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          f16x2 pl[2], ph[2];
          decode_word_subnormal(slot[i][j], pl, ph);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            lo[m] = dot2(pl[0], as_f16x2(xv[m][j][0]), lo[m]);
            hi[m] = dot2(ph[0], as_f16x2(xv[m][j][1]), hi[m]);
            lo[m] = dot2(pl[1], as_f16x2(xv[m][j][2]), lo[m]);
            hi[m] = dot2(ph[1], as_f16x2(xv[m][j][3]), hi[m]);
          }
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
          // sum((u - 8) x) over the lane's 32 k (exactly 0 for zero weights), then the group scale
          const float part = fmaf(lo[m] - xs[m][0], 16777216.0f, (hi[m] - xs[m][1]) * 1048576.0f);
          acc[i][m] = fmaf(part, scale, acc[i][m]);
        }
      }
    } else {
      load_x32<M>(x, K, 128 * c + 32 * q, xv);
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const float scale = (float)lds_s[srow[i] + g];
#pragma unroll
        for (int m = 0; m < M; ++m) acc[i][m] = fmaf(dot32(slot[i], xv[m]), scale, acc[i][m]);
      }
    }
  };
  if constexpr (LR > 0) {
    // wave-load j sits in slot j % LR; the LR - 1 after it are in flight. Refills past the last wave-load read zeros
    // (out of the buffer's range: no memory access) and are drained before the LDS is reused.
    uint32_t slot = ring0;
    const uint32_t ring_end = ring0 + (uint32_t)(LR << 10);
    for (int j = 0; j < nj; ++j) {
      const u32x4 piece[1] = {lds_wait_read16<LR - 1>(slot + 16 * lane)};
      const int c = wave + j * nwaves;
      dma16_nt(wr[0], woff[0] + (c + LR * nwaves) * wstep[0], slot);
      slot = slot + 1024u == ring_end ? ring0 : slot + 1024u;
      consume(piece, c);
    }
    vm_drain();
  } else {
    int j0 = 0;
    for (; j0 + D < nj; j0 += D) {                          // a later group follows: refill behind each consume
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int c = wave + (j0 + d) * nwaves;
        consume(ring[d], c);
#pragma unroll
        for (int i = 0; i < R; ++i) ring[d][i] = buffer_load16_nt(wr[i], woff[i] + (c + D * nwaves) * wstep[i]);
      }
    }
#pragma unroll
    for (int d = 0; d < D; ++d)                              // the last group, up to D wave-loads, without refills
      if (j0 + d < nj) consume(ring[d], wave + (j0 + d) * nwaves);
  }

  // RoPE epilogue (M = 1): rows n (dim d of a head) and n + 8 (dim d + 64) -> bias, RoPE, q_out or the caches. The
  // position, the pair's two bias values and inv_freq[d] are requested together by rope_load (before the cross-wave
  // reduction where there is one), so their round trip overlaps the reduction and is paid once, not twice (the
  // position, then what the position check guarded)
  struct RopeIn {
    int64_t p;
    f16 b1, b2;
    float invf;
  };
  auto rope_load = [&](int n) -> RopeIn {
    const int pj = n & 127, d = 8 * (pj >> 4) + (pj & 7);
    return RopeIn{epi.rope.pos[0], epi.aux[n], epi.aux[n + 8], epi.rope.inv_freq[d]};
  };
  auto rope_store = [&](int n, float v1, float v2, const RopeIn& in) {
    const RopeArgs& ra = epi.rope;
    const int64_t p = in.p;
    if (p < 0 || p >= ra.L) return;                         // the host checks positions; never write out of bounds
    const f16 x1 = (f16)v1 + in.b1, x2 = (f16)v2 + in.b2;
    const int hh = n >> 7, pj = n & 127, d = 8 * (pj >> 4) + (pj & 7);
    if (hh >= ra.Hq + ra.Hkv) {
      f16* dst = ra.v_cache + ((size_t)(hh - ra.Hq - ra.Hkv) * ra.L + p) * 128;
      dst[d] = x1;
      dst[d + 64] = x2;
      return;
    }
    f16 o1, o2;
    rope_pair(x1, x2, p, in.invf, o1, o2);
    f16* dst = hh < ra.Hq ? ra.q_out + (size_t)hh * 128 : ra.k_cache + ((size_t)(hh - ra.Hq) * ra.L + p) * 128;
    dst[d] = o1;
    dst[d + 64] = o2;
  };
  if constexpr (CS > 1) {                                   // the CS chunks of a wave-load: lanes 64 / CS apart
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        acc[i][m] += __shfl_xor(acc[i][m], 32, 64);
        if (CS == 4) acc[i][m] += __shfl_xor(acc[i][m], 16, 64);
      }
  }
  // silu-mul and RoPE pair row r with row r + 8 of the tile, which one workgroup holds only when CS = 1
  const bool pairs = kFused && CS == 1 && (epi.mode == kEpiSiluMul || epi.mode == kEpiRopeQKV);
  if (nwaves == 1) {                                        // no split of K: the quad sums are the outputs
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float v = quad_sum(acc[i][m]);
        const int n = 16 * (t0 + i) + r;
        if (pairs) {                                        // row r + 8 sits 32 lanes on
          const float up = shfl_down32(v);
          if (q == 0 && r < 8 && n < N) {
            if (epi.mode == kEpiSiluMul) y[(size_t)m * (N / 2) + 8 * (t0 + i) + r] = silu_mul(v, up);
            else rope_store(n, v, up, rope_load(n));
          }
        } else if (q == 0 && cs == 0 && n < N) {
          if constexpr (kFused && M == 1 && R == 1) y[n] = epi_apply(epi.mode, aux_out, v);
          else y[(size_t)m * N + n] = kFused ? epi_value(epi.mode, epi.aux, v, m, n, N) : (f16)v;
        }
      }
    return;
  }
  // the RoPE inputs of the first pair this thread stores below, requested before the reduction's barriers
  RopeIn rope_first{};
  {
    const int idx = threadIdx.x, i = idx / (M * RS), rr = idx % RS;
    const int n = 16 * (t0 + i) + RS * sub + rr;
    if (pairs && epi.mode == kEpiRopeQKV && idx < R * M * RS && rr < 8 && n < N) rope_first = rope_load(n);
  }
  float* red = reinterpret_cast<float*>(smem);              // x is dead after the barrier below
  __syncthreads();
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float v = quad_sum(acc[i][m]);
      if (q == 0 && cs == 0) red[wave * (R * M * RS) + (i * M + m) * RS + rl] = v;
    }
  __syncthreads();
  for (int idx = threadIdx.x; idx < R * M * RS; idx += blockDim.x) {
    const int i = idx / (M * RS), m = (idx / RS) % M, rr = idx % RS;
    const int n = 16 * (t0 + i) + RS * sub + rr;
    if (pairs) {
      if (rr >= 8 || n >= N) continue;
      float g = 0.f, u = 0.f;
      for (int wv2 = 0; wv2 < nwaves; ++wv2) {
        g += red[wv2 * (R * M * RS) + idx];
        u += red[wv2 * (R * M * RS) + idx + 8];
      }
      if (epi.mode == kEpiSiluMul) y[(size_t)m * (N / 2) + 8 * (t0 + i) + rr] = silu_mul(g, u);
      else rope_store(n, g, u, idx == (int)threadIdx.x ? rope_first : rope_load(n));
      continue;
    }
    float v = 0.f;
    for (int wv2 = 0; wv2 < nwaves; ++wv2) v += red[wv2 * (R * M * RS) + idx];
    if constexpr (kFused && M == 1 && R == 1) {              // idx is threadIdx.x here (blockDim.x >= RS)
      if (n < N) y[n] = epi_apply(epi.mode, aux_out, v);
    } else if (n < N) {
      y[(size_t)m * N + n] = kFused ? epi_value(epi.mode, epi.aux, v, m, n, N) : (f16)v;
    }
  }
}

template <int M, int R, bool kV3>
__global__ __launch_bounds__(256) void gemv_rowmajor(const f16* __restrict__ x, const uint8_t* __restrict__ w,
                                                     const f16* __restrict__ s, f16* __restrict__ y, int N, int K,
                                                     int G) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * (blockDim.x >> 6) + wave) * R;
  if (n0 >= N) return;
  const int KB = K >> 5, KG = K / G;
  float acc[R][M];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[i][m] = 0.f;
  for (int b = lane; b < KB; b += 64) {
    u32x4 wv[R];
    float sc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int n = min(n0 + i, N - 1);           // rows past N re-read row N - 1; their sums are never stored
      wv[i] = load_stream(w + (size_t)n * (K / 2) + 16 * b);
      sc[i] = (float)s[(size_t)n * KG + (32 * b) / G];
    }
    u32x4 xv[M][4];
    load_x32<M>(x, K, 32 * b, xv);
    if (!kV3) {
      // canonical words decode to (k0,k4), (k1,k5), (k2,k6), (k3,k7): pair x the same way
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u32x4 X = xv[m][j];
          xv[m][j] = u32x4{(X[0] & 0xFFFFu) | (X[2] << 16), (X[0] >> 16) | (X[2] & 0xFFFF0000u),
                           (X[1] & 0xFFFFu) | (X[3] << 16), (X[1] >> 16) | (X[3] & 0xFFFF0000u)};
        }
    }
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[i][m] = fmaf(dot32(wv[i], xv[m]), sc[i], acc[i][m]);
  }
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float v = wave_sum(acc[i][m]);
      if (lane == 0 && n0 + i < N) y[(size_t)m * N + n0 + i] = (f16)v;
    }
}

// ---- host-side launchers ----

namespace {

// M = 1, one tile per workgroup, weight ring of LR slots per wave in LDS
template <int CS, int LR>
hipError_t launch_lds_ring(const GemvArgs& a, int waves) {
  const int ntiles = (a.N + 15) / 16;
  dim3 grid(CS == 1 ? ntiles : ntiles * CS), block(64 * waves);
  const bool fused = a.epi.mode != kEpiStore || a.norm_w;
  const size_t bytes = std::max<size_t>(gemv_ring_lds(a.K, a.K / a.G, 16 / CS, waves, LR, a.norm_w).total,
                                        (size_t)waves * 16 * 4);
  if (fused) {
    auto k = gemv_mfma_layout<1, 1, 4, true, true, CS, LR>;
    if (bytes > 65536)
      if (hipError_t e = allow_lds(k, bytes)) return e;
    return launch(k, grid, block, bytes, a.stream, a.x, a.w, a.s, a.y, a.N, a.K, a.G, a.epi, a.norm_w, a.eps);
  }
  auto k = gemv_mfma_layout<1, 1, 4, true, false, CS, LR>;
  if (bytes > 65536)
    if (hipError_t e = allow_lds(k, bytes)) return e;
  return launch(k, grid, block, bytes, a.stream, a.x, a.w, a.s, a.y, a.N, a.K, a.G, a.epi, a.norm_w, a.eps);
}

template <int CS>
hipError_t dispatch_lds_ring(const GemvArgs& a, int waves, int LR) {
  switch (LR) {
    case 4: return launch_lds_ring<CS, 4>(a, waves);
    case 8: return launch_lds_ring<CS, 8>(a, waves);
    case 12: return launch_lds_ring<CS, 12>(a, waves);
    default: return launch_lds_ring<CS, 16>(a, waves);
  }
}

// M = 1 over an fp16 weight (row-major [N, K]): the kF16 instances, epilogue and norm code compiled in
template <int CS>
hipError_t launch_f16w(const GemvArgs& a, int waves) {
  const int ntiles = (a.N + 15) / 16;
  dim3 grid(CS == 1 ? ntiles : ntiles * CS), block(64 * waves);
  const size_t bytes = std::max<size_t>((size_t)a.K * 2, (size_t)waves * 16 * 4);
  if (a.epi.attn_part)
    return launch(gemv_mfma_layout<1, 1, 4, true, true, CS, 0, true, true>, grid, block, bytes, a.stream, a.x, a.w, a.s,
                  a.y, a.N, a.K, a.K, a.epi, a.norm_w, a.eps);
  return launch(gemv_mfma_layout<1, 1, 4, true, true, CS, 0, true>, grid, block, bytes, a.stream, a.x, a.w, a.s, a.y,
                a.N, a.K, a.K, a.epi, a.norm_w, a.eps);
}

template <int M, int R, int D, int CS = 1>
hipError_t launch_mfma_layout(const GemvArgs& a, int waves) {
  const int ntiles = (a.N + 15) / 16;
  dim3 grid(CS == 1 ? (ntiles + R - 1) / R : ntiles * CS), block(64 * waves);
  const size_t s_bytes = (size_t)16 * R * (a.K / a.G) * 2;
  const size_t x_bytes = (size_t)M * a.K * 2 + (size_t)M * (a.K / 32) * 8;
  const size_t red_bytes = (size_t)waves * R * M * 16 * 4;
  const bool fused = a.epi.mode != kEpiStore || a.norm_w;
  if constexpr (M == 1) {                                    // only the M = 1 path carries epilogues and the norm
    if constexpr (R == 1 && D == 4) {
      if (a.epi.attn_part) {                                  // x merged from attention partials (kAttnX)
        if (x_bytes + s_bytes > kGemvLdsX) return hipErrorInvalidValue;
        return launch(gemv_mfma_layout<1, 1, 4, true, true, CS, 0, false, true>, grid, block,
                      std::max(x_bytes + s_bytes, red_bytes), a.stream, a.x, a.w, a.s, a.y, a.N, a.K, a.G, a.epi,
                      a.norm_w, a.eps);
      }
    }
    if (fused) {
      if (x_bytes + s_bytes <= kGemvLdsX)
        return launch(gemv_mfma_layout<M, R, D, true, true, CS>, grid, block, std::max(x_bytes + s_bytes, red_bytes),
                      a.stream, a.x, a.w, a.s, a.y, a.N, a.K, a.G, a.epi, a.norm_w, a.eps);
      if (a.norm_w) return hipErrorInvalidValue;             // the fused norm needs x in LDS (the C ABI checks K)
      return launch(gemv_mfma_layout<M, R, D, false, true, CS>, grid, block, std::max(s_bytes, red_bytes), a.stream,
                    a.x, a.w, a.s, a.y, a.N, a.K, a.G, a.epi, a.norm_w, a.eps);
    }
  } else {
    if (fused) return hipErrorInvalidValue;                   // callers send M >= 2 with an epilogue to the MFMA GEMM
  }
  if (x_bytes + s_bytes <= kGemvLdsX)
    return launch(gemv_mfma_layout<M, R, D, true, false, CS>, grid, block, std::max(x_bytes + s_bytes, red_bytes),
                  a.stream, a.x, a.w, a.s, a.y, a.N, a.K, a.G, a.epi, a.norm_w, a.eps);
  return launch(gemv_mfma_layout<M, R, D, false, false, CS>, grid, block, std::max(s_bytes, red_bytes), a.stream,
                a.x, a.w, a.s, a.y, a.N, a.K, a.G, a.epi, a.norm_w, a.eps);
}

template <int M>
hipError_t dispatch_mfma_layout(const GemvArgs& a, int R, int waves, int D, int CS) {
  if (CS == 2) return launch_mfma_layout<M, 1, 4, 2>(a, waves);   // the planner pairs CS > 1 with R = 1, D = 4
  if (CS == 4) return launch_mfma_layout<M, 1, 4, 4>(a, waves);
  if constexpr (M <= 2) {
    if (D > 4) {
      switch (R) {
        case 1: return launch_mfma_layout<M, 1, 8>(a, waves);
        case 2: return launch_mfma_layout<M, 2, 8>(a, waves);
        default: break;
      }
    }
  }
  switch (R) {
    case 1: return launch_mfma_layout<M, 1, 4>(a, waves);
    case 2: return launch_mfma_layout<M, 2, 4>(a, waves);
    default: return launch_mfma_layout<M, 4, 4>(a, waves);
  }
}

template <int M, int R>
hipError_t launch_rowmajor(const GemvArgs& a, bool v3) {
  const int rows = 4 * R;
  dim3 grid((a.N + rows - 1) / rows), block(256);
  if (v3) return launch(gemv_rowmajor<M, R, true>, grid, block, 0, a.stream, a.x, a.w, a.s, a.y, a.N, a.K, a.G);
  return launch(gemv_rowmajor<M, R, false>, grid, block, 0, a.stream, a.x, a.w, a.s, a.y, a.N, a.K, a.G);
}

template <int M>
hipError_t dispatch_rowmajor(const GemvArgs& a, int R, bool v3) {
  switch (R) {
    case 1: return launch_rowmajor<M, 1>(a, v3);
    case 2: return launch_rowmajor<M, 2>(a, v3);
    default: return launch_rowmajor<M, 4>(a, v3);
  }
}

}  // namespace

GemvPlan plan_gemv_mfma_layout(int M, int N, int K, int rows_per_wave, bool row_split_ok, bool lds_ring_ok) {
  GemvPlan p;
  const int ntiles = (N + 15) / 16, KC = K / 128;
  const GemvOverride o = gemv_override();
  // From the MI355X graph-mode sweep over the Qwen2.5-1.5B/3B and 7B-shaped projections (M = 1): one 16-row tile
  // per wave always. A layer with at most 128 tiles and K >= 2048 splits each tile over the most workgroups (2 or 4)
  // that still fit one round of the 256 CUs: the decode ALU work of its busiest CU then halves or quarters (8960 x
  // 1536: 5.5 -> 4.3 us, 11008 x 2048: 6.1 -> 4.9 us); a split that leaves a CU two workgroups, or a short K, gains
  // nothing. 8 waves splitting K on narrow and split layers (16 on long rows), fewer as the tile count grows (below);
  // never more waves than wave-loads; 4 wave-loads in flight per wave.
  p.R = rows_per_wave ? rows_per_wave : 1;
  auto split_fits = [&](int cs) { return p.R == 1 && row_split_ok && KC % cs == 0; };
  if (o.splits == 1 || ((o.splits == 2 || o.splits == 4) && split_fits(o.splits))) {
    p.CS = o.splits;
  } else if (KC >= 16) {
    for (int cs = 4; cs >= 2 && p.CS == 1; cs /= 2)
      if (split_fits(cs) && ntiles * cs <= 256) p.CS = cs;
  }
  const int blocks = p.CS == 1 ? (ntiles + p.R - 1) / p.R : ntiles * p.CS;
  int waves;
  if (p.CS == 1 && blocks >= 256) {
    // about 1.5k waves in flight, at most 16 wave-loads each (2048 x 22016: 1 wave, 6.4 vs 7.0 us at 2; 2048 x 11008:
    // 2, 4.6 vs 4.8 at 4; 3584 x 4608: 4, 4.2 vs 4.5 at 8; 3584 x 18944 keeps 2: 28 wave-loads on 1 wave take 10.3 us)
    waves = 1;
    while (waves < 8 && blocks * waves * 2 <= 1536) waves *= 2;
    while (waves < 8 && KC / waves > 16) waves *= 2;
  } else {
    waves = KC / p.CS >= 128 ? 16 : 8;
  }
  while (waves > 1 && waves > KC / p.CS) waves /= 2;
  if (o.waves > 0) waves = o.waves;
  p.D = ((o.ring == 4 || o.ring == 8) && M <= 2) ? o.ring : 4;
  p.waves = std::min(waves, gemv_max_threads(M, p.R, p.D) / 64);
  // the weight ring in LDS: M = 1, one tile per wave, when the workgroup's LDS fits a CU and the scale tensor is a
  // whole number of 16-byte pieces (its last piece is loaded whole). Automatic on long rows (at least 128 wave-loads
  // per workgroup): 4 slots and 8 waves (MI355X graph sweep, cold weights: 18944 x 3584 8.10 us against 8.52 for
  // the best register-ring shape, 16 waves; on every shorter-K decode shape the register ring is level or faster,
  // e.g. 11008 x 2048 4.47 against 5.09, 2048 x 11008 4.66 against 5.00)
  const bool auto_lds = lds_ring_ok && o.lds_ring == 0 && o.waves == 0 && p.CS == 1 && KC / p.CS >= 128;
  if (M == 1 && p.R == 1 && lds_ring_ok && (o.lds_ring > 0 || auto_lds) && (int64_t)N * (K / 128) % 8 == 0) {
    const int waves = auto_lds ? 8 : p.waves;
    const bool norm = K <= 16384;                           // room for the fused norm's weights where it may run
    int lr = o.lds_ring > 0 ? o.lds_ring : 4;
    while (lr > 4 && gemv_ring_lds(K, K / 128, 16 / p.CS, waves, lr, norm).total > kLdsPerCu) lr -= 4;
    if (gemv_ring_lds(K, K / 128, 16 / p.CS, waves, lr, norm).total <= kLdsPerCu) {
      p.LR = lr;
      p.waves = waves;
    }
  }
  return p;
}

int pick_rows_rowmajor(int N, int M) { return N >= 512 ? 4 : (M >= 4 ? 2 : 1); }

hipError_t gemv_mfma_layout_launch(const GemvArgs& a, int rows_per_wave) {
  // a tile may split over workgroups unless the epilogue pairs rows r and r + 8 of a tile
  const bool row_split_ok = a.epi.mode != kEpiSiluMul && a.epi.mode != kEpiRopeQKV;
  GemvPlan p = plan_gemv_mfma_layout(a.M, a.N, a.K, rows_per_wave, row_split_ok);
  if (a.norm_w) {                                             // every 32-k block of x held by a thread (2 per thread)
    const int need = (a.K / 32 + 127) / 128;
    while (p.waves < need) p.waves *= 2;
  }
  if (a.epi.attn_part) {                                      // the plan of x as given, on the register ring
    if (a.M != 1 || p.R != 1) return hipErrorInvalidValue;
    return dispatch_mfma_layout<1>(a, 1, p.waves, 4, p.CS);
  }
  if (p.LR > 0 && a.M == 1 && (int64_t)a.N * (a.K / a.G) % 8 == 0 &&
      gemv_ring_lds(a.K, a.K / a.G, 16 / p.CS, p.waves, p.LR, a.norm_w).total <= kLdsPerCu) {
    if (p.CS == 2) return dispatch_lds_ring<2>(a, p.waves, p.LR);
    if (p.CS == 4) return dispatch_lds_ring<4>(a, p.waves, p.LR);
    return dispatch_lds_ring<1>(a, p.waves, p.LR);
  }
  switch (a.M) {
    case 1: return dispatch_mfma_layout<1>(a, p.R, p.waves, p.D, p.CS);
    case 2: return dispatch_mfma_layout<2>(a, p.R, p.waves, p.D, p.CS);
    case 3: return dispatch_mfma_layout<3>(a, p.R, p.waves, p.D, p.CS);
    case 4: return dispatch_mfma_layout<4>(a, p.R, p.waves, p.D, p.CS);
    case 5: return dispatch_mfma_layout<5>(a, p.R, p.waves, p.D, p.CS);
    case 6: return dispatch_mfma_layout<6>(a, p.R, p.waves, p.D, p.CS);
    case 7: return dispatch_mfma_layout<7>(a, p.R, p.waves, p.D, p.CS);
    default: return dispatch_mfma_layout<8>(a, p.R, p.waves, p.D, p.CS);
  }
}

hipError_t gemv_f16w_launch(const GemvArgs& a) {
  // the int4 GEMV's plan with K counted in 32-k wave-loads (4 per 128-k chunk): the same waves and tile splits per
  // wave-load
  const bool row_split_ok = a.epi.mode != kEpiSiluMul && a.epi.mode != kEpiRopeQKV;
  GemvPlan p = plan_gemv_mfma_layout(1, a.N, 4 * a.K, 1, row_split_ok, false);
  if (a.norm_w) {
    const int need = (a.K / 32 + 127) / 128;
    while (p.waves < need) p.waves *= 2;
  }
  if (p.CS == 2) return launch_f16w<2>(a, p.waves);
  if (p.CS == 4) return launch_f16w<4>(a, p.waves);
  return launch_f16w<1>(a, p.waves);
}

hipError_t gemv_rowmajor_launch(const GemvArgs& a, int rows_per_wave, bool v3) {
  const int R = rows_per_wave ? rows_per_wave : pick_rows_rowmajor(a.N, a.M);
  switch (a.M) {
    case 1: return dispatch_rowmajor<1>(a, R, v3);
    case 2: return dispatch_rowmajor<2>(a, R, v3);
    case 3: return dispatch_rowmajor<3>(a, R, v3);
    case 4: return dispatch_rowmajor<4>(a, R, v3);
    case 5: return dispatch_rowmajor<5>(a, R, v3);
    case 6: return dispatch_rowmajor<6>(a, R, v3);
    case 7: return dispatch_rowmajor<7>(a, R, v3);
    default: return dispatch_rowmajor<8>(a, R, v3);
  }
}

}  // namespace lowbit
