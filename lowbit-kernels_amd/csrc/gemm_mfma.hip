// Skinny GEMM on the MFMA layout, 1 <= M <= 64: y[M, N] = x[M, K] . dequant(W)^T with v_mfma_f32_16x16x32_f16.
// The role of the reference's tensor-core gemm_v5 (csrc/w4_gemv.cu:215-294), designed for CDNA4 wave64 MFMA.
//
// Operands of one 16x16x32 MFMA (lane l, r = l % 16, q = l / 16):
//   A (16 weight rows x 32 k): row r, 8 consecutive k of quarter q. In the MFMA layout lane l's 16-byte piece of a
//     1 KB block is exactly row r, k = 128 c + 32 q + [0, 32): word j of it feeds k-step j, so one coalesced 1 KB
//     wave-load gives the A fragments of four MFMAs with no shuffle.
//   B (32 k x 16 activation rows): x[16 mt + r][128 c + 32 q + 8 j + 0..7], 16 bytes read from LDS.
//   D: lane l holds rows n = 16 t + 4 q + v (v = 0..3) of column m = 16 mt + r.
//
// Decode: each v3 word becomes the eight A values (pairs (k0,k1), (k2,k3), (k4,k5), (k6,k7)) u - 8, exact in fp16
// (magic number, nine instructions per word with the constants in registers), so every product (u - 8) x is exact in
// fp32 whatever the magnitude of x and zero weights give exactly 0. The four MFMAs of a 128-k chunk sum those products
// in fp32; the chunk's sum is multiplied by its rows' fp32 group scales into the running sums (one FMA per output).
// (An earlier decode put each nibble alone in an fp16 subnormal u 2^-24 and removed the offset 8 with a second set
// of MFMAs on the constant "all nibbles 8": twice the MFMAs, and the per-chunk difference of two large sums
// amplified fp32 rounding about 16-fold.)
//
// Workgroup: 4 x KS waves. Wave w owns RW 16-row tiles (tile-wave w % 4) in K-group w / 4; the K-groups split the
// workgroup's 128-k chunks round-robin. The 4 waves of a K-group walk the same chunks, so each chunk of x is loaded
// from memory once per K-group (coalesced, 16 bytes per thread and row piece) and shared through LDS (double buffered,
// one barrier per step). Each wave keeps D chunks in flight: per slot its tiles' weight pieces and scales and the
// thread's x pieces, issued together because load counters retire in order. Buffer loads make tails free: rows past
// N and chunks past the workgroup's range read zeros (and add nothing), activation rows past M read zeros. At the end
// the K-groups are summed through LDS.
//
// Narrow N cannot fill 256 CUs with row groups alone, so K is also split over S workgroups per row group (grid.y)
// when the caller passes a workspace. Each writes its fp32 partial sums as agent-coherent stores (store_partial), waits
// for them, and one thread per workgroup counts the arrival; the last to arrive reads the S partials the same way,
// adds them in split order, writes y and resets the counter to 0. Results do not depend on timing.
#include <algorithm>
#include <climits>

#include "kernels.hpp"

namespace lowbit {

namespace {

constexpr int kW = 4;              // tile-waves per K-group of the default shape
constexpr int kXPitch = 256;       // bytes per staged activation row (one 128-k chunk of fp16)
// 16-byte block b of staged x row m sits at block b ^ xswz(m % 16) of the row. A lane (r = m % 16, q) reading k-step j
// of a B fragment takes block b = 4 q + j, which lands at 4 (q ^ (r & 3)) + (j ^ (r >> 2)): each wave-wide fragment
// read covers all 16 block positions of 16 rows. An MI355X probe of those reads (16 ds_read_b128 per wave with
// immediate offsets, 10 and 16 waves per CU): 168 / 209 B/clk per CU, against 105 / 113 for rows padded to 272 bytes
// (the layout before), 108 / 117 for b ^ r and 116 / 123 for 288-byte rows; the staging stores run at 73 B/clk in all
// of these layouts. In the kernel: 7B gate/up at M = 64 22.8 -> 21.0 us, 7B down 32.3 -> 31.5, 3B merged gate|up
// 15.4 -> 14.8 (a few shapes at 48 rows lose up to 3%: 2048 x 11008 9.5 -> 9.85).
constexpr int xswz(int r) { return ((r & 3) << 2) | (r >> 2); }
constexpr int kTilesNormMaxMT = 3;           // gemm_mfma_tiles normalizes its input up to 48 rows
constexpr size_t kGemmMaxLds = 144 * 1024;   // dynamic LDS of a row-group workgroup: 128 KB of x buffers + 16 KB of norm weights
}  // namespace

template <int MT, int RW, int D, int KS, int TW, bool ROPE>
__global__ __launch_bounds__(64 * TW * KS) void gemm_mfma(const f16* __restrict__ x, const uint8_t* __restrict__ w,
                                                      const f16* __restrict__ s, f16* y, int M, int N, int K, int G,
                                                      int S, uint32_t* __restrict__ ctr, float* __restrict__ part,
                                                      Epilogue epi) {
  constexpr int T = TW * RW;                               // 16-row tiles per workgroup
  constexpr int kXBuf = 16 * MT * kXPitch;                 // one staged chunk of x
  // a chunk of x is 16 MT rows x 16 pieces of 16 bytes, staged by the 64 TW threads of a K-group, kPer pieces each
  constexpr int kPieces = 16 * 16 * MT, kGroupThreads = 64 * TW;
  constexpr int kPer = (kPieces + kGroupThreads - 1) / kGroupThreads;
  constexpr bool kWhole = kPieces % kGroupThreads == 0;    // else the last round of pieces is partial
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_last;
  args_in_sgprs(x, w, s, y, M, N, K, G, S, ctr, part, epi.aux, (int)gridDim.y);   // (the grid's line: the order)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = wave / TW, tw = wave - kg * TW;            // K-group, tile-wave
  const int gt = tid - kGroupThreads * kg;                  // thread index inside the K-group
  const int r = lane & 15, q = lane >> 4;
  const int ntiles = (N + 15) >> 4, KC = K >> 7, KG = K / G, cpg = G >> 7;
  // a two-dimensional grid numbers row groups fastest (the S splits of a row group on one XCD when the row groups
  // number a multiple of 8); a one-dimensional one numbers the splits fastest (workgroup i on XCD i % 8, so the
  // workgroups of a split, which read the same slice of x, share an XCD and its L2)
  const bool flat = gridDim.y == 1;
  const int grp = flat ? (int)blockIdx.x / S : (int)blockIdx.x, split = flat ? (int)blockIdx.x % S : (int)blockIdx.y;
  const int n0 = 16 * T * grp;
  const int cb = (int)((int64_t)KC * split / S), ce = (int)((int64_t)KC * (split + 1) / S);
  const int nsteps = (ce - cb + KS - 1) / KS;               // K-group kg takes chunks cb + kg + KS j
  const size_t tile_bytes = (size_t)8 * K;
  uint8_t* xbuf = smem + kg * 2 * kXBuf;                    // this K-group's two x buffers

  // per tile: weight resource and offsets, scale offset of this lane's row 4 q + (r & 3)
  __amdgpu_buffer_rsrc_t wr[RW];
  int woff[RW], wstep[RW], soff[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const int t = T * grp + tw * RW + i;
    const int tc = min(t, ntiles - 1);
    const int rows = t < ntiles ? min(16, N - 16 * t) : 0;
    wr[i] = make_rsrc(w + tc * tile_bytes, (uint32_t)(rows * (K / 2)));
    woff[i] = r < rows ? 64 * r + 16 * q : kOutOfRange;
    wstep[i] = r < rows ? rows * 64 : 0;                    // bytes from one chunk to the next inside the tile
    const int srow = 16 * t + 4 * q + (r & 3);
    soff[i] = srow < N ? 2 * srow * KG : kOutOfRange;
  }
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(s, (uint32_t)N * (uint32_t)KG * 2u);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)M * (uint32_t)K * 2u);
  // the input RMSNorm (epi.norm_w): each x piece is normalized as it is staged, with its row's 1 / RMS (s_rn, over all
  // of K) and the norm weights of its 8 columns (the split's chunks of them staged in LDS after the x buffers, lds_g)
  const bool norm = epi.norm_w != nullptr;
  uint8_t* lds_g = smem + KS * 2 * kXBuf;
  __shared__ float s_rn[64];
  // this thread's x pieces: piece pc = gt + 64 TW u is row pc / 16, bytes 16 (pc % 16) of the chunk; rows >= M read
  // past the end (zeros); in a partial last round, threads past the last piece (xl < 0) load and store nothing
  int xoff[kPer], xl[kPer], goff[kPer], xrow[kPer];       // goff: the piece's byte offset in a chunk of lds_g
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int pc = gt + kGroupThreads * u;
    const bool in = kWhole || pc < kPieces;
    xoff[u] = in ? ((pc >> 4) * K + 8 * (pc & 15)) * 2 : kOutOfRange;
    xl[u] = in ? (pc >> 4) * kXPitch + 16 * ((pc & 15) ^ xswz((pc >> 4) & 15)) : -1;
    goff[u] = 16 * (pc & 15);
    xrow[u] = in ? pc >> 4 : 0;
  }
  auto piece_live = [&](int u) { return kWhole || u + 1 < kPer || xl[u] >= 0; };

  u32x4 rw[D][RW], rx[D][kPer];
  uint32_t rs[D][RW];
  const uint32_t gmagic = cpg == 1 ? 0u : (uint32_t)(0xFFFFFFFFu / (uint32_t)cpg) + 1u;   // c / cpg == mulhi(c, gmagic)
  auto issue = [&](int d, int step) {
    const int c = cb + kg + KS * step;
    const bool live = c < ce;
    const int g = cpg == 1 ? c : (int)__umulhi((uint32_t)c, gmagic);
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      rw[d][i] = buffer_load16_nt(wr[i], live ? woff[i] + c * wstep[i] : kOutOfRange);
      rs[d][i] = buffer_load2(sr, live ? soff[i] + 2 * g : kOutOfRange);
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) rx[d][u] = buffer_load16(xr, live && piece_live(u) ? xoff[u] + 256 * c : kOutOfRange);
  };
  auto stage_x = [&](int d, int b, int step) {              // x pieces of slot d (step) -> LDS buffer b
#pragma unroll
    for (int u = 0; u < kPer; ++u)
      if (piece_live(u))
        *reinterpret_cast<u32x4*>(xbuf + b * kXBuf + xl[u]) =
            norm && kg + KS * step < ce - cb    // a step past the group's chunks stages its zeros as they are
                ? rms_apply8(rx[d][u], *reinterpret_cast<const u32x4*>(lds_g + goff[u] + 256 * (kg + KS * step)),
                             s_rn[xrow[u]])
                : rx[d][u];
  };

#pragma unroll
  for (int d = 0; d < D; ++d) issue(d, d);
  if (norm) {                                               // the rows' statistics while the ring is in flight
    stage_norm_weights(epi.norm_w, cb, ce, lds_g);
    rms_rows(xr, M, K, 16 * MT, epi.norm_eps, wave, TW * KS, lane, s_rn);
    __syncthreads();
  }
  stage_x(0, 0, 0);
  __syncthreads();

  f32x4 acc[RW][MT];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const DecodeRegs dc = decode_regs();
  int xrd[4];                                               // lane (r, q): block 4 q + j of row r, swizzled
#pragma unroll
  for (int j = 0; j < 4; ++j) xrd[j] = r * kXPitch + 16 * ((4 * q + j) ^ xswz(r));

  auto consume = [&](int d, int b) {
    f32x4 pt[RW][MT];
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) pt[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f16x8 bx[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        bx[mt] = *reinterpret_cast<const f16x8*>(xbuf + b * kXBuf + 16 * mt * kXPitch + xrd[j]);
#pragma unroll
      for (int i = 0; i < RW; ++i) {
        const f16x8 a = decode_word_a(rw[d][i][j], dc);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) pt[i][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bx[mt], pt[i][mt], 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      const uint32_t sb = rs[d][i];
      const float sc[4] = {(float)__builtin_bit_cast(f16, (uint16_t)quad_bcast<0>(sb)),
                           (float)__builtin_bit_cast(f16, (uint16_t)quad_bcast<1>(sb)),
                           (float)__builtin_bit_cast(f16, (uint16_t)quad_bcast<2>(sb)),
                           (float)__builtin_bit_cast(f16, (uint16_t)quad_bcast<3>(sb))};
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][mt][v] = fmaf(pt[i][mt][v], sc[v], acc[i][mt][v]);
    }
  };

  // step j uses ring slot j % D and LDS buffer j % 2; full groups of D refill their slot D steps ahead, the last
  // partial group drains the ring. After step j the next step's x goes to the other buffer. Every K-group runs the
  // same number of steps (a step past the group's chunks reads zeros and adds nothing), so the barriers match.
  int j0 = 0;
  for (; j0 + D <= nsteps; j0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int j = j0 + d;
      consume(d, j & 1);
      issue(d, j + D);
      if (j + 1 < nsteps) stage_x((d + 1) % D, (j + 1) & 1, j + 1);
      __syncthreads();
    }
  }
#pragma unroll
  for (int d = 0; d < D - 1; ++d) {
    const int j = j0 + d;
    if (j < nsteps) {
      consume(d, j & 1);
      if (j + 1 < nsteps) stage_x(d + 1, (j + 1) & 1, j + 1);
      __syncthreads();
    }
  }

  // sum the K-groups through LDS (the x buffers are free after the last barrier); K-group 0 keeps the totals
  if (KS > 1) {
    f32x4* red = reinterpret_cast<f32x4*>(smem);            // [KS - 1][4][RW][MT][64]
    if (kg > 0) {
#pragma unroll
      for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) red[((((kg - 1) * TW + tw) * RW + i) * MT + mt) * 64 + lane] = acc[i][mt];
    }
    __syncthreads();
    if (kg == 0) {
#pragma unroll
      for (int g2 = 1; g2 < KS; ++g2)
#pragma unroll
        for (int i = 0; i < RW; ++i)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[i][mt] += red[((((g2 - 1) * TW + tw) * RW + i) * MT + mt) * 64 + lane];
    }
  }

  // epilogue: K-group 0 holds the totals; the lane has rows n .. n + 3 of column m per (tile, column tile). Every
  // wave stays to the end, so each barrier below sees the whole workgroup.
  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0;
  // four outputs n .. n + 3 of column m (store / bias / residual), vectorized when aligned
  auto store4 = [&](int m, int n, const f32x4& v) {
    f16* dst = y + (size_t)m * N + n;
    if (vec) {
      const f16x2 lo = {epi_value(epi.mode, epi.aux, v[0], m, n, N), epi_value(epi.mode, epi.aux, v[1], m, n + 1, N)};
      const f16x2 hi = {epi_value(epi.mode, epi.aux, v[2], m, n + 2, N), epi_value(epi.mode, epi.aux, v[3], m, n + 3, N)};
      *reinterpret_cast<uint2*>(dst) = make_uint2(as_u32(lo), as_u32(hi));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < N) dst[e] = epi_value(epi.mode, epi.aux, v[e], m, n + e, N);
    }
  };
  // store4 with the bias / residual elements already loaded (aux_load4)
  auto store4_pre = [&](int m, int n, const f32x4& v, const Aux4& a) {
    f16* dst = y + (size_t)m * N + n;
    if (vec) {
      const f16x2 lo = {epi_apply(epi.mode, a.v[0], v[0]), epi_apply(epi.mode, a.v[1], v[1])};
      const f16x2 hi = {epi_apply(epi.mode, a.v[2], v[2]), epi_apply(epi.mode, a.v[3], v[3])};
      *reinterpret_cast<uint2*>(dst) = make_uint2(as_u32(lo), as_u32(hi));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < N) dst[e] = epi_apply(epi.mode, a.v[e], v[e]);
    }
  };
  // silu(gate rows n .. n + 3) * (up rows n + 8 .. n + 11) -> output columns 8 (n / 16) + n % 16 .. + 3
  auto store4_silu = [&](int m, int n, const f32x4& g, const f32x4& u) {
    f16* dst = y + (size_t)m * (N / 2) + 8 * (n >> 4) + (n & 15);
    const f16x2 lo = {silu_mul(g[0], u[0]), silu_mul(g[1], u[1])}, hi = {silu_mul(g[2], u[2]), silu_mul(g[3], u[3])};
    *reinterpret_cast<uint2*>(dst) = make_uint2(as_u32(lo), as_u32(hi));
  };
  if (S == 1) {
    if (kg > 0) return;
    if constexpr (ROPE) {                                   // every tile's loads and RoPE first, the stores after
      Out4 out[RW][MT];
#pragma unroll
      for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = 16 * mt + r, n = n0 + 16 * (tw * RW + i) + 4 * q;
          const f32x4 v = acc[i][mt];                       // partner rows 8 + 4 q + v sit 32 lanes on (q + 2)
          const f32x4 up = {shfl_down32(v[0]), shfl_down32(v[1]), shfl_down32(v[2]), shfl_down32(v[3])};
          out[i][mt] = q < 2 && m < M && n < N ? rope_qkv_out4(epi, m, n, v, up) : Out4{};
        }
#pragma unroll
      for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) store_rope4(out[i][mt]);
      return;
    }
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + r, n = n0 + 16 * (tw * RW + i) + 4 * q;
        const f32x4 v = acc[i][mt];
        if (epi.mode == kEpiSiluMul) {                      // up rows 8 + 4 q + v sit 32 lanes on (q + 2)
          const f32x4 up = {shfl_down32(v[0]), shfl_down32(v[1]), shfl_down32(v[2]), shfl_down32(v[3])};
          if (q < 2 && m < M && n < N) store4_silu(m, n, v, up);
          continue;
        }
        if (m >= M || n >= N) continue;
        store4(m, n, v);
      }
    return;
  }
  // [S][M][N] fp32 partials, byte offsets into the workspace (S M N 4 bytes, within the 32-bit range the planner keeps)
  const __amdgpu_buffer_rsrc_t pr = make_rsrc(part, (uint32_t)((size_t)S * M * N * 4));
  auto poff = [&](int k, int m, int n) { return (int)((((size_t)k * M + m) * N + n) * 4); };
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + r, n = n0 + 16 * (tw * RW + i) + 4 * q;
      if (kg > 0 || m >= M || n >= N) continue;
      const f32x4 v = acc[i][mt];
      const int off = poff(split, m, n);
      if (vec) {
        store_partial4(pr, off, v);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < N) store_partial(pr, off + 4 * e, v[e]);
      }
    }
  // every wave waits for its partials' acknowledgements before the barrier, so thread 0 counts the workgroup's
  // arrival only once all of them are visible to every XCD
  __atomic_signal_fence(__ATOMIC_SEQ_CST);                 // the partials' stores stay before the wait
  __builtin_amdgcn_s_waitcnt(0);                            // every partial acknowledged: visible to all XCDs
  __builtin_amdgcn_s_barrier();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(ctr + grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == (uint32_t)(S - 1);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);                 // the partials' loads stay after the count
  if (!s_last) return;
  if (tid == 0) __hip_atomic_store(ctr + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int nrows = min(16 * T, N - n0), nq = (nrows + 3) >> 2;
  auto split_sum = [&](int m, int n) {                      // partials of rows n .. n + 3, added in split order
    return sum_partials4(pr, S, (N & 3) == 0 ? 4 : min(4, N - n), [&](int sp) { return poff(sp, m, n); });
  };
  for (int it = tid; it < M * nq; it += kGroupThreads * KS) {
    const int m = it / nq, n = n0 + 4 * (it - m * nq);
    if constexpr (ROPE) {
      if ((n & 15) < 8) store_rope4(rope_qkv_out4(epi, m, n, split_sum(m, n), split_sum(m, n + 8)));
    } else if (epi.mode == kEpiSiluMul) {
      if ((n & 15) < 8) store4_silu(m, n, split_sum(m, n), split_sum(m, n + 8));
    } else {                                                // bias / residual requested with the partials
      const Aux4 a = aux_load4(epi, m, n, N, vec);
      store4_pre(m, n, split_sum(m, n), a);
    }
  }
}

// gemm_mfma_tiles: the same MFMA arithmetic with one 16-row tile per workgroup, for M <= 64 on attention-sized layers
// (few tiles, short K; the selection rule is tiles_win below). The row-group kernel above stages activations for 64
// rows with a barrier per chunk and, on narrow layers, splits K over workgroups that hand their partials over through
// memory; here the workgroup's waves split the tile's 128-k chunks round-robin and are summed through LDS at
// the end, so no workgroup waits for another. Each wave loads, next to its weight piece, the activation piece its B
// fragments need (lane l: 64 contiguous bytes, x row 16 mt + l % 16, k = 128 c + 32 (l / 16) + [0, 32)) straight into
// registers: no staging buffer and no barrier inside the K loop. Lane l's weight piece is row l % 16, quarter l / 16
// (the A fragments of four MFMAs, one coalesced 1 KB wave-load); its scale is row 4 (l / 16) + l % 4, broadcast
// within the quad to the four D rows the lane holds. Rows past N, chunks past K and activation rows past M read
// zeros through the buffer bounds.
template <int MT, int D, int kThreads, bool ROPE>
__global__ __launch_bounds__(kThreads) void gemm_mfma_tiles(const f16* __restrict__ x, const uint8_t* __restrict__ w,
                                                        const f16* __restrict__ s, f16* y, int M, int N, int K, int G,
                                                        Epilogue epi) {
  args_in_sgprs(x, w, s, y, M, N, K, G, epi.aux, (int)blockDim.x);
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), W = blockDim.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int t = blockIdx.x, n0 = 16 * t;
  const int rows = min(16, N - n0), KC = K >> 7, KG = K / G, cpg = G >> 7;
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(w + (size_t)t * 8 * K, (uint32_t)(rows * (K / 2)));
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(s, (uint32_t)N * (uint32_t)KG * 2u);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)M * (uint32_t)K * 2u);
  // the input RMSNorm (epi.norm_w): each B fragment normalized before its MFMA, with its row's 1 / RMS (over all of K)
  // and the norm weights of its 8 columns (staged in LDS after the reduction scratch, lds_g). Not built for MT = 4,
  // whose registers it would spill (the launcher sends a normalized 49..64-row input to the row-group kernel).
  const bool norm = MT <= kTilesNormMaxMT && epi.norm_w != nullptr;
  uint8_t* lds_g = smem + (size_t)(W - 1) * MT * 64 * 16;
  __shared__ float s_rn[64];
  const bool wlive = r < rows;
  const int woff = wlive ? 64 * r + 16 * q : 0, wstep = rows * 64;
  const int srow = n0 + 4 * q + (r & 3);
  const bool slive = srow < N;
  const int soff = slive ? 2 * srow * KG : 0;
  int xoff[MT];
  bool xlive[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    xlive[mt] = 16 * mt + r < M;
    xoff[mt] = xlive[mt] ? ((16 * mt + r) * K + 32 * q) * 2 : 0;
  }
  const uint32_t gmagic = cpg == 1 ? 0u : (uint32_t)(0xFFFFFFFFu / (uint32_t)cpg) + 1u;   // c / cpg == mulhi(c, gmagic)

  u32x4 rw[D], rx[D][MT][4];
  uint32_t rs[D];
  auto issue = [&](int d, int j) {                          // this wave's j-th chunk into slot d
    const int c = wave + j * W;
    const bool live = c < KC;
    const int g = cpg == 1 ? c : (int)__umulhi((uint32_t)c, gmagic);
    rw[d] = buffer_load16_nt(wr, live && wlive ? woff + c * wstep : kOutOfRange);
    // scales non-temporal like the weights: 0.15-0.2 us per call sooner on 2048 x 2048 and 2048 x 256 (MI355X); the
    // row-group kernel above measured 0.3-1.5 us slower with it and keeps the default policy
    rs[d] = buffer_load2_nt(sr, live && slive ? soff + 2 * g : kOutOfRange);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        rx[d][mt][e] = buffer_load16(xr, live && xlive[mt] ? xoff[mt] + 256 * c + 16 * e : kOutOfRange);
  };
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const DecodeRegs dc = decode_regs();
  float rnr[MT];                                            // 1 / RMS of this lane's B rows (norm)
  auto consume = [&](int d, int c) {                        // slot d holds chunk c
    f32x4 pt[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) pt[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x8 a = decode_word_a(rw[d][j], dc);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const u32x4 b =
            norm ? rms_apply8(rx[d][mt][j], *reinterpret_cast<const u32x4*>(lds_g + 2 * (128 * c + 32 * q + 8 * j)), rnr[mt])
                 : rx[d][mt][j];
        pt[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(f16x8, b), pt[mt], 0, 0, 0);
      }
    }
    const uint32_t sb = rs[d];
    const float sc[4] = {(float)__builtin_bit_cast(f16, (uint16_t)quad_bcast<0>(sb)),
                         (float)__builtin_bit_cast(f16, (uint16_t)quad_bcast<1>(sb)),
                         (float)__builtin_bit_cast(f16, (uint16_t)quad_bcast<2>(sb)),
                         (float)__builtin_bit_cast(f16, (uint16_t)quad_bcast<3>(sb))};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[mt][v] = fmaf(pt[mt][v], sc[v], acc[mt][v]);
  };

  // this wave's chunks are wave + j W, j < nj; full groups of D refill their slot D chunks ahead (past the end the
  // refill reads zeros), the last partial group drains the ring
  const int nj = (KC - wave + W - 1) / W;
#pragma unroll
  for (int d = 0; d < D; ++d) issue(d, d);
  // wave 0 stores the outputs: up to 32 rows, their bias / residual elements are requested with the first weights
  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0;
  constexpr bool kAuxAhead = !ROPE && MT <= 2;
  Aux4 aux_pre[kAuxAhead ? MT : 1];
  if constexpr (kAuxAhead) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + r, n = n0 + 4 * q;
      aux_pre[mt] = wave == 0 && m < M && n < N ? aux_load4(epi, m, n, N, vec) : Aux4{};
    }
  }
  if (norm) {                                               // the rows' statistics while the ring is in flight
    stage_norm_weights(epi.norm_w, 0, KC, lds_g);
    rms_rows(xr, M, K, 16 * MT, epi.norm_eps, wave, W, lane, s_rn);
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) rnr[mt] = s_rn[16 * mt + r];
  }
  int j0 = 0;
  for (; j0 + D <= nj; j0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      consume(d, wave + (j0 + d) * W);
      issue(d, j0 + d + D);
    }
  }
#pragma unroll
  for (int d = 0; d < D - 1; ++d)
    if (j0 + d < nj) consume(d, wave + (j0 + d) * W);

  // waves 1 .. W-1 hand their sums to wave 0, which adds them in wave order
  if (W > 1) {
    f32x4* red = reinterpret_cast<f32x4*>(smem);             // [W - 1][MT][64]
    if (wave > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[((wave - 1) * MT + mt) * 64 + lane] = acc[mt];
    }
    __syncthreads();
    if (wave > 0) return;
    for (int w2 = 1; w2 < W; ++w2)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] += red[((w2 - 1) * MT + mt) * 64 + lane];
  }
  // lane (r, q) holds rows n0 + 4 q + v of column m = 16 mt + r
  if constexpr (ROPE) {                                     // every tile's loads and RoPE first, the stores after
    Out4 out[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + r, n = n0 + 4 * q;
      const f32x4 v = acc[mt];                              // partner rows 8 + 4 q + v sit 32 lanes on (q + 2)
      const f32x4 up = {shfl_down32(v[0]), shfl_down32(v[1]), shfl_down32(v[2]), shfl_down32(v[3])};
      out[mt] = q < 2 && m < M && n < N ? rope_qkv_out4(epi, m, n, v, up) : Out4{};
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) store_rope4(out[mt]);
    return;
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + r, n = n0 + 4 * q;
    const f32x4 v = acc[mt];
    if (epi.mode == kEpiSiluMul) {                          // up rows 8 + 4 q + v sit 32 lanes on (q + 2)
      const f32x4 up = {shfl_down32(v[0]), shfl_down32(v[1]), shfl_down32(v[2]), shfl_down32(v[3])};
      if (q < 2 && m < M && n < N) {
        f16* dst = y + (size_t)m * (N / 2) + 8 * (n >> 4) + (n & 15);
        const f16x2 lo = {silu_mul(v[0], up[0]), silu_mul(v[1], up[1])}, hi = {silu_mul(v[2], up[2]), silu_mul(v[3], up[3])};
        *reinterpret_cast<uint2*>(dst) = make_uint2(as_u32(lo), as_u32(hi));
      }
      continue;
    }
    if (m >= M || n >= N) continue;
    f16* dst = y + (size_t)m * N + n;
    if constexpr (kAuxAhead) {
      const Aux4& a = aux_pre[mt];
      if (vec) {
        const f16x2 lo = {epi_apply(epi.mode, a.v[0], v[0]), epi_apply(epi.mode, a.v[1], v[1])};
        const f16x2 hi = {epi_apply(epi.mode, a.v[2], v[2]), epi_apply(epi.mode, a.v[3], v[3])};
        *reinterpret_cast<uint2*>(dst) = make_uint2(as_u32(lo), as_u32(hi));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < N) dst[e] = epi_apply(epi.mode, a.v[e], v[e]);
      }
    } else if (vec) {
      const f16x2 lo = {epi_value(epi.mode, epi.aux, v[0], m, n, N), epi_value(epi.mode, epi.aux, v[1], m, n + 1, N)};
      const f16x2 hi = {epi_value(epi.mode, epi.aux, v[2], m, n + 2, N), epi_value(epi.mode, epi.aux, v[3], m, n + 3, N)};
      *reinterpret_cast<uint2*>(dst) = make_uint2(as_u32(lo), as_u32(hi));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < N) dst[e] = epi_value(epi.mode, epi.aux, v[e], m, n + e, N);
    }
  }
}

namespace {

template <int MT, int RW, int D, int KS, int TW = kW>
hipError_t launch_gemm(const GemvArgs& a, const GemvPlan& p, uint32_t* ctr, float* part) {
  if constexpr (!gemm_fits(MT, RW, D, KS, TW)) {
    return hipErrorInvalidConfiguration;                    // never planned
  } else {
    const int ntiles = (a.N + 15) / 16, groups = (ntiles + TW * RW - 1) / (TW * RW);
    // x buffers, then (input norm) the norm weights of the longest split's chunks; the K-group sums reuse the space
    const int KC = a.K / 128;
    const size_t xbytes = (size_t)KS * 2 * 16 * MT * kXPitch, redbytes = (size_t)(KS - 1) * TW * RW * MT * 1024;
    const size_t gbytes = a.epi.norm_w ? (size_t)256 * ((KC + p.S - 1) / p.S) : 0;
    const size_t shmem = std::max(xbytes + gbytes, redbytes);
    // the RoPE epilogue is its own instantiation: its registers would cost every other epilogue occupancy
    auto kern = a.epi.mode == kEpiRopeQKV ? gemm_mfma<MT, RW, D, KS, TW, true> : gemm_mfma<MT, RW, D, KS, TW, false>;
    if (shmem > 65536) {                                     // above the default dynamic LDS limit (gfx950 has 160 KB)
      // (x buffers at most 128 KB; the norm weights of K <= 8192 at most 16 KB more)
      static const hipError_t attr[2] = {allow_lds(gemm_mfma<MT, RW, D, KS, TW, false>, kGemmMaxLds),
                                         allow_lds(gemm_mfma<MT, RW, D, KS, TW, true>, kGemmMaxLds)};
      if (attr[0] != hipSuccess) return attr[0];
      if (attr[1] != hipSuccess) return attr[1];
    }
    const dim3 grid = p.XO ? dim3(groups * p.S) : dim3(groups, p.S);
    return launch(kern, grid, dim3(64 * TW * KS), shmem, a.stream, a.x, a.w, a.s, a.y, a.M, a.N, a.K, a.G, p.S, ctr,
                  part, a.epi);
  }
}

// K-groups of 3, 5, 6 or 8 tile-waves are built with one tile per wave and 2 ring slots (3 also for 5 and 6)
template <int MT, int D>
hipError_t dispatch_wide56(const GemvArgs& a, const GemvPlan& p, uint32_t* ctr, float* part, int ks) {
  if (p.KW == 5) return ks == 1 ? launch_gemm<MT, 1, D, 1, 5>(a, p, ctr, part) : launch_gemm<MT, 1, D, 2, 5>(a, p, ctr, part);
  return ks == 1 ? launch_gemm<MT, 1, D, 1, 6>(a, p, ctr, part) : launch_gemm<MT, 1, D, 2, 6>(a, p, ctr, part);
}

template <int MT>
hipError_t dispatch_wide(const GemvArgs& a, const GemvPlan& p, uint32_t* ctr, float* part) {
  const int ks = p.waves / p.KW;
  switch (p.KW) {
    case 3:
      return ks == 1 ? launch_gemm<MT, 1, 2, 1, 3>(a, p, ctr, part)
           : ks == 2 ? launch_gemm<MT, 1, 2, 2, 3>(a, p, ctr, part) : launch_gemm<MT, 1, 2, 4, 3>(a, p, ctr, part);
    case 5:
    case 6: return p.D == 3 ? dispatch_wide56<MT, 3>(a, p, ctr, part, ks) : dispatch_wide56<MT, 2>(a, p, ctr, part, ks);
    default: return ks == 1 ? launch_gemm<MT, 1, 2, 1, 8>(a, p, ctr, part) : launch_gemm<MT, 1, 2, 2, 8>(a, p, ctr, part);
  }
}

template <int MT, int RW, int D>
hipError_t dispatch_kgroups(const GemvArgs& a, const GemvPlan& p, uint32_t* ctr, float* part) {
  switch (p.waves / kW) {
    case 1: return launch_gemm<MT, RW, D, 1>(a, p, ctr, part);
    case 2: return launch_gemm<MT, RW, D, 2>(a, p, ctr, part);
    default: return launch_gemm<MT, RW, D, 4>(a, p, ctr, part);
  }
}

template <int MT, int RW>
hipError_t dispatch_ring(const GemvArgs& a, const GemvPlan& p, uint32_t* ctr, float* part) {
  switch (p.D) {
    case 2: return dispatch_kgroups<MT, RW, 2>(a, p, ctr, part);
    case 3: return dispatch_kgroups<MT, RW, 3>(a, p, ctr, part);
    default: return dispatch_kgroups<MT, RW, 4>(a, p, ctr, part);
  }
}

// one tile per workgroup, up to 8 waves (the register budget of 2 waves per SIMD); ring slots as tiles_ring allows
template <int MT, int D>
hipError_t launch_tiles_d(const GemvArgs& a, int waves) {
  constexpr int kThreads = 512;
  if (waves < 1 || 64 * waves > kThreads) return hipErrorInvalidConfiguration;   // never planned
  const size_t shmem = (size_t)(waves - 1) * MT * 64 * 16 + (a.epi.norm_w ? (size_t)2 * a.K : 0);   // + norm weights
  auto kern = a.epi.mode == kEpiRopeQKV ? gemm_mfma_tiles<MT, D, kThreads, true> : gemm_mfma_tiles<MT, D, kThreads, false>;
  return launch(kern, dim3((a.N + 15) / 16), dim3(64 * waves), shmem, a.stream, a.x, a.w,
                a.s, a.y, a.M, a.N, a.K, a.G, a.epi);
}

template <int MT>
hipError_t launch_tiles(const GemvArgs& a, int waves, int D) {
  if constexpr (MT <= 2) {
    if (D >= 4) return launch_tiles_d<MT, 4>(a, waves);
  }
  if constexpr (MT <= 3) {
    if (D == 3) return launch_tiles_d<MT, 3>(a, waves);
  }
  return launch_tiles_d<MT, 2>(a, waves);
}

template <int MT>
hipError_t dispatch_rows(const GemvArgs& a, const GemvPlan& p, uint32_t* ctr, float* part) {
  if (p.KW != kW) return dispatch_wide<MT>(a, p, ctr, part);
  switch (p.R) {
    case 1: return dispatch_ring<MT, 1>(a, p, ctr, part);
    default: return dispatch_ring<MT, 2>(a, p, ctr, part);
  }
}

}  // namespace

// One tile per workgroup beats row groups, from an MI355X sweep (graph-timed, cold weights, M = 2..64 on the
// Qwen2.5-1.5B/3B/7B projections), on the attention-sized layers: up to 256 tiles (one round of workgroups), K up to
// 4096 (KC <= 32) and KC * M <= 256 (384 for K <= 1536), i.e. while every wave's own activation loads (4 KB per 1 KB
// of weights per 16 rows of M) stay cheap: 2048 x 2560 at M = 16 5.7 us against 6.3 for the best row-group plan,
// 1536 x 2048 at M = 32 6.6 against 6.9, 3584 x 3584 at M = 8 6.6 against 7.9; 2048 x 2048 at M = 24 7.4 against
// 7.0 with row groups. Past that, row groups with K split over workgroups (since the split partials are handed over
// without an L2 write-back) win: 2048 x 2048 at M = 32 7.0 against 8.0, at M = 48 7.9 against 10.2; 3584 x 3584 at
// M = 16 8.0 against 8.4; 3584 x 4608 (288 tiles) at M = 16 8.2 against 12.5. Long K (8960 and up) keeps row groups
// at every M (11008 x 2048, M = 2: 9.9 against 12.9).
bool tiles_win(int M, int ntiles, int KC) { return ntiles <= 256 && KC <= 32 && KC * M <= (KC <= 12 ? 384 : 256); }

// deepest ring the one-tile kernel holds without spilling at 8 waves (hipcc -O3, gfx950: 112 / 186 / 204 registers at
// MT = 1 / 2 / 3 with 4 / 4 / 3 slots; MT = 4 spills at 3 slots)
int tiles_ring(int MT) { return MT <= 2 ? 4 : MT == 3 ? 3 : 2; }

// tile-waves per K-group for one tile per wave: 4, or 5, 6 or 8 where that lets every workgroup run in one round on
// the 256 CUs, or 3 where 4 would leave CUs idle. A CU that receives a second workgroup of 4 tile-waves takes ~1.7x as
// long as one with a single workgroup (3584 x 17408 at M = 64: 28.6 us with 272 workgroups, 3584 x 16384: 17.4 us
// with 256), so a layer of 1025 to 2048 tiles takes the fewest tile-waves that fit one round (MI355X graph sweep,
// M = 16..64: 3584 x 18944 with 237 workgroups of 5, M = 64 29.3 -> 23.0 us, M = 32 18.7 -> 14.1; 2048 x 22016 with
// 230 of 6, M = 64 18.7 -> 15.2; 1536 x 17920 with 224 of 5, M = 64 15.0 -> 12.5). Past 2048 tiles, up to 48 rows, the
// count that leaves the fewest tiles per CU, (workgroups / 256 rounded up) x tile-waves (3584 x 37888: 5, M = 32
// 27.9 -> 23.2 us); at 64 rows those layers take 6 with one K-group (3584 x 37888: 39.4 us with 4, 38.4 with 5 and
// 2 K-groups, 34.4 with 6 and 1; 35.0 vs 39.6 for 4 in an earlier sweep). Up to 16 rows a layer of 385 to 768
// tiles takes 3, so that its 129-256 workgroups occupy more CUs than the 97-192 of 4 (2048 x 11008: 6.82 -> 6.46 us;
// 1536 x 8960: 6.04 -> 5.78); from 17 rows 4 is level or up to 3% faster.
int balanced_tile_waves(int ntiles, int MT) {
  constexpr int kCUs = 256;
  if (MT == 1 && ntiles > 3 * 128 && ntiles <= 3 * kCUs) return 3;
  if (ntiles <= kW * kCUs) return kW;
  for (int tw : {5, 6, 8})
    if ((ntiles + tw - 1) / tw <= kCUs) return tw;
  if (MT > 3) return 6;
  int best = kW;
  long best_tiles = (long)((ntiles + kW - 1) / kW + kCUs - 1) / kCUs * kW;
  for (int tw : {5, 6, 8}) {
    const long tiles = (long)((ntiles + tw - 1) / tw + kCUs - 1) / kCUs * tw;
    if (tiles < best_tiles) best = tw, best_tiles = tiles;
  }
  return best;
}

// Launch shape from an MI355X sweep (graph-timed, cold weights, M in 2..64 on the Qwen2.5-3B/7B MLP shapes): one
// tile per wave; K split across workgroups while the row groups times the split stay within 256 workgroups (narrow
// N) and every split keeps at least 4 chunks, or 2 while the workgroups stay within half of 256, only for layers with
// fewer than 128 row groups (1536 x 8960, 140 row groups, split 2 ways 19.7 us, unsplit 5.9 us; 3584 x 3584, 56 row
// groups, 4 ways; 2048 x 2048 at M = 32 6.6-7.0 us with 4 ways against 7.1-8.4 with 8; 3584 x 4608, 72 row groups,
// 9.6 with 2 against 10.8 with 4). The 2-chunk splits pay since the fixup requests every partial at once (`bench.py
// --sweep splits`: 3584 x 512 at M = 16..64 8 ways 5.9-9.1 us against 6.6-10.4 with 4; 2048 x 256 at M = 32..64 8
// ways, 6-9% faster; 1536 x 2048 and 1536 x 256 at M = 64 4 ways, 8.9 / 8.8 us against 9.6 unsplit). K-groups per
// workgroup until
// about kGemmTargetWaves waves run (at most 2 K-groups for 17..32 rows; up to 16 rows 4, also where the row groups
// alone reach that many waves: 3584 x 16384, 256 row groups, M = 16, 10.3 -> 9.6 us against 2); from 33 rows K-groups
// double only while the waves stay within kGemmMaxWavesWide (3B gate/up at M = 64 12.3 us with 2 K-groups against
// 13.5 with 4, 7B gate/up 28.4 with 1 against 29.1 with 2, best or within 1% of best on the eight 1.5B / 3B / 7B MLP
// shapes at M = 48 and 64, while at M = 24..32 two K-groups stay faster on the widest layers: 7B gate/up 17.9 vs
// 18.8 us at M = 24); a 3-slot ring for M <= 16 with up to two K-groups of 4 tile-waves, else 2 slots.
GemvPlan plan_gemm_mfma(int M, int N, int K, int row_tiles, size_t workspace_bytes) {
  GemvPlan p;
  const GemvOverride o = gemv_override();
  const int ntiles = (N + 15) / 16, KC = K / 128;
  p.MT = (M + 15) / 16;
  if (p.MT <= 4 && row_tiles == 0 && (o.gemm_kernel == 2 || (o.gemm_kernel == 0 && tiles_win(M, ntiles, KC)))) {
    int waves = KC >= 16 ? 8 : 4;                             // same sweep (2048 x 2048, M = 2: 4.35 us against 4.84)
    if (o.waves > 0) waves = o.waves;
    waves = std::min(waves, 8);
    while (waves > 1 && waves > KC) waves /= 2;
    p.TW = waves;
    p.D = (o.ring >= 2 && o.ring <= 4) ? std::min(o.ring, tiles_ring(p.MT)) : tiles_ring(p.MT);
    return p;
  }
  p.R = row_tiles >= 2 ? 2 : 1;
  if (p.R == 1) p.KW = o.tile_waves > 0 ? o.tile_waves : balanced_tile_waves(ntiles, p.MT);
  const int KW = p.KW;
  const int groups = (ntiles + KW * p.R - 1) / (KW * p.R);
  // the partials are addressed with 32-bit byte offsets (a buffer resource): at most 2^31 - 1 bytes of them
  const size_t part_bytes = std::min<size_t>(workspace_bytes > kCounterBytes ? workspace_bytes - kCounterBytes : 0,
                                             (size_t)INT_MAX);
  int S = 1;
  if (o.splits > 0) {
    S = o.splits;
  } else if (part_bytes > 0) {
    while (S < kMaxSplits && groups < 128 && (long)groups * S * 2 <= kGemmMaxGroups &&
           KC >= ((long)groups * S * 2 <= kGemmMaxGroups / 2 ? 4 : 8) * S)
      S *= 2;
  }
  S = std::min(S, std::max(1, KC));
  while (S > 1 && (size_t)S * M * N * sizeof(float) > part_bytes) --S;
  if (groups > (int)(kCounterBytes / 4)) S = 1;
  int ks = 1;
  if (o.waves >= 4) {
    ks = o.waves / 4;
  } else if (KW != kW && groups <= 256) {                   // one round of 3, 5, 6 or 8 tile-waves: 2 K-groups (the
    ks = KW == 3 && p.MT == 1 ? 4 : 2;                      // same sweep: 3584 x 18944, M = 48, 20.6 -> 16.8 us), 4
  } else if (p.MT == 1 && S == 1) {                         // for 3 tile-waves at 16 rows (2048 x 11008: 7.19 -> 6.46)
    while (ks < 4 && 2 * ks <= KC) ks *= 2;
  } else if (p.MT <= 2) {
    // a K split up to 16 rows, or 17-32 rows: 2 K-groups (2048 x 11008 at M = 32 8.2 us against 8.6 with 1; split
    // layers at M = 16: 8960 x 1536 9.7 against 10.1 with 4)
    while (ks < 2 && (long)groups * S * KW * ks < kGemmTargetWaves && 2 * ks * S <= KC) ks *= 2;
  } else {
    // from 33 rows: fewer, longer K-groups (see above), and on an unsplit layer at least 4 chunks each (1536 x 2048
    // at M = 48: 7.97 us with 2 against 8.35 with 4); but up to 4 on layers split 4 or more ways (2048 x 2560 7.9 us
    // against 8.2 with 2; 2048 x 2048 7.8 against 8.0), except, at 33-48 rows, where each split keeps 6 chunks or more
    // (8960 x 1536 at M = 48 10.9 us with 2 against 11.8 with 4, 11008 x 2048 12.0 against 12.6, 3584 x 3584 10.0
    // against 10.2)
    const long cap = S >= 4 ? 2L * kGemmMaxWavesWide : (long)kGemmMaxWavesWide;
    const int ks_max = p.MT == 3 && KC / S >= 6 ? 2 : 4;
    while (ks < ks_max && (long)groups * S * KW * 2 * ks <= cap && 2 * ks * S <= KC && (S > 1 || 8 * ks <= KC)) ks *= 2;
  }
  while (ks > 1 && ks * S > KC) ks /= 2;
  p.D = (o.ring >= 2 && o.ring <= 4) ? o.ring : ((p.MT == 1 && ks <= 2) ? 3 : 2);
  // 5 or 6 tile-waves: 2 slots, or 3 on one round of workgroups with 2 K-groups of at least 12 chunks each up to 32
  // rows (MI355X graph sweep, 3584 x 18944: M = 16 11.64 -> 11.46 us, M = 32 14.11 -> 13.84; at 48 and 64 rows, and on
  // 1536 x 17920, 2048 x 22016 and the two-round 3584 x 37888, the third slot costs 1-3%)
  if (KW != kW) {
    const bool deep = p.MT <= 2 && ks == 2 && groups <= 256 && KC >= 24 && (KW == 5 || KW == 6);
    p.D = o.ring == 2 || o.ring == 3 ? (o.ring == 3 && (KW == 5 || KW == 6) ? 3 : 2) : (deep ? 3 : 2);
  }
  while (!gemm_fits(p.MT, p.R, p.D, ks, KW)) {              // fewer K-groups, then fewer slots, then fewer tiles
    if (ks > 1) ks /= 2;
    else if (p.D > 2) --p.D;
    else p.R = 1;
  }
  p.waves = KW * ks;
  p.S = std::max(S, 1);
  p.XO = p.S > 1 && o.gemm_order == 2 ? 1 : 0;
  // one arrival counter per row group of the final shape (R may have dropped to 1 above)
  if (p.S > 1 && (ntiles + KW * p.R - 1) / (KW * p.R) > (int)(kCounterBytes / 4)) p.S = 1;
  return p;
}

// clears n 32-bit words with vector stores (a kernel rather than a memset, so that it may sit in a captured graph)
__global__ __launch_bounds__(256) void zero_words(uint32_t* __restrict__ p, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

hipError_t zero_words_launch(void* p, int n, hipStream_t stream) {
  const int blocks = std::max(1, std::min((n + 255) / 256, 64));
  return launch(zero_words, dim3(blocks), dim3(256), 0, stream, static_cast<uint32_t*>(p), n);
}

hipError_t gemm_mfma_launch(const GemvArgs& a0, int row_tiles, void* workspace, size_t workspace_bytes) {
  GemvArgs a = a0;                                          // the input norm travels with the epilogue
  a.epi.norm_w = a0.norm_w;
  a.epi.norm_eps = a0.eps;
  GemvPlan p = plan_gemm_mfma(a.M, a.N, a.K, row_tiles, workspace ? workspace_bytes : 0);
  if (p.TW > 0 && p.MT > kTilesNormMaxMT && a.norm_w)    // row groups normalize at every M
    p = plan_gemm_mfma(a.M, a.N, a.K, 1, workspace ? workspace_bytes : 0);
  if (p.TW > 0)
    return p.MT == 1 ? launch_tiles<1>(a, p.TW, p.D) : p.MT == 2 ? launch_tiles<2>(a, p.TW, p.D)
         : p.MT == 3 ? launch_tiles<3>(a, p.TW, p.D) : launch_tiles<4>(a, p.TW, p.D);
  uint32_t* ctr = static_cast<uint32_t*>(workspace);
  float* part = workspace ? reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kCounterBytes) : nullptr;
  switch (p.MT) {
    case 1: return dispatch_rows<1>(a, p, ctr, part);
    case 2: return dispatch_rows<2>(a, p, ctr, part);
    case 3: return dispatch_rows<3>(a, p, ctr, part);
    default: return dispatch_rows<4>(a, p, ctr, part);
  }
}

}  // namespace lowbit
