// Prefill GEMM on the MFMA layout, M > 64: y[M, N] = x[M, K] . dequant(W)^T with v_mfma_f32_16x16x32_f16, reading
// the int4 weights directly (no fp16 copy of W). The reference's prefill dequantizes into an fp16 W and calls cuBLAS
// (lowbit/ops.py:126-135,163-178); this kernel computes the same products without writing W out.
//
// Operands (lane l, r = l % 16, q = l / 16), as in the skinny kernel:
//   A (16 weight rows x 32 k): lane l's 16-byte piece of a 1 KB block holds row r, k = 128 c + 32 q + 8 s + 0..7 in
//     word s, which feeds k-step s. Each word is decoded to (u - 8) exactly in fp16 and multiplied by the row's fp16
//     group scale with one rounding, so A holds exactly the dequantized weights of the reference's rule.
//   B (32 k x 16 activation rows): x[m0 + 16 mt + r][128 c + 32 q + 8 s + 0..7], 16 bytes from LDS.
//   D: lane l holds y[m0 + 16 mt + r][16 t + 4 q + v], v = 0..3.
//
// Workgroup: 4 waves, each owning PT 16-row tiles (64 PT weight rows per workgroup; PT = 4, or 2 or 1 when the grid
// would leave CUs idle), against 16 MT activation rows.
// Every wave decodes only its own rows, so no weight is decoded twice; the activation chunk is loaded once per
// workgroup (16 bytes per thread and row piece) and shared through LDS, double buffered with one barrier per 128-k
// chunk. LDS rows are 256 bytes with the 16-byte column blocks XOR-swizzled by the row (block b of row m at
// b ^ (m % 16)), so both the stores of a row and the 16-row fragment reads hit 16 different bank groups.
// Weight pieces and scales run D chunks ahead in registers; the next chunk of x is requested before the current
// chunk's MFMAs and written to LDS after them. Buffer loads make tails free: rows past N, chunks past the split's
// range and activation rows past M read zeros.
//
// Work items (tile = 256 rows x 16 MT activation rows, times S splits of K) are numbered with the split fastest, then
// the activation group, then the row group, and the workgroup -> item map puts consecutive items on the same XCD
// (workgroup i runs on XCD i % 8), so the workgroups that share weight rows share that XCD's L2. With S > 1 each
// workgroup writes fp32 partials to the workspace (agent-coherent stores); the last to arrive on a per-tile counter
// adds them in split order, applies the epilogue and resets the counter, as in the skinny kernel.
#include <algorithm>
#include <climits>

#include "kernels.hpp"

namespace lowbit {

namespace {


__device__ __forceinline__ int swz(int row, int blk) { return row * 16 + (blk ^ (row & 15)); }   // 16-byte slot

}  // namespace

// Waves per SIMD the register allocation must leave room for: 2 for the 4-tile, 2-slot shapes (at most 256 registers
// a wave, so two 4-wave workgroups share a CU), which fit in that budget without spilling; 1 for the 8-tile and 3-slot
// shapes, which do not. Without the bound hipcc gave the 4 x 4-tile shape 260 registers (188 + 72 accumulation
// registers): one workgroup per CU, and 3B gate|up at 2048 rows took 455 us instead of 249 (MI355X, cold weights).
constexpr int prefill_min_waves(int MT, int D) { return MT == 4 && D == 2 ? 2 : 1; }

template <int MT, int D, int NW, int XL, int PT, bool ROPE>
__global__ __launch_bounds__(64 * NW, prefill_min_waves(MT, D)) void gemm_prefill(const f16* __restrict__ x, const uint8_t* __restrict__ w,
                                                    const f16* __restrict__ s, f16* y, int M, int N, int K, int G,
                                                    int S, int MG, int items, uint32_t* __restrict__ ctr,
                                                    float* __restrict__ part, Epilogue epi) {
  constexpr int kXBuf = 16 * MT * 256;                      // one staged chunk of x
  constexpr int kRows = 16 * PT * NW;                       // weight rows per workgroup
  args_in_sgprs(x, w, s, y, M, N, K, G, S, MG, items, ctr, part, epi.aux);
  constexpr int kThreads = 64 * NW;
  constexpr int XP = 16 * MT * 16 / kThreads;               // 16-byte x pieces per thread and chunk
  static_assert(XP >= 1 && XP * kThreads == 16 * MT * 16, "x pieces must divide evenly");
  static_assert(D == 2 || XL == 1, "a 3-deep weight ring runs with a one-chunk x lookahead");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q = lane >> 4;

  // workgroup -> work item: consecutive items on one XCD
  const int per = items >> 3, rem = items & 7, xcd = blockIdx.x & 7, idx = blockIdx.x >> 3;
  const int item = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  const int sp = item % S, tile = item / S, mg = tile % MG, ng = tile / MG;
  const int m0 = 16 * MT * mg, n0 = kRows * ng;
  const int ntiles = (N + 15) >> 4, KC = K >> 7, KG = K / G, cpg = G >> 7;
  const int cb = (int)((int64_t)KC * sp / S), ce = (int)((int64_t)KC * (sp + 1) / S);
  const int nsteps = ce - cb;
  const size_t tile_bytes = (size_t)8 * K;

  __amdgpu_buffer_rsrc_t wr[PT];
  int woff[PT], wstep[PT], soff[PT];
#pragma unroll
  for (int i = 0; i < PT; ++i) {
    const int t = n0 / 16 + PT * wave + i;
    const int tc = min(t, ntiles - 1);
    const int rows = t < ntiles ? min(16, N - 16 * t) : 0;
    wr[i] = make_rsrc(w + tc * tile_bytes, (uint32_t)(rows * (K / 2)));
    woff[i] = r < rows ? 64 * r + 16 * q : kOutOfRange;
    wstep[i] = r < rows ? rows * 64 : 0;
    soff[i] = r < rows ? 2 * (16 * t + r) * KG : kOutOfRange;   // the scale of this lane's A row
  }
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(s, (uint32_t)N * (uint32_t)KG * 2u);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)M * (uint32_t)K * 2u);
  int xoff[XP], xslot[XP];                                  // piece tid + kThreads u: row p / 16, block p % 16
#pragma unroll
  for (int u = 0; u < XP; ++u) {
    const int pc = tid + kThreads * u;
    xoff[u] = ((m0 + (pc >> 4)) * K + 8 * (pc & 15)) * 2;
    xslot[u] = 16 * swz(pc >> 4, pc & 15);
  }

  u32x4 rw[D][PT], rx[XL][XP];
  uint32_t rs[D][PT];
  const uint32_t gmagic = cpg == 1 ? 0u : (uint32_t)(0xFFFFFFFFu / (uint32_t)cpg) + 1u;   // c / cpg == mulhi(c, gmagic)
  auto issue_w = [&](int d, int c) {
    const bool live = c < ce;
    const int g = cpg == 1 ? c : (int)__umulhi((uint32_t)c, gmagic);
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      rw[d][i] = buffer_load16(wr[i], live ? woff[i] + c * wstep[i] : kOutOfRange);   // re-read by other m-groups
      rs[d][i] = buffer_load2(sr, live ? soff[i] + 2 * g : kOutOfRange);
    }
  };
  auto issue_x = [&](int e, int c) {
#pragma unroll
    for (int u = 0; u < XP; ++u) rx[e][u] = buffer_load16(xr, c < ce ? xoff[u] + 256 * c : kOutOfRange);
  };
  auto stage_x = [&](int e, int b) {
#pragma unroll
    for (int u = 0; u < XP; ++u) *reinterpret_cast<u32x4*>(smem + b * kXBuf + xslot[u]) = rx[e][u];
  };

  f32x4 acc[PT][MT];
#pragma unroll
  for (int i = 0; i < PT; ++i)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const f16x2 m1032 = {(f16)-1032.0f, (f16)-1032.0f}, m72 = {(f16)-72.0f, (f16)-72.0f};
  const f16x2 inv16 = {(f16)0.0625f, (f16)0.0625f};
  const DecodeRegs dc = decode_regs();                      // masks and magic in registers: v_and_or_b32
  // one chunk: the 16 A fragments (4 tiles x 4 k-steps) are decoded first; then per activation tile its 4 B
  // fragments are read and 16 MFMAs issued, so at most two tiles' B fragments are live
  auto consume = [&](int d, int b) {
    f16x8 a[PT][4];
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const f16 sv = __builtin_bit_cast(f16, (uint16_t)rs[d][i]);
      const f16x2 sc = {sv, sv};
#pragma unroll
      for (int st = 0; st < 4; ++st) {                      // (u - 8) exact, times the scale: one rounding
        const uint32_t wd = rw[d][i][st], w8 = wd >> 8;
        const f16x2 p0 = (as_f16x2((wd & dc.lo) | dc.magic) + m1032) * sc;
        const f16x2 p1 = (as_f16x2((wd & dc.hi) | dc.magic) * inv16 + m72) * sc;
        const f16x2 p2 = (as_f16x2((w8 & dc.lo) | dc.magic) + m1032) * sc;
        const f16x2 p3 = (as_f16x2((w8 & dc.hi) | dc.magic) * inv16 + m72) * sc;
        a[i][st] = __builtin_bit_cast(f16x8, u32x4{as_u32(p0), as_u32(p1), as_u32(p2), as_u32(p3)});
      }
    }
    const uint8_t* xb = smem + b * kXBuf;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f16x8 bx[4];
#pragma unroll
      for (int st = 0; st < 4; ++st)
        bx[st] = *reinterpret_cast<const f16x8*>(xb + 16 * swz(16 * mt + r, 4 * q + st));
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < PT; ++i) acc[i][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i][st], bx[st], acc[i][mt], 0, 0, 0);
    }
  };

#pragma unroll
  for (int e = 0; e < XL; ++e) issue_x(e, cb + e);
#pragma unroll
  for (int d = 0; d < D; ++d) issue_w(d, cb + d);
  stage_x(0, 0);
  __syncthreads();

  // step j: chunk cb + j, weight slot j % D, x register set j % XL, LDS buffer j % 2. The x of chunk j + XL goes
  // into the set chunk j used (already in LDS) before the MFMAs; after them chunk j + 1 is staged into the other
  // buffer and the weight slot just consumed is refilled D chunks ahead. The loop is unrolled D times (D % XL == 0),
  // so every slot and set index is a constant.
  int j0 = 0;
  for (; j0 + D <= nsteps; j0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int j = j0 + d;
      if (j + XL < nsteps) issue_x(d % XL, cb + j + XL);
      consume(d, j & 1);
      issue_w(d, cb + j + D);
      if (j + 1 < nsteps) stage_x((d + 1) % XL, (j + 1) & 1);
      __syncthreads();
    }
  }
#pragma unroll
  for (int d = 0; d < D - 1; ++d) {
    const int j = j0 + d;
    if (j < nsteps) {
      if (j + XL < nsteps) issue_x(d % XL, cb + j + XL);
      consume(d, j & 1);
      if (j + 1 < nsteps) stage_x((d + 1) % XL, (j + 1) & 1);
      __syncthreads();
    }
  }

  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0;
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
  auto store4_silu = [&](int m, int n, const f32x4& g, const f32x4& u) {
    f16* dst = y + (size_t)m * (N / 2) + 8 * (n >> 4) + (n & 15);
    const f16x2 lo = {silu_mul(g[0], u[0]), silu_mul(g[1], u[1])}, hi = {silu_mul(g[2], u[2]), silu_mul(g[3], u[3])};
    *reinterpret_cast<uint2*>(dst) = make_uint2(as_u32(lo), as_u32(hi));
  };
  if (S == 1) {
    if constexpr (ROPE) {                                   // per tile: the MT column tiles' loads and RoPE, then stores
#pragma unroll
      for (int i = 0; i < PT; ++i) {
        Out4 out[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = m0 + 16 * mt + r, n = n0 + 16 * (PT * wave + i) + 4 * q;
          const f32x4 v = acc[i][mt];                       // partner rows 8 + 4 q + v sit 32 lanes on (q + 2)
          const f32x4 up = {shfl_down32(v[0]), shfl_down32(v[1]), shfl_down32(v[2]), shfl_down32(v[3])};
          out[mt] = q < 2 && m < M && n < N ? rope_qkv_out4(epi, m, n, v, up) : Out4{};
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) store_rope4(out[mt]);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < PT; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = m0 + 16 * mt + r, n = n0 + 16 * (PT * wave + i) + 4 * q;
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
  for (int i = 0; i < PT; ++i)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m0 + 16 * mt + r, n = n0 + 16 * (PT * wave + i) + 4 * q;
      if (m >= M || n >= N) continue;
      const int off = poff(sp, m, n);
      if (vec) {
        store_partial4(pr, off, acc[i][mt]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < N) store_partial(pr, off + 4 * e, acc[i][mt][e]);
      }
    }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);                 // the partials' stores stay before the wait
  __builtin_amdgcn_s_waitcnt(0);                            // every partial acknowledged: visible to all XCDs
  __builtin_amdgcn_s_barrier();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(ctr + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == (uint32_t)(S - 1);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);                 // the partials' loads stay after the count
  if (!s_last) return;
  if (tid == 0) __hip_atomic_store(ctr + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int nrows = min(kRows, N - n0), nq = (nrows + 3) >> 2, mrows = min(16 * MT, M - m0);
  auto split_sum = [&](int m, int n) {                      // partials of rows n .. n + 3, added in split order
    return sum_partials4(pr, S, (N & 3) == 0 ? 4 : min(4, N - n), [&](int k) { return poff(k, m, n); });
  };
  for (int it = tid; it < mrows * nq; it += kThreads) {
    const int m = m0 + it / nq, n = n0 + 4 * (it % nq);
    if constexpr (ROPE) {
      if ((n & 15) < 8) store_rope4(rope_qkv_out4(epi, m, n, split_sum(m, n), split_sum(m, n + 8)));
    } else if (epi.mode == kEpiSiluMul) {
      if ((n & 15) < 8) store4_silu(m, n, split_sum(m, n), split_sum(m, n + 8));
    } else {
      store4(m, n, split_sum(m, n));
    }
  }
}

namespace {

template <int MT, int D, int NW, int XL, int PT = 4>
hipError_t launch_prefill(const GemvArgs& a, const PrefillPlan& p, uint32_t* ctr, float* part) {
  if constexpr (!prefill_fits(MT, D, NW, XL)) {
    return hipErrorInvalidConfiguration;                    // never planned
  } else {
  const size_t shmem = (size_t)2 * 16 * MT * 256;
  // the RoPE epilogue is its own instantiation: its registers would cost every other epilogue occupancy
  auto kern = a.epi.mode == kEpiRopeQKV ? gemm_prefill<MT, D, NW, XL, PT, true> : gemm_prefill<MT, D, NW, XL, PT, false>;
  if (shmem > 65536) {
    static const hipError_t attr[2] = {allow_lds(gemm_prefill<MT, D, NW, XL, PT, false>, shmem),
                                       allow_lds(gemm_prefill<MT, D, NW, XL, PT, true>, shmem)};
    if (attr[0] != hipSuccess) return attr[0];
    if (attr[1] != hipSuccess) return attr[1];
  }
  return launch(kern, dim3(p.items), dim3(64 * NW), shmem, a.stream, a.x, a.w, a.s, a.y, a.M, a.N, a.K, a.G, p.S, p.MG,
                p.items, ctr, part, a.epi);
  }
}

template <int MT, int NW>
hipError_t dispatch_prefill_ring(const GemvArgs& a, const PrefillPlan& p, uint32_t* ctr, float* part) {
  if constexpr (MT == 4 && NW == 4) {                       // fewer tiles per wave: the default shape only
    if (p.D == 2 && p.XL == 1 && p.PT == 1) return launch_prefill<4, 2, 4, 1, 1>(a, p, ctr, part);
    if (p.D == 2 && p.XL == 1 && p.PT == 2) return launch_prefill<4, 2, 4, 1, 2>(a, p, ctr, part);
  }
  if (p.D == 3) return launch_prefill<MT, 3, NW, 1>(a, p, ctr, part);
  return p.XL == 2 ? launch_prefill<MT, 2, NW, 2>(a, p, ctr, part) : launch_prefill<MT, 2, NW, 1>(a, p, ctr, part);
}

}  // namespace

// Launch shape from an MI355X sweep (graph-timed, M = 128 / 256 / 512 / 2048 on the Qwen2.5-3B and 7B projections):
// 64 activation rows x 4 waves with a 2-deep weight ring (2 workgroups per CU; deeper rings or the x lookahead cost
// the second wave per SIMD and lose), 4, 2 or 1 weight tiles per wave (below); K split into the largest power of two
// that keeps >= 16 chunks per split and at most two rounds of kPrefillTargetGroups workgroups, within the workspace
// and the counters. The tuning override selects (waves_per_group: 1 = MT 4 / 4 waves, 2 = MT 4 / 8 waves, 4 = MT 8 /
// 4 waves, 8 = MT 8 / 8 waves; ring: 2 or 3 = weight chunks in flight, 4 = two in flight with a two-chunk x lookahead),
// always with 4 tiles per wave.
PrefillPlan plan_gemm_prefill(int M, int N, int K, size_t workspace_bytes) {
  PrefillPlan p;
  const GemvOverride o = gemv_override();
  const int KC = K / 128;
  switch (o.waves) {
    case 1: p.MT = 4; p.NW = 4; break;
    case 2: p.MT = 4; p.NW = 8; break;
    case 4: p.MT = 8; p.NW = 4; break;
    case 8: p.MT = 8; p.NW = 8; break;
    default: p.MT = 4; p.NW = 4; break;
  }
  p.D = o.ring == 3 ? 3 : 2;
  p.XL = o.ring == 4 ? 2 : 1;
  if (!prefill_fits(p.MT, p.D, p.NW, p.XL)) p.NW = 4;      // 8 waves: 256 registers per wave, D = 2 and MT = 4 only
  if (!prefill_fits(p.MT, p.D, p.NW, p.XL)) p.D = 2;
  p.MG = (M + 16 * p.MT - 1) / (16 * p.MT);
  // fewer 16-row tiles per wave (default shape only): 2 up to 8 activation tiles (168 instead of 256 registers, a third
  // wave per SIMD: 3B merged gate|up at M = 512 89 -> 77 us, 7B gate|up 133 -> 106; at M = 2048 4 tiles stay ahead,
  // 365 vs 388), then halved while the grid holds less than two workgroups per CU. A wave's activation bytes per
  // chunk stay the same while its weight bytes shrink (x : w = 4 : PT), so past 4 activation tiles a long K (>= 128
  // chunks) splits across workgroups instead (7B down, M = 512: 130 us at 4 tiles and 2 splits vs 142 at 1 tile;
  // M = 2048: 351 vs 451; at M <= 256 and on K <= 11008 the thin tiles win up to 2.9x)
  auto groups = [&](int pt) { return (long)((N + 16 * pt * p.NW - 1) / (16 * pt * p.NW)) * p.MG; };
  p.PT = 4;
  if (o.waves == 0 && o.ring == 0 && (KC < 128 || p.MG <= 4)) {
    if (p.MG <= 8) p.PT = 2;
    while (p.PT > 1 && groups(p.PT) < 2 * kPrefillTargetGroups) p.PT /= 2;
  }
  const long tiles = groups(p.PT);
  // the partials are addressed with 32-bit byte offsets (a buffer resource): at most 2^31 - 1 bytes of them
  const size_t part_bytes = std::min<size_t>(workspace_bytes > kCounterBytes ? workspace_bytes - kCounterBytes : 0,
                                             (size_t)INT_MAX);
  int S = 1;
  if (o.splits > 0) {
    S = o.splits;
  } else if (part_bytes > 0) {
    while (S < kMaxSplits && tiles * 2 * S <= 2 * kPrefillTargetGroups && KC >= 16 * 2 * S) S *= 2;
  }
  S = std::min(S, std::max(1, KC));
  while (S > 1 && (size_t)S * M * N * sizeof(float) > part_bytes) --S;
  if (tiles > (long)(kCounterBytes / 4)) S = 1;
  p.S = std::max(S, 1);
  p.items = (int)(tiles * p.S);
  return p;
}

hipError_t gemm_prefill_launch(const GemvArgs& a, void* workspace, size_t workspace_bytes) {
  const PrefillPlan p = plan_gemm_prefill(a.M, a.N, a.K, workspace ? workspace_bytes : 0);
  uint32_t* ctr = static_cast<uint32_t*>(workspace);
  float* part = workspace ? reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kCounterBytes) : nullptr;
  if (p.MT == 4) return p.NW == 8 ? dispatch_prefill_ring<4, 8>(a, p, ctr, part) : dispatch_prefill_ring<4, 4>(a, p, ctr, part);
  return p.NW == 8 ? dispatch_prefill_ring<8, 8>(a, p, ctr, part) : dispatch_prefill_ring<8, 4>(a, p, ctr, part);
}

}  // namespace lowbit
