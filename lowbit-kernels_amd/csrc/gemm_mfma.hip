// Skinny GEMM on the MFMA layout, 1 <= M <= 64: y[M, N] = x[M, K] . dequant(W)^T with v_mfma_f32_16x16x32_f16.
// The role of the reference's tensor-core gemm_v5 (csrc/w4_gemv.cu:215-294), designed for CDNA4 wave64 MFMA.
//
// Operands of one 16x16x32 MFMA (lane l, r = l % 16, q = l / 16):
//   A (16 weight rows x 32 k): row r, 8 consecutive k of quarter q. In the MFMA layout lane l's 16-byte piece of a
//     1 KB block is exactly row r, k = 128 c + 32 q + [0, 32): word j of it feeds k-step j, so one coalesced 1 KB
//     wave-load gives the A fragments of four MFMAs with no shuffle.
//   B (32 k x 16 activation rows): x[16 mt + r][128 c + 32 q + 8 j + 0..7], one 16-byte load per lane and k-step.
//   D: lane l holds rows n = 16 t + 4 q + v (v = 0..3) of column m = 16 mt + r.
// Each lane decodes its words to exact (u - 8) fp16 values and multiplies them by the group's fp16 scale (one
// rounding: the same fp16 weights the dequant kernel writes), so accumulation across groups stays inside the MFMA
// accumulators. The waves of a workgroup split the K chunks and are summed through LDS at the end.
#include "kernels.hpp"

namespace lowbit {

template <int MT, int RT>
__global__ __launch_bounds__(256) void gemm_mfma(const f16* __restrict__ x, const uint8_t* __restrict__ w,
                                                 const f16* __restrict__ s, f16* __restrict__ y, int M, int N, int K,
                                                 int G) {
  extern __shared__ float red[];                          // [nwaves][RT][MT][64 lanes][4]
  const int lane = threadIdx.x & 63, nwaves = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int ntiles = (N + 15) >> 4, KC = K >> 7, KG = K / G, cpg = G >> 7;
  const size_t tile_bytes = (size_t)8 * K;
  const uint8_t* wp[RT];
  const f16* sp[RT];
  int rows[RT];
  bool live[RT];
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const int t = blockIdx.x * RT + i;
    rows[i] = t < ntiles ? min(16, N - 16 * t) : 0;
    live[i] = r < rows[i];
    wp[i] = w + (live[i] ? t * tile_bytes + 64 * r + 16 * q : 0);
    sp[i] = s + (size_t)(live[i] ? 16 * t + r : 0) * KG;
  }
  const f16* xr[MT];
  bool xlive[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + r;
    xlive[mt] = m < M;
    xr[mt] = x + (size_t)(xlive[mt] ? m : 0) * K + 32 * q;
  }
  f32x4 acc[RT][MT];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int c = wave; c < KC; c += nwaves) {
    u32x4 wv[RT];
    f16x2 sc[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      wv[i] = live[i] ? load_stream(wp[i] + (size_t)c * rows[i] * 64) : u32x4{0, 0, 0, 0};
      const f16 sv = sp[i][c / cpg];
      sc[i] = f16x2{sv, sv};
    }
    u32x4 xv[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[mt][j] = xlive[mt] ? load16(xr[mt] + 128 * c + 8 * j) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        f16x2 p[4];
        decode_word(wv[i][j], p);
        const f16x8 a = {(f16)0, (f16)0, (f16)0, (f16)0, (f16)0, (f16)0, (f16)0, (f16)0};
        f16x8 av = a;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f16x2 wsc = p[e] * sc[i];              // exact (u - 8) times the fp16 scale, rounded once
          av[2 * e] = wsc[0];
          av[2 * e + 1] = wsc[1];
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[i][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, __builtin_bit_cast(f16x8, xv[mt][j]), acc[i][mt], 0,
                                                              0, 0);
      }
    }
  }
  if (nwaves > 1) {
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        *reinterpret_cast<f32x4*>(red + ((((size_t)wave * RT + i) * MT + mt) * 64 + lane) * 4) = acc[i][mt];
    __syncthreads();
    // the waves share the final sums: tile-pair (i, mt) goes to wave (i * MT + mt) % nwaves
    for (int tp = wave; tp < RT * MT; tp += nwaves) {
      const int i = tp / MT, mt = tp % MT;
      f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int wv2 = 0; wv2 < nwaves; ++wv2)
        v += *reinterpret_cast<const f32x4*>(red + ((((size_t)wv2 * RT + i) * MT + mt) * 64 + lane) * 4);
      const int m = 16 * mt + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int n = 16 * (blockIdx.x * RT + i) + 4 * q + e;
        if (m < M && n < N) y[(size_t)m * N + n] = (f16)v[e];
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int n = 16 * (blockIdx.x * RT + i) + 4 * q + e;
          if (m < M && n < N) y[(size_t)m * N + n] = (f16)acc[i][mt][e];
        }
      }
  }
}

namespace {

template <int MT, int RT>
hipError_t launch_gemm(const GemvArgs& a, int waves) {
  const int ntiles = (a.N + 15) / 16;
  dim3 grid((ntiles + RT - 1) / RT), block(64 * waves);
  const size_t shmem = waves > 1 ? (size_t)waves * RT * MT * 64 * 4 * sizeof(float) : 0;
  return launch(gemm_mfma<MT, RT>, grid, block, shmem, a.stream, a.x, a.w, a.s, a.y, a.M, a.N, a.K, a.G);
}

template <int MT>
hipError_t dispatch_gemm(const GemvArgs& a, int RT, int waves) {
  switch (RT) {
    case 1: return launch_gemm<MT, 1>(a, waves);
    case 2: return launch_gemm<MT, 2>(a, waves);
    default: return launch_gemm<MT, 4>(a, waves);
  }
}

}  // namespace

GemvPlan plan_gemm_mfma(int M, int N, int K, int row_tiles) {
  GemvPlan p;
  const int MT = (M + 15) / 16, ntiles = (N + 15) / 16, KC = K / 128;
  int RT = row_tiles ? row_tiles : (M <= 16 ? 1 : 2);
  if (MT >= 3 && RT > 2) RT = 2;                 // accumulators: 4 RT MT floats per lane
  p.R = RT;
  const int blocks = (ntiles + RT - 1) / RT;
  int waves = 1;
  while (waves < 4 && waves * 2 <= KC && (long)blocks * waves < 2048) waves *= 2;
  p.waves = waves;
  p.MT = MT;
  return p;
}

hipError_t gemm_mfma_launch(const GemvArgs& a, int row_tiles) {
  const GemvPlan p = plan_gemm_mfma(a.M, a.N, a.K, row_tiles);
  switch (p.MT) {
    case 1: return dispatch_gemm<1>(a, p.R, p.waves);
    case 2: return dispatch_gemm<2>(a, p.R, p.waves);
    case 3: return dispatch_gemm<3>(a, p.R, p.waves);
    default: return dispatch_gemm<4>(a, p.R, p.waves);
  }
}

}  // namespace lowbit
