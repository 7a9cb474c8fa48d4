// Internal interface between the C ABI (capi.hip) and the kernel files. Callers validate every argument first.
#pragma once
#include "common.hpp"

namespace lowbit {

// What the MFMA-layout kernels do with each fp32 sum before storing it (all roundings as the unfused torch ops do
// them: the product is rounded to fp16 first):
//   kEpiStore     y[m][n] = fp16(acc)
//   kEpiBias      y[m][n] = fp16(acc) + bias[n]                          (aux = bias [N])
//   kEpiResidual  y[m][n] = residual[m][n] + fp16(acc)                   (aux = residual [M][N]; may be y itself)
//   kEpiSiluMul   rows interleaved 8 gate, 8 up per 16-row tile; y [M][N/2] = silu(fp16(gate)) * fp16(up),
//                 output column 8 t + r for gate row 16 t + r, up row 16 t + 8 + r
//   kEpiRopeQKV   the q|k|v projection of a decoder layer with its rows permuted per 128-row head so that tile j
//                 holds dims 8 j .. 8 j + 7 and 64 + 8 j .. 64 + 8 j + 7: fp16(acc) + aux[n] (bias), then RoPE at
//                 rope.pos[m] on q and k heads; q -> rope.q_out [M][Hq][128], k and v -> the caches' row pos[m] (as
//                 lowbit_rope_kv on the unfused output); the GEMV for one row (angles from rope.inv_freq), the MFMA
//                 and prefill GEMMs for more (cos and sin from the table rope.cos_sin)
enum : int { kEpiStore = 0, kEpiBias = 1, kEpiResidual = 2, kEpiSiluMul = 3, kEpiRopeQKV = 4 };
struct RopeArgs {
  const int64_t* pos = nullptr;
  const float* inv_freq = nullptr;         // the GEMV's: cos and sin evaluated in its store
  const uint32_t* cos_sin = nullptr;       // the GEMMs': the step's table [M][64] of fp16 (cos, sin) (rope_table)
  f16* q_out = nullptr;
  f16* k_cache = nullptr;
  f16* v_cache = nullptr;
  int Hq = 0, Hkv = 0, L = 0;
};
struct Epilogue {
  int mode = kEpiStore;
  const f16* aux = nullptr;
  RopeArgs rope;
  // one-row GEMV whose x is the merge of an attention step's key partitions (attention_partials_launch): the records
  // [head][partition] of kAttnRec floats, attn_parts partitions per head (2 .. kAttnXMaxParts); nullptr: x as given
  const float* attn_part = nullptr;
  int attn_parts = 0;
  // the MFMA GEMMs (M >= 2): project RMSNorm(x) * norm_w instead of x (lowbit_rmsnorm's arithmetic); nullptr: x
  const f16* norm_w = nullptr;
  float norm_eps = 0.f;
};

// RMSNorm statistics of rows 0 .. rows - 1 of x [M, K] (rows past M get 0) into rn[] (LDS): 1 / sqrt(mean(x^2) + eps),
// with lowbit_rmsnorm's arithmetic to the bit. That kernel's thread t (of 256) adds the squares of pieces t, t + 256,
// ... in order, each wave sums its threads with wave_sum and the four wave totals are added in wave order; here lane l
// keeps the sums of threads l, l + 64, l + 128, l + 192 apart (u = 0..3: pieces l + 64 u + 256 c, c = 0, 1, ...) and
// adds them the same way. Wave w takes rows 2w, 2w + 1, then 2w + 2W, ... (the loads of a pair of rows, 4 pieces each,
// requested before the first add; K <= 2048 is one batch). The caller synchronizes before reading rn.
__device__ __forceinline__ void rms_rows(__amdgpu_buffer_rsrc_t xr, int M, int K, int rows, float eps, int wave,
                                         int W, int lane, float* rn) {
  const int np = K >> 3;
  for (int m0 = 2 * wave; m0 < rows; m0 += 2 * W) {
    float ss[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    for (int p0 = lane; p0 < np; p0 += 64 * 4) {
      u32x4 v[2][4];
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int m = m0 + r, p = p0 + 64 * u;
          v[r][u] = buffer_load16(xr, m < M && p < np ? (m * K + 8 * p) * 2 : kOutOfRange);
        }
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int j = 0; j < 4; ++j) {                     // (a piece past the row adds exact zeros)
            const f16x2 h = as_f16x2(v[r][u][j]);
            ss[r][u] = fmaf((float)h[0], (float)h[0], ss[r][u]);
            ss[r][u] = fmaf((float)h[1], (float)h[1], ss[r][u]);
          }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      float s = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) s += wave_sum(ss[r][u]);
      const int m = m0 + r;
      if (lane == 0 && m < rows) rn[m] = m < M ? rsqrtf(s / (float)K + eps) : 0.f;
    }
  }
}

// the norm weights of 128-k chunks c0 .. c1 - 1 into LDS at g (16-byte pieces round robin over the workgroup)
__device__ __forceinline__ void stage_norm_weights(const f16* w, int c0, int c1, uint8_t* g) {
  const u32x4* src = reinterpret_cast<const u32x4*>(w) + 16 * c0;
  for (int p = threadIdx.x; p < 16 * (c1 - c0); p += blockDim.x) reinterpret_cast<u32x4*>(g)[p] = src[p];
}

// fp16 of an fp32 value that the compiler must hold in fp32 first: hipcc otherwise may fuse the product that made it
// and this conversion into one mixed-precision multiply-add (v_fma_mixlo_f16), rounding once instead of twice, which
// differs in rare cases (an fp32 product that lands on an fp16 rounding midpoint)
__device__ __forceinline__ f16 f16_of_f32(float a) {
  asm("" : "+v"(a));
  return (f16)a;
}

// eight values of a row normalized as torch's fp16 RMSNorm (transformers' Qwen2RMSNorm) writes them: fp16 of the
// fp32 product x r, then fp16 of w times that (exact in fp32, so one rounding). lowbit_rmsnorm, the GEMV's and the
// MFMA GEMMs' input norm all normalize with this function.
__device__ __forceinline__ u32x4 rms_apply8(const u32x4& v, const u32x4& g, float r) {
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const f16x2 p = as_f16x2(v[j]), w = as_f16x2(g[j]);
    const f16x2 n = {f16_of_f32((float)p[0] * r), f16_of_f32((float)p[1] * r)};
    o[j] = as_u32(f16x2{(f16)((float)w[0] * (float)n[0]), (f16)((float)w[1] * (float)n[1])});
  }
  return o;
}

// The bias or residual elements of outputs n .. n + 3 of row m (what epi_value reads), loaded ahead of the sums they
// are added to, so that their round trip overlaps the work before the store; zeros for the other modes and past N.
// One 8-byte load where n % 4 == 0 lines up (vec: N % 4 == 0) and aux is 8-byte aligned.
struct Aux4 {
  f16 v[4];
};
__device__ __forceinline__ Aux4 aux_load4(const Epilogue& e, int m, int n, int N, bool vec) {
  Aux4 a{};
  if (e.mode != kEpiBias && e.mode != kEpiResidual) return a;
  const f16* p = e.mode == kEpiBias ? e.aux + n : e.aux + (size_t)m * N + n;
  if (vec && (reinterpret_cast<uintptr_t>(e.aux) & 7) == 0) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    const f16x2 lo = as_f16x2(u.x), hi = as_f16x2(u.y);
    a.v[0] = lo[0];
    a.v[1] = lo[1];
    a.v[2] = hi[0];
    a.v[3] = hi[1];
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (n + j < N) a.v[j] = p[j];
  }
  return a;
}

// Four outputs of the kEpiRopeQKV epilogue, packed fp16, and where they go (dst == nullptr: nothing to store): dims
// d .. d + 3 of a head in `lo`, their partners d + 64 .. d + 67 in `hi`, stored 64 values on.
struct Out4 {
  f16* dst = nullptr;
  uint2 lo, hi;
};

// kEpiRopeQKV for token m of a multi-row step: rows n .. n + 3 of a 16-row tile of the RoPE-permuted q|k|v output
// (n % 4 == 0, n % 16 < 8) with their partners n + 8 .. n + 11, fp32 sums v1 and v2: + bias, RoPE at rope.pos[m] on
// q and k heads, q -> rope.q_out [M][Hq][128], k and v -> the caches' row pos[m] (none written outside 0..L-1). The
// four rows are dims d .. d + 3 (d % 4 == 0) of one head, so the bias, the (cos, sin) pairs and each output half move
// as one vector (the entry point checks the 8- and 16-byte alignments). cos and sin come from the step's table: the
// angle of (token, dim) is the same in every head and layer, and evaluating it here would leave 4 sin + cos per 16
// tokens to each lane of a tile at the kernel's end. The same roundings as the bias epilogue followed by
// lowbit_rope_kv on the permuted output.
__device__ __forceinline__ Out4 rope_qkv_out4(const Epilogue& e, int m, int n, const f32x4& v1, const f32x4& v2) {
  const RopeArgs& ra = e.rope;
  Out4 o;
  const int64_t p = ra.pos[m];
  if (p < 0 || p >= ra.L) return o;
  const int hh = n >> 7, pj = n & 127, d = 8 * (pj >> 4) + (pj & 7);
  const uint2 b1 = *reinterpret_cast<const uint2*>(e.aux + n), b2 = *reinterpret_cast<const uint2*>(e.aux + n + 8);
  const f16x2 b[4] = {as_f16x2(b1.x), as_f16x2(b1.y), as_f16x2(b2.x), as_f16x2(b2.y)};
  f16 x1[4], x2[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x1[i] = (f16)v1[i] + b[i >> 1][i & 1];
    x2[i] = (f16)v2[i] + b[2 + (i >> 1)][i & 1];
  }
  if (hh >= ra.Hq + ra.Hkv) {
    o.dst = ra.v_cache + ((size_t)(hh - ra.Hq - ra.Hkv) * ra.L + p) * 128 + d;
  } else {
    const u32x4 cs = *reinterpret_cast<const u32x4*>(ra.cos_sin + (size_t)m * 64 + d);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f16x2 c_s = as_f16x2(cs[i]);
      rope_rotate(x1[i], x2[i], c_s[0], c_s[1], x1[i], x2[i]);
    }
    o.dst = hh < ra.Hq ? ra.q_out + ((size_t)m * ra.Hq + hh) * 128 + d : ra.k_cache + ((size_t)(hh - ra.Hq) * ra.L + p) * 128 + d;
  }
  o.lo = make_uint2(as_u32(f16x2{x1[0], x1[1]}), as_u32(f16x2{x1[2], x1[3]}));
  o.hi = make_uint2(as_u32(f16x2{x2[0], x2[1]}), as_u32(f16x2{x2[2], x2[3]}));
  return o;
}

__device__ __forceinline__ void store_rope4(const Out4& o) {
  if (!o.dst) return;
  *reinterpret_cast<uint2*>(o.dst) = o.lo;
  *reinterpret_cast<uint2*>(o.dst + 64) = o.hi;
}

struct GemvArgs {
  const f16* x;
  const uint8_t* w;
  const f16* s;
  f16* y;
  int M, N, K, G;
  hipStream_t stream;
  Epilogue epi = {};
  const f16* norm_w = nullptr;   // M = 1 GEMV only: project RMSNorm(x) * norm_w instead of x
  float eps = 0.f;
};

struct GemvPlan {
  int R = 1;        // 16-row tiles per wave (MFMA layout) or rows per wave (row-major layouts)
  int waves = 1;    // waves per workgroup, splitting K
  int MT = 1;       // 16-column activation tiles (MFMA GEMM)
  int D = 4;        // chunk slots in flight per wave
  int S = 1;        // workgroups splitting K per row group (MFMA GEMM)
  int CS = 1;       // workgroups sharing a 16-row tile, 16 / CS rows each (MFMA-layout GEMV, R = 1)
  int TW = 0;       // MFMA GEMM: waves of the one-tile-per-workgroup kernel (0: the row-group kernel)
  int KW = 4;       // MFMA GEMM row groups: tile-waves per K-group (4, or 5, 6, 8 with one tile per wave)
  int LR = 0;       // M = 1 GEMV: weight ring slots per wave held in LDS (direct-to-LDS loads); 0 = ring in registers
  int XO = 0;       // MFMA GEMM with a K split: 0 row groups fastest in the workgroup order, 1 splits fastest
};

// launch shape of the prefill GEMM (M > 64)
struct PrefillPlan {
  int MT = 8;       // 16-row activation tiles per workgroup
  int D = 2;        // weight chunks in flight per wave
  int S = 1;        // workgroups splitting K per tile
  int MG = 1;       // activation-row groups
  int items = 1;    // workgroups: tiles x S
  int NW = 4;       // waves per workgroup, 16 PT weight rows each
  int XL = 1;       // chunks of x in flight
  int PT = 4;       // 16-row weight tiles per wave
};

// process-wide launch-shape override for tuning sweeps (lowbit_set_launch_override); 0 = automatic
struct GemvOverride {
  int waves = 0;
  int ring = 0;
  int splits = 0;
  int gemm_kernel = 0;  // MFMA GEMM structure: 0 automatic, 1 row groups (K split across workgroups), 2 one tile each
  int tile_waves = 0;   // MFMA GEMM row groups: tile-waves per K-group (0 automatic, 3, 4, 5, 6 or 8)
  int lds_ring = 0;     // M = 1 GEMV: 0 automatic, -1 ring in registers, 4 / 8 / 12 / 16 slots per wave in LDS
  int gemm_order = 0;   // MFMA GEMM with a K split: 0 automatic, 1 row groups fastest, 2 splits fastest
};
GemvOverride gemv_override();

// largest workgroup the M=1..8 MFMA-layout GEMV uses, from its register needs (x pairs, R weight pieces, D slots)
constexpr int gemv_max_threads(int M, int R, int D = 4) {
  return (M * R == 1 && D <= 4) ? 1024 : (M * R <= 4 ? 512 : 256);
}

constexpr size_t kGemvLdsX = 65536;      // x staged in LDS up to this many bytes (the default dynamic LDS limit)

// LDS of the M = 1 GEMV whose weight ring sits in LDS (GemvPlan::LR > 0): x [K] fp16 padded to 1 KB, its zero-weight
// sums [K / 32][2] fp32, the workgroup's scales [rows][K / G] fp16 padded to 1 KB, the norm weights [K] fp16 padded
// to 1 KB (fused RMSNorm only), then LR slots of 1 KB per wave. Every direct-to-LDS wave-load writes a whole 1 KB
// (lanes past the data read zeros), hence the padding.
struct GemvRingLds {
  uint32_t xs, s, g, ring, total;
};
__host__ __device__ constexpr uint32_t round_1k(uint32_t b) { return (b + 1023u) & ~1023u; }
__host__ __device__ constexpr GemvRingLds gemv_ring_lds(int K, int KG, int rows, int waves, int LR, bool norm) {
  GemvRingLds L{};
  L.xs = round_1k(2u * (uint32_t)K);
  L.s = L.xs + (uint32_t)(K / 32) * 8u;
  L.g = L.s + round_1k(2u * (uint32_t)(rows * KG));
  L.ring = L.g + (norm ? round_1k(2u * (uint32_t)K) : 0u);
  L.total = L.ring + (uint32_t)(waves * LR) * 1024u;
  return L;
}
constexpr size_t kLdsPerCu = 160 * 1024;  // gfx950

// MFMA GEMM launch shape: K splits across workgroups up to kGemmMaxGroups workgroups (at most kMaxSplits ways), then
// K-groups inside a workgroup up to kGemmTargetWaves waves. A workspace starts with kCounterBytes of arrival
// counters (zero before first use, left zero by every launch), followed by the fp32 partial sums [splits][M][N].
constexpr int kGemmMaxGroups = 256;
constexpr int kGemmTargetWaves = 1792;
constexpr int kGemmMaxWavesWide = 2048;
// prefill GEMM: K is split while the work items fill fewer than two rounds of this many workgroups
constexpr int kPrefillTargetGroups = 256;
// decode attention: when the cache holds at least kAttnMinSplitKeys keys, keys are split across blocks while
// (token, head group) blocks number fewer than kAttnTargetBlocks, down to kAttnMinKeys keys per block
constexpr int kAttnTargetBlocks = 256;
constexpr int kAttnMinKeys = 64;
constexpr int kAttnMinSplitKeys = 512;
constexpr int kAttnMaxParts = 16;
// key partitions hand their partial softmax sums over in records of kAttnRec floats: the max, the sum, two unused
// (the output then starts 16-byte aligned) and the unnormalized output of the head's kAttnHeadDim dims
constexpr int kAttnHeadDim = 128;
constexpr int kAttnRec = 4 + kAttnHeadDim;
// the one-row GEMV that merges an attention step's partials into its x holds at most this many partitions per head
constexpr int kAttnXMaxParts = 8;
// the attention workspace's fp32 partials start this many bytes in (the bytes before them are not used; they held
// arrival counters in an earlier version of the library, so callers size workspaces with them)
constexpr size_t kAttnCounterBytes = 4096;
// the MFMA attention takes steps with at least kAttnMfmaMinRows query rows (tokens x query heads per KV head), and
// splits keys while its waves number fewer than kAttnMfmaTargetWaves
constexpr int kAttnMfmaMinRows = 32;
constexpr int kAttnMfmaTargetWaves = 512;
constexpr int kAttnManyBlocks = 512;      // from this many blocks on, at most 4 waves per block
constexpr int kMaxSplits = 32;
constexpr size_t kCounterBytes = 16384;
// (column tiles, row tiles per wave, ring slots, K-groups, tile-waves per K-group) the MFMA GEMM is built for: what
// fits the register budget of TW KS waves per workgroup without spilling (hipcc -O3, gfx950: 128 registers at 16
// waves, 168 at 9-12, 256 at up to 8), and the LDS of the K-groups' x buffers. K-groups of 3, 5, 6 or 8 tile-waves
// are built with one tile per wave and 2 slots, at most 2 K-groups (4 of 3 tile-waves up to 32 rows).
constexpr bool gemm_fits(int MT, int RW, int D, int KS, int TW = 4) {
  if (TW == 3) return RW == 1 && D == 2 && (KS <= 2 || MT <= 2);
  if (TW != 4) return RW == 1 && (D == 2 || (D == 3 && (TW == 5 || TW == 6))) && KS <= 2 && (TW * KS <= 12 || MT <= 3);
  if (KS == 4) return D == 2 ? (RW == 1 ? MT <= 3 : MT <= 2) : (RW == 1 && MT == 1);
  if (KS == 2) return !((RW == 2 && (MT >= 3 ? D >= 3 : (MT == 2 && D == 4))) || (MT == 4 && RW == 1 && D == 4));
  return true;
}
constexpr int kMaxGroups = 2048;         // K / G limit of the MFMA-layout GEMV (scales staged in LDS)
constexpr int64_t kMaxK = 1 << 22;       // K limit of the MFMA-layout kernels (32-bit buffer offsets)

constexpr int kMaxClip = 64;
struct ClipGrid {
  int n;                 // 0: plain absmax
  float a[kMaxClip];
};

GemvPlan plan_gemv_mfma_layout(int M, int N, int K, int rows_per_wave, bool row_split_ok = true,
                               bool lds_ring_ok = true);
GemvPlan plan_gemm_mfma(int M, int N, int K, int row_tiles, size_t workspace_bytes);
int pick_rows_rowmajor(int N, int M);

hipError_t gemv_mfma_layout_launch(const GemvArgs& a, int rows_per_wave);
hipError_t gemv_rowmajor_launch(const GemvArgs& a, int rows_per_wave, bool v3);
// the M = 1 GEMV over an fp16 weight [N, K] (a.w, row-major; a.s unused), with the same epilogues and norm
hipError_t gemv_f16w_launch(const GemvArgs& a);
hipError_t gemm_mfma_launch(const GemvArgs& a, int row_tiles, void* workspace, size_t workspace_bytes);
hipError_t zero_words_launch(void* p, int n, hipStream_t stream);
// prefill variants that compile without register spills (hipcc -O3, gfx950): an 8-wave workgroup has 256 registers
// per wave, enough for 4 activation tiles and a 2-deep weight ring only
constexpr bool prefill_fits(int MT, int D, int NW, int XL) {
  return (D == 2 || XL == 1) && (NW == 4 || (MT == 4 && D == 2));
}
PrefillPlan plan_gemm_prefill(int M, int N, int K, size_t workspace_bytes);
hipError_t gemm_prefill_launch(const GemvArgs& a, void* workspace, size_t workspace_bytes);
hipError_t rmsnorm_launch(const f16* x, const f16* w, f16* out, int M, int H, float eps, hipStream_t st);
hipError_t rope_table_launch(const int64_t* pos, const float* inv_freq, uint32_t* table, int M, hipStream_t st);
hipError_t rope_kv_launch(const f16* qkv, const int64_t* pos, const float* inv_freq, f16* q_out, f16* k_cache,
                          f16* v_cache, int M, int Hq, int Hkv, int L, bool permuted, hipStream_t st);
hipError_t gemv_f16_launch(const f16* x, const f16* w, f16* y, int M, int N, int K, hipStream_t st);
int head_pick_parts(int N);                                  // 64-bit keys head_pick_launch keeps in its workspace
hipError_t head_pick_launch(const f16* x, const f16* w, f16* y, int N, int K, uint64_t* pick, int64_t* tokens,
                            int64_t* positions, int64_t* out, int out_cap, int* out_count, const f16* embed, f16* h_out,
                            hipStream_t st);
hipError_t hbm_read_launch(const void* src, size_t bytes, uint32_t* sink, int blocks, hipStream_t stream);
hipError_t hbm_copy_launch(const void* src, void* dst, size_t bytes, int blocks, hipStream_t stream);
hipError_t attention_launch(const f16* q, const f16* k, const f16* v, const int64_t* pos, f16* out, int M, int Hq,
                            int Hkv, int L, int max_keys, float scale, void* ws, size_t ws_bytes, hipStream_t st);
// one token's attention without the merge of its key partitions: their records (kAttnRec floats, [head][partition])
// start kAttnCounterBytes into ws and their count goes to *parts (<= kAttnXMaxParts); with one partition out is
// written instead and *parts is 1
hipError_t attention_partials_launch(const f16* q, const f16* k, const f16* v, const int64_t* pos, f16* out, int Hq,
                                     int Hkv, int L, int max_keys, float scale, void* ws, size_t ws_bytes, int* parts,
                                     hipStream_t st);
hipError_t dequant_launch(const uint8_t* w, const f16* s, f16* out, int N, int K, int G, bool mfma, hipStream_t st);
hipError_t relayout_launch(const uint8_t* src, uint8_t* dst, int N, int K, bool mfma, hipStream_t st);
hipError_t quantize_launch(const void* w, int dtype, uint8_t* packed, f16* scales, int N, int K, int G,
                           const ClipGrid& grid, hipStream_t st);

}  // namespace lowbit
