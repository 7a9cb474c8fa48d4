// Internal interface between the C ABI (capi.hip) and the kernel files. Callers validate every argument first.
#pragma once
#include "common.hpp"

namespace lowbit {

struct GemvArgs {
  const f16* x;
  const uint8_t* w;
  const f16* s;
  f16* y;
  int M, N, K, G;
  hipStream_t stream;
};

struct GemvPlan {
  int R = 1;        // 16-row tiles per wave (MFMA layout) or rows per wave (row-major layouts)
  int waves = 1;    // waves per workgroup, splitting K
  int MT = 1;       // 16-column activation tiles (MFMA GEMM)
  int D = 4;        // chunk slots in flight per wave (M <= 8 GEMV)
};

// process-wide launch-shape override for tuning sweeps (lowbit_set_launch_override); 0 = automatic
struct GemvOverride {
  int waves = 0;
  int ring = 0;
};
GemvOverride gemv_override();

// largest workgroup the M=1..8 MFMA-layout GEMV uses, from its register needs (x pairs, R weight pieces, D slots)
constexpr int gemv_max_threads(int M, int R, int D = 4) {
  return (M * R == 1 && D <= 4) ? 1024 : (M * R <= 4 ? 512 : 256);
}

constexpr size_t kGemvLdsX = 65536;      // x staged in LDS up to this many bytes (the default dynamic LDS limit)

constexpr int kMaxClip = 64;
struct ClipGrid {
  int n;                 // 0: plain absmax
  float a[kMaxClip];
};

GemvPlan plan_gemv_mfma_layout(int M, int N, int K, int rows_per_wave);
GemvPlan plan_gemm_mfma(int M, int N, int K, int row_tiles);
int pick_rows_rowmajor(int N, int M);

hipError_t gemv_mfma_layout_launch(const GemvArgs& a, int rows_per_wave);
hipError_t gemv_rowmajor_launch(const GemvArgs& a, int rows_per_wave, bool v3);
hipError_t gemm_mfma_launch(const GemvArgs& a, int row_tiles);
hipError_t dequant_launch(const uint8_t* w, const f16* s, f16* out, int N, int K, int G, bool mfma, hipStream_t st);
hipError_t relayout_launch(const uint8_t* src, uint8_t* dst, int N, int K, bool mfma, hipStream_t st);
hipError_t quantize_launch(const void* w, int dtype, uint8_t* packed, f16* scales, int N, int K, int G,
                           const ClipGrid& grid, hipStream_t st);

}  // namespace lowbit
