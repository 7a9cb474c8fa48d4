// The C ABI (include/lowbit_w4.h): argument validation with the reference's messages, then dispatch to the kernels.
// The validation mirrors the reference's check() / TORCH_CHECKs (csrc/w4_gemv.cu:312-325,454-540); checks that need
// tensor metadata (device, dtype, contiguity, dims) are done by the Python layer, which owns the tensors.
#include <atomic>
#include <climits>
#include <cstring>
#include <mutex>

#include "kernels.hpp"
#include "lowbit_w4.h"
#include "status.hpp"

namespace lowbit {

namespace {

constexpr int kMaxDevices = 64;
int g_arch_ok[kMaxDevices];     // 0 unknown, 1 gfx950, -1 other (benign race: every writer stores the same value)

int check_device() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(LOWBIT_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return LOWBIT_OK;
  if (g_arch_ok[dev] == 0) {
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return fail(LOWBIT_ERR_HIP, "hipGetDeviceProperties failed: %s", hipGetErrorString(e));
    g_arch_ok[dev] = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -1;
    if (g_arch_ok[dev] < 0)
      return fail(LOWBIT_ERR_DEVICE, "liblowbit_w4 is built for gfx950 only; device %d is %s", dev, prop.gcnArchName);
  }
  if (g_arch_ok[dev] < 0) return fail(LOWBIT_ERR_DEVICE, "liblowbit_w4 is built for gfx950 only (device %d)", dev);
  return LOWBIT_OK;
}

std::atomic<int> g_override_waves{0}, g_override_ring{0}, g_override_splits{0}, g_override_gemm{0},
    g_override_tile_waves{0}, g_override_lds_ring{0}, g_override_gemm_order{0};

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(LOWBIT_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool fits_int(int64_t v) { return v >= 0 && v <= INT_MAX; }

// the reference's check() (csrc/w4_gemv.cu:312-325), minus the tensor-metadata part
int check_common(const void* x, const void* w, const void* s, const void* y, int64_t M, int64_t N, int64_t K,
                 int64_t group) {
  if (!x || !w || !s || !y) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (group <= 0) return fail(LOWBIT_ERR_GROUP, "group size must be positive");
  if (group % 32 || K % group || K <= 0)
    return fail(LOWBIT_ERR_GROUP, "K must be a multiple of the group size, itself a multiple of 32");
  if (N < 1 || !fits_int(N) || !fits_int(K) || !fits_int(M))
    return fail(LOWBIT_ERR_SHAPE, "shape mismatch");
  if (!aligned16(x) || !aligned16(w)) return fail(LOWBIT_ERR_ALIGN, "x and w must be 16-byte aligned for the 128-bit loads");
  return LOWBIT_OK;
}

// 32-bit buffer offsets bound K and the scale count for the MFMA-layout kernels; the GEMV also stages the scales of
// its tiles in LDS (16 rows x K / G fp16 per tile, gemv_tiles tiles per wave; 0 = not the GEMV), which bounds K / G
int check_mfma_layout_limits(int64_t N, int64_t K, int64_t group, int gemv_tiles) {
  if (K > kMaxK) return fail(LOWBIT_ERR_SHAPE, "K is at most %lld for the MFMA-layout kernels", (long long)kMaxK);
  if (gemv_tiles > 0 && (int64_t)16 * gemv_tiles * (K / group) * 2 > (int64_t)kGemvLdsX)
    return fail(LOWBIT_ERR_GROUP, "K / group is at most %d for the v6 GEMV with %d tile(s) per wave",
                kMaxGroups / gemv_tiles, gemv_tiles);
  if (N * (K / group) * 2 > INT_MAX) return fail(LOWBIT_ERR_SHAPE, "N * K / group scales exceed 2^30");
  return LOWBIT_OK;
}

int gemv_impl(const void* x, const void* w, const void* s, void* y, int64_t M, int64_t N, int64_t K, int64_t group,
              int version, int rows_per_wave, void* stream) {
  if (int rc = check_common(x, w, s, y, M, N, K, group)) return rc;
  if (M < 1 || M > 8)
    return fail(LOWBIT_ERR_ROWS, "the GEMV kernels take 1..8 rows; use the dequantize + matmul path above that");
  if (!((version >= 1 && version <= 4) || version == 6)) return fail(LOWBIT_ERR_VERSION, "version is 1..4 or 6");
  if (version == 6 && (K % 128 || group % 128))
    return fail(LOWBIT_ERR_LAYOUT, "v6 needs K and the group size to be multiples of 128");
  if (!(rows_per_wave == 0 || rows_per_wave == 1 || rows_per_wave == 2 || rows_per_wave == 4))
    return fail(LOWBIT_ERR_TUNING, "rows_per_warp is 0 (auto), 1, 2 or 4");
  if (version == 6)
    if (int rc = check_mfma_layout_limits(N, K, group, rows_per_wave ? rows_per_wave : 1)) return rc;
  if (int rc = check_device()) return rc;
  GemvArgs a{static_cast<const f16*>(x), static_cast<const uint8_t*>(w), static_cast<const f16*>(s), static_cast<f16*>(y),
             (int)M, (int)N, (int)K, (int)group, static_cast<hipStream_t>(stream)};
  hipError_t e = version == 6 ? gemv_mfma_layout_launch(a, rows_per_wave)
                              : gemv_rowmajor_launch(a, rows_per_wave, version >= 3);
  return hip_status(e, "w4_gemv");
}

int check_gemm(const void* x, const void* w, const void* s, const void* y, int64_t M, int64_t N, int64_t K,
               int64_t group, int row_tiles) {
  if (int rc = check_common(x, w, s, y, M, N, K, group)) return rc;
  if (M < 1 || M > 64) return fail(LOWBIT_ERR_ROWS, "the MFMA kernel takes 1..64 rows");
  if (K % 128 || group % 128) return fail(LOWBIT_ERR_LAYOUT, "v5 needs K and the group size to be multiples of 128");
  if (int rc = check_mfma_layout_limits(N, K, group, 0)) return rc;
  if (!(row_tiles == 0 || row_tiles == 1 || row_tiles == 2 || row_tiles == 4))
    return fail(LOWBIT_ERR_TUNING, "row_tiles must be 1, 2 or 4");
  return LOWBIT_OK;
}

int gemm_impl(const void* x, const void* w, const void* s, void* y, int64_t M, int64_t N, int64_t K, int64_t group,
              int row_tiles, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_gemm(x, w, s, y, M, N, K, group, row_tiles)) return rc;
  if (workspace && (!aligned16(workspace) || workspace_bytes < kCounterBytes))
    return fail(LOWBIT_ERR_ARG, "the workspace must be 16-byte aligned and hold at least %zu bytes", kCounterBytes);
  if (int rc = check_device()) return rc;
  GemvArgs a{static_cast<const f16*>(x), static_cast<const uint8_t*>(w), static_cast<const f16*>(s), static_cast<f16*>(y),
             (int)M, (int)N, (int)K, (int)group, static_cast<hipStream_t>(stream)};
  return hip_status(gemm_mfma_launch(a, row_tiles, workspace, workspace_bytes), "w4_gemm_mfma");
}

}  // namespace

GemvOverride gemv_override() {
  GemvOverride o;
  o.waves = g_override_waves.load(std::memory_order_relaxed);
  o.ring = g_override_ring.load(std::memory_order_relaxed);
  o.splits = g_override_splits.load(std::memory_order_relaxed);
  o.gemm_kernel = g_override_gemm.load(std::memory_order_relaxed);
  o.tile_waves = g_override_tile_waves.load(std::memory_order_relaxed);
  o.lds_ring = g_override_lds_ring.load(std::memory_order_relaxed);
  o.gemm_order = g_override_gemm_order.load(std::memory_order_relaxed);
  return o;
}

}  // namespace lowbit

// ---- the allocation-free MFMA GEMM (lowbit_w4_gemm_mfma_noalloc) ----
// Its split-K workspace (arrival counters, then fp32 partial sums) is this file-scope device array, the same size as
// the workspace the Python binding gives lowbit_w4_gemm_mfma, so both entry points plan every shape alike. Each GPU
// the library runs on holds one copy until the process ends. In host code `scratch` names a host-side stand-in, not
// the device memory: only the address hipGetSymbolAddress returns for the current device is passed to kernels.
static __device__ __align__(256) uint8_t scratch[LOWBIT_NOALLOC_SCRATCH_BYTES];

namespace lowbit {
namespace {

struct ScratchSlot {
  std::atomic<void*> ptr{nullptr};        // this device's copy of `scratch`
  std::atomic<bool> cleared{false};       // counters cleared by an executed (not captured) kernel
};
ScratchSlot g_scratch[kMaxDevices];
std::mutex g_scratch_mutex;

// The current device's scratch address, looked up once per device with that device current. Its arrival counters
// must start at zero (every GEMM leaves them zero again): until a clear has run outside graph capture, each call
// first clears them on its own stream with a kernel (a captured clear is part of its graph and runs before the GEMM
// on every replay, but does not clear the counters for eager calls).
int scratch_for_current_device(hipStream_t stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(LOWBIT_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(LOWBIT_ERR_DEVICE, "device index %d is beyond %d", dev, kMaxDevices);
  ScratchSlot& slot = g_scratch[dev];
  void* p = slot.ptr.load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = slot.ptr.load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p)
        return fail(LOWBIT_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
      slot.ptr.store(p, std::memory_order_release);
    }
  }
  if (!slot.cleared.load(std::memory_order_acquire)) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &status);
    if (e != hipSuccess) return fail(LOWBIT_ERR_HIP, "hipStreamIsCapturing failed: %s", hipGetErrorString(e));
    e = zero_words_launch(p, (int)(kCounterBytes / 4), stream);
    if (e != hipSuccess) return fail(LOWBIT_ERR_HIP, "clearing the scratch counters failed: %s", hipGetErrorString(e));
    if (status == hipStreamCaptureStatusNone) slot.cleared.store(true, std::memory_order_release);
  }
  *out = p;
  return LOWBIT_OK;
}

}  // namespace
}  // namespace lowbit

using namespace lowbit;

extern "C" {

const char* lowbit_version(void) { return "lowbit_w4 0.3 gfx950"; }

int lowbit_set_launch_override(int waves_per_group, int ring, int k_splits) {
  if (!(waves_per_group == 0 || waves_per_group == 1 || waves_per_group == 2 || waves_per_group == 4 ||
        waves_per_group == 8 || waves_per_group == 16))
    return fail(LOWBIT_ERR_TUNING, "waves_per_group is 0 (auto), 1, 2, 4, 8 or 16");
  if (!(ring == 0 || ring == 2 || ring == 3 || ring == 4 || ring == 8))
    return fail(LOWBIT_ERR_TUNING, "ring is 0 (auto), 2, 3, 4 or 8");
  if (k_splits < 0 || k_splits > kMaxSplits) return fail(LOWBIT_ERR_TUNING, "k_splits is 0 (auto) .. %d", kMaxSplits);
  g_override_waves.store(waves_per_group, std::memory_order_relaxed);
  g_override_ring.store(ring, std::memory_order_relaxed);
  g_override_splits.store(k_splits, std::memory_order_relaxed);
  return ok();
}

int lowbit_set_gemv_lds_ring(int slots) {
  if (!(slots == 0 || slots == -1 || slots == 4 || slots == 8 || slots == 12 || slots == 16))
    return fail(LOWBIT_ERR_TUNING, "slots is 0 (auto), -1 (ring in registers), 4, 8, 12 or 16");
  g_override_lds_ring.store(slots, std::memory_order_relaxed);
  return ok();
}

int lowbit_set_gemm_order(int order) {
  if (order < 0 || order > 2) return fail(LOWBIT_ERR_TUNING, "order is 0 (auto), 1 (row groups fastest) or 2 (splits fastest)");
  g_override_gemm_order.store(order, std::memory_order_relaxed);
  return ok();
}

int lowbit_set_gemm_kernel(int kernel) {
  if (kernel < 0 || kernel > 2) return fail(LOWBIT_ERR_TUNING, "kernel is 0 (auto), 1 (row groups) or 2 (one tile each)");
  g_override_gemm.store(kernel, std::memory_order_relaxed);
  return ok();
}

int lowbit_set_gemm_tile_waves(int tile_waves) {
  if (!(tile_waves == 0 || tile_waves == 3 || tile_waves == 4 || tile_waves == 5 || tile_waves == 6 || tile_waves == 8))
    return fail(LOWBIT_ERR_TUNING, "tile_waves is 0 (auto), 3, 4, 5, 6 or 8");
  g_override_tile_waves.store(tile_waves, std::memory_order_relaxed);
  return ok();
}

int lowbit_w4_gemv(const void* x, const void* w, const void* s, void* y, int64_t M, int64_t N, int64_t K, int64_t group,
                   int version, int rows_per_wave, void* stream) {
  return gemv_impl(x, w, s, y, M, N, K, group, version, rows_per_wave, stream);
}

int lowbit_w4_gemm_mfma(const void* x, const void* w, const void* s, void* y, int64_t M, int64_t N, int64_t K,
                        int64_t group, int row_tiles, void* workspace, size_t workspace_bytes, void* stream) {
  return gemm_impl(x, w, s, y, M, N, K, group, row_tiles, workspace, workspace_bytes, stream);
}

int lowbit_w4_gemm_mfma_noalloc(const void* x, const void* w, const void* s, void* y, int64_t M, int64_t N, int64_t K,
                                int64_t group, int row_tiles, void* stream) {
  if (int rc = check_gemm(x, w, s, y, M, N, K, group, row_tiles)) return rc;
  if (int rc = check_device()) return rc;
  constexpr size_t kScratch = LOWBIT_NOALLOC_SCRATCH_BYTES;
  // the planner lowers the K split to what the scratch holds; refuse a plan that would not fit it all the same
  const GemvPlan plan = plan_gemm_mfma((int)M, (int)N, (int)K, row_tiles, kScratch);
  // row groups of plan.KW tile-waves x plan.R tiles (one arrival counter each when K is split)
  const int ntiles = ((int)N + 15) / 16, groups = (ntiles + plan.KW * plan.R - 1) / (plan.KW * plan.R);
  if (plan.S > 1 && ((size_t)plan.S * M * N * sizeof(float) > kScratch - kCounterBytes ||
                     (size_t)groups * sizeof(uint32_t) > kCounterBytes))
    return fail(LOWBIT_ERR_SHAPE, "w4_gemm_mfma_noalloc: %d-way split partials of M=%lld x N=%lld exceed the %zu-byte scratch",
                plan.S, (long long)M, (long long)N, kScratch);
  void* ws = nullptr;
  if (int rc = scratch_for_current_device(static_cast<hipStream_t>(stream), &ws)) return rc;
  GemvArgs a{static_cast<const f16*>(x), static_cast<const uint8_t*>(w), static_cast<const f16*>(s), static_cast<f16*>(y),
             (int)M, (int)N, (int)K, (int)group, static_cast<hipStream_t>(stream)};
  return hip_status(gemm_mfma_launch(a, row_tiles, ws, kScratch), "w4_gemm_mfma_noalloc");
}

int lowbit_w4_dequant(const void* w, const void* s, void* out, int64_t N, int64_t K, int64_t group, int mfma_layout,
                      void* stream) {
  if (!w || !s || !out) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (group <= 0) return fail(LOWBIT_ERR_GROUP, "w [N,K/2], scales [N,K/G], positive group size");
  if (group % 32 || K % group || K <= 0 || N < 1 || !fits_int(N) || !fits_int(K))
    return fail(LOWBIT_ERR_SHAPE, "shape mismatch");
  if (!aligned16(w)) return fail(LOWBIT_ERR_ALIGN, "packed weights must be contiguous and 16-byte aligned");
  if (!aligned16(out)) return fail(LOWBIT_ERR_ALIGN, "the output must be 16-byte aligned");
  if (mfma_layout && (K % 128 || group % 128))
    return fail(LOWBIT_ERR_LAYOUT, "the v5 layout needs K and group % 128 == 0");
  if (N * (K / 8) >= (int64_t{1} << 32) - 1024) return fail(LOWBIT_ERR_SHAPE, "dequant takes N * K < 2^35");
  if (int rc = check_device()) return rc;
  return hip_status(dequant_launch(static_cast<const uint8_t*>(w), static_cast<const f16*>(s), static_cast<f16*>(out),
                                   (int)N, (int)K, (int)group, mfma_layout != 0, static_cast<hipStream_t>(stream)),
                    "w4_dequant");
}

int lowbit_w4_quantize(const void* w, int w_dtype, void* packed, void* scales, int64_t N, int64_t K, int64_t group,
                       const float* clip_grid, int n_clip, void* stream) {
  if (!w || !packed || !scales) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (w_dtype < LOWBIT_DTYPE_F32 || w_dtype > LOWBIT_DTYPE_BF16) return fail(LOWBIT_ERR_ARG, "unknown weight dtype");
  if (group <= 0 || group % 32 || K <= 0 || K % group)
    return fail(LOWBIT_ERR_GROUP, "K=%lld must be a multiple of the group size %lld, itself a multiple of 32",
                (long long)K, (long long)group);
  if (group > 1024) return fail(LOWBIT_ERR_GROUP, "the GPU quantizer takes group sizes up to 1024");
  if (N < 1 || !fits_int(N) || !fits_int(K)) return fail(LOWBIT_ERR_SHAPE, "shape mismatch");
  if (n_clip < 0 || n_clip > kMaxClip || (n_clip > 0 && !clip_grid))
    return fail(LOWBIT_ERR_ARG, "clip grid must hold 0..%d values", kMaxClip);
  if (int rc = check_device()) return rc;
  ClipGrid grid;
  std::memset(&grid, 0, sizeof(grid));
  grid.n = n_clip;
  for (int i = 0; i < n_clip; ++i) grid.a[i] = clip_grid[i];
  return hip_status(quantize_launch(w, w_dtype, static_cast<uint8_t*>(packed), static_cast<f16*>(scales), (int)N, (int)K,
                                    (int)group, grid, static_cast<hipStream_t>(stream)),
                    "w4_quantize");
}

int lowbit_w4_relayout(const void* src, void* dst, int64_t N, int64_t K, int layout, void* stream) {
  if (!src || !dst) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (src == dst) return fail(LOWBIT_ERR_ARG, "dst must not alias src");
  if (layout != LOWBIT_LAYOUT_V3 && layout != LOWBIT_LAYOUT_MFMA)
    return fail(LOWBIT_ERR_ARG, "device relayout targets the v3 or the MFMA layout");
  if (N < 1 || K <= 0 || K % 32 || !fits_int(N) || !fits_int(K)) return fail(LOWBIT_ERR_SHAPE, "shape mismatch");
  if (layout == LOWBIT_LAYOUT_MFMA && K % 128)
    return fail(LOWBIT_ERR_LAYOUT, "the MFMA layout needs K to be a multiple of 128");
  if (!aligned16(src) || !aligned16(dst)) return fail(LOWBIT_ERR_ALIGN, "packed weights must be 16-byte aligned");
  if (int rc = check_device()) return rc;
  return hip_status(relayout_launch(static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), (int)N, (int)K,
                                    layout == LOWBIT_LAYOUT_MFMA, static_cast<hipStream_t>(stream)),
                    "w4_relayout");
}

int lowbit_w4_linear_fused(const void* x, const void* w, const void* s, void* y, int64_t M, int64_t N, int64_t K,
                           int64_t group, int epilogue, const void* aux, const void* norm_weight, float eps,
                           void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_common(x, w, s, y, M, N, K, group)) return rc;
  if (M < 1 || M > 64) return fail(LOWBIT_ERR_ROWS, "the fused projection takes 1..64 rows");
  if (K % 128 || group % 128) return fail(LOWBIT_ERR_LAYOUT, "the MFMA layout needs K and the group size to be multiples of 128");
  if (int rc = check_mfma_layout_limits(N, K, group, M == 1 ? 1 : 0)) return rc;
  if (epilogue < LOWBIT_EPI_STORE || epilogue > LOWBIT_EPI_SILU_MUL) return fail(LOWBIT_ERR_ARG, "unknown epilogue");
  if ((epilogue == LOWBIT_EPI_BIAS || epilogue == LOWBIT_EPI_RESIDUAL) && !aux)
    return fail(LOWBIT_ERR_ARG, "the bias and residual epilogues need aux");
  if (epilogue == LOWBIT_EPI_SILU_MUL && (N % 16 || (reinterpret_cast<uintptr_t>(y) & 7)))
    return fail(LOWBIT_ERR_SHAPE, "silu-mul needs N (gate and up rows) a multiple of 16 and an 8-byte aligned y");
  if (workspace && (!aligned16(workspace) || workspace_bytes < kCounterBytes))
    return fail(LOWBIT_ERR_ARG, "the workspace must be 16-byte aligned and hold at least %zu bytes", kCounterBytes);
  if (norm_weight && (K > (M == 1 ? 16384 : 8192) || !aligned16(norm_weight)))
    return fail(LOWBIT_ERR_ARG, "the fused input norm takes K <= 16384 (one row) or K <= 8192 (2..64 rows) and a 16-byte "
                                "aligned weight");
  if (int rc = check_device()) return rc;
  GemvArgs a{static_cast<const f16*>(x), static_cast<const uint8_t*>(w), static_cast<const f16*>(s), static_cast<f16*>(y),
             (int)M, (int)N, (int)K, (int)group, static_cast<hipStream_t>(stream)};
  a.epi.mode = epilogue;
  a.epi.aux = static_cast<const f16*>(aux);
  a.norm_w = static_cast<const f16*>(norm_weight);
  a.eps = eps;
  return hip_status(M == 1 ? gemv_mfma_layout_launch(a, 0) : gemm_mfma_launch(a, 0, workspace, workspace_bytes),
                    "w4_linear_fused");
}

int lowbit_w4_gemm_prefill(const void* x, const void* w, const void* s, void* y, int64_t M, int64_t N, int64_t K,
                           int64_t group, int epilogue, const void* aux, void* workspace, size_t workspace_bytes,
                           void* stream) {
  if (int rc = check_common(x, w, s, y, M, N, K, group)) return rc;
  if (M < 1) return fail(LOWBIT_ERR_ROWS, "the prefill GEMM takes at least one row");
  if (K % 128 || group % 128) return fail(LOWBIT_ERR_LAYOUT, "the MFMA layout needs K and the group size to be multiples of 128");
  if (int rc = check_mfma_layout_limits(N, K, group, 0)) return rc;
  if ((M + 128) * K * 2 > INT_MAX) return fail(LOWBIT_ERR_SHAPE, "the prefill GEMM takes (M + 128) * K * 2 < 2^31");
  if (epilogue < LOWBIT_EPI_STORE || epilogue > LOWBIT_EPI_SILU_MUL) return fail(LOWBIT_ERR_ARG, "unknown epilogue");
  if ((epilogue == LOWBIT_EPI_BIAS || epilogue == LOWBIT_EPI_RESIDUAL) && !aux)
    return fail(LOWBIT_ERR_ARG, "the bias and residual epilogues need aux");
  if (epilogue == LOWBIT_EPI_SILU_MUL && (N % 16 || (reinterpret_cast<uintptr_t>(y) & 7)))
    return fail(LOWBIT_ERR_SHAPE, "silu-mul needs N (gate and up rows) a multiple of 16 and an 8-byte aligned y");
  if (workspace && (!aligned16(workspace) || workspace_bytes < kCounterBytes))
    return fail(LOWBIT_ERR_ARG, "the workspace must be 16-byte aligned and hold at least %zu bytes", kCounterBytes);
  if (int rc = check_device()) return rc;
  GemvArgs a{static_cast<const f16*>(x), static_cast<const uint8_t*>(w), static_cast<const f16*>(s), static_cast<f16*>(y),
             (int)M, (int)N, (int)K, (int)group, static_cast<hipStream_t>(stream)};
  a.epi.mode = epilogue;
  a.epi.aux = static_cast<const f16*>(aux);
  return hip_status(gemm_prefill_launch(a, workspace, workspace_bytes), "w4_gemm_prefill");
}

int lowbit_rmsnorm(const void* x, const void* weight, void* out, int64_t M, int64_t H, float eps, void* stream) {
  if (!x || !weight || !out) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (M < 1 || H < 8 || H % 8 || !fits_int(M) || H > 65536) return fail(LOWBIT_ERR_SHAPE, "rmsnorm takes H % 8 == 0, H <= 65536");
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out)) return fail(LOWBIT_ERR_ALIGN, "rmsnorm needs 16-byte aligned rows");
  if (int rc = check_device()) return rc;
  return hip_status(rmsnorm_launch(static_cast<const f16*>(x), static_cast<const f16*>(weight), static_cast<f16*>(out),
                                   (int)M, (int)H, eps, static_cast<hipStream_t>(stream)),
                    "rmsnorm");
}

int lowbit_rope_kv(const void* qkv, const int64_t* positions, const float* inv_freq, void* q_out, void* k_cache,
                   void* v_cache, int64_t M, int64_t Hq, int64_t Hkv, int64_t L, int permuted, void* stream) {
  if (!qkv || !positions || !inv_freq || !q_out || !k_cache || !v_cache) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (M < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || L < 1 || !fits_int(M * (Hq + 2 * Hkv) * 64) || !fits_int(L * 128 * Hkv))
    return fail(LOWBIT_ERR_SHAPE, "rope_kv: M, Hq, Hkv (dividing Hq), L must be positive");
  if (int rc = check_device()) return rc;
  return hip_status(rope_kv_launch(static_cast<const f16*>(qkv), positions, inv_freq, static_cast<f16*>(q_out),
                                   static_cast<f16*>(k_cache), static_cast<f16*>(v_cache), (int)M, (int)Hq, (int)Hkv,
                                   (int)L, permuted != 0, static_cast<hipStream_t>(stream)),
                    "rope_kv");
}

int lowbit_w4_qkv_rope(const void* x, const void* w, const void* s, int64_t N, int64_t K, int64_t group,
                       const void* bias, const void* norm_weight, float eps, const int64_t* positions,
                       const float* inv_freq, void* q_out, void* k_cache, void* v_cache, int64_t Hq, int64_t Hkv,
                       int64_t L, void* stream) {
  if (int rc = check_common(x, w, s, q_out, 1, N, K, group)) return rc;
  if (!bias || !positions || !inv_freq || !k_cache || !v_cache) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (Hq < 1 || Hkv < 1 || Hq % Hkv || L < 1 || N != (Hq + 2 * Hkv) * 128 || !fits_int(L * 128 * Hkv))
    return fail(LOWBIT_ERR_SHAPE, "qkv_rope: N must be (Hq + 2 Hkv) * 128 with Hkv dividing Hq, L positive");
  if (K % 128 || group % 128) return fail(LOWBIT_ERR_LAYOUT, "the MFMA layout needs K and the group size to be multiples of 128");
  if (int rc = check_mfma_layout_limits(N, K, group, 1)) return rc;
  if (norm_weight && (K > 16384 || !aligned16(norm_weight)))
    return fail(LOWBIT_ERR_ARG, "the fused input norm takes K <= 16384 and a 16-byte aligned weight");
  if (int rc = check_device()) return rc;
  GemvArgs a{static_cast<const f16*>(x), static_cast<const uint8_t*>(w), static_cast<const f16*>(s), static_cast<f16*>(q_out),
             1, (int)N, (int)K, (int)group, static_cast<hipStream_t>(stream)};
  a.epi.mode = kEpiRopeQKV;
  a.epi.aux = static_cast<const f16*>(bias);
  a.epi.rope = RopeArgs{positions, inv_freq, nullptr, static_cast<f16*>(q_out), static_cast<f16*>(k_cache),
                        static_cast<f16*>(v_cache), (int)Hq, (int)Hkv, (int)L};
  a.norm_w = static_cast<const f16*>(norm_weight);
  a.eps = eps;
  return hip_status(gemv_mfma_layout_launch(a, 0), "w4_qkv_rope");
}

// the fp16-weight GEMV (the W4A16 decode's comparator): one row, K % 128 == 0, x and its norm staged in LDS
int check_f16_fused(const void* x, const void* w, const void* y, int64_t N, int64_t K, const void* norm_weight) {
  if (!x || !w || !y) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (N < 1 || !fits_int(N) || K < 128 || K % 128 || K > 16384)
    return fail(LOWBIT_ERR_SHAPE, "the fp16 fused GEMV takes K a multiple of 128, at most 16384");
  if (!aligned16(x) || !aligned16(w)) return fail(LOWBIT_ERR_ALIGN, "x and w must be 16-byte aligned");
  if (norm_weight && !aligned16(norm_weight)) return fail(LOWBIT_ERR_ALIGN, "the norm weight must be 16-byte aligned");
  return LOWBIT_OK;
}

int lowbit_f16_linear_fused(const void* x, const void* w, void* y, int64_t N, int64_t K, int epilogue,
                            const void* aux, const void* norm_weight, float eps, void* stream) {
  if (int rc = check_f16_fused(x, w, y, N, K, norm_weight)) return rc;
  if (epilogue < LOWBIT_EPI_STORE || epilogue > LOWBIT_EPI_SILU_MUL) return fail(LOWBIT_ERR_ARG, "unknown epilogue");
  if ((epilogue == LOWBIT_EPI_BIAS || epilogue == LOWBIT_EPI_RESIDUAL) && !aux)
    return fail(LOWBIT_ERR_ARG, "the bias and residual epilogues need aux");
  if (epilogue == LOWBIT_EPI_SILU_MUL && (N % 16 || (reinterpret_cast<uintptr_t>(y) & 7)))
    return fail(LOWBIT_ERR_SHAPE, "silu-mul needs N (gate and up rows) a multiple of 16 and an 8-byte aligned y");
  if (int rc = check_device()) return rc;
  GemvArgs a{static_cast<const f16*>(x), static_cast<const uint8_t*>(w), static_cast<const f16*>(x), static_cast<f16*>(y),
             1, (int)N, (int)K, (int)K, static_cast<hipStream_t>(stream)};
  a.epi.mode = epilogue;
  a.epi.aux = static_cast<const f16*>(aux);
  a.norm_w = static_cast<const f16*>(norm_weight);
  a.eps = eps;
  return hip_status(gemv_f16w_launch(a), "f16_linear_fused");
}

int lowbit_f16_qkv_rope(const void* x, const void* w, int64_t N, int64_t K, const void* bias, const void* norm_weight,
                        float eps, const int64_t* positions, const float* inv_freq, void* q_out, void* k_cache,
                        void* v_cache, int64_t Hq, int64_t Hkv, int64_t L, void* stream) {
  if (int rc = check_f16_fused(x, w, q_out, N, K, norm_weight)) return rc;
  if (!bias || !positions || !inv_freq || !k_cache || !v_cache) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (Hq < 1 || Hkv < 1 || Hq % Hkv || L < 1 || N != (Hq + 2 * Hkv) * 128 || !fits_int(L * 128 * Hkv))
    return fail(LOWBIT_ERR_SHAPE, "qkv_rope: N must be (Hq + 2 Hkv) * 128 with Hkv dividing Hq, L positive");
  if (int rc = check_device()) return rc;
  GemvArgs a{static_cast<const f16*>(x), static_cast<const uint8_t*>(w), static_cast<const f16*>(x), static_cast<f16*>(q_out),
             1, (int)N, (int)K, (int)K, static_cast<hipStream_t>(stream)};
  a.epi.mode = kEpiRopeQKV;
  a.epi.aux = static_cast<const f16*>(bias);
  a.epi.rope = RopeArgs{positions, inv_freq, nullptr, static_cast<f16*>(q_out), static_cast<f16*>(k_cache),
                        static_cast<f16*>(v_cache), (int)Hq, (int)Hkv, (int)L};
  a.norm_w = static_cast<const f16*>(norm_weight);
  a.eps = eps;
  return hip_status(gemv_f16w_launch(a), "f16_qkv_rope");
}

int lowbit_rope_table(const int64_t* positions, const float* inv_freq, void* table, int64_t M, void* stream) {
  if (!positions || !inv_freq || !table) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (M < 1 || !fits_int(M * 64)) return fail(LOWBIT_ERR_SHAPE, "rope_table: M must be positive");
  if (reinterpret_cast<uintptr_t>(table) & 3) return fail(LOWBIT_ERR_ALIGN, "rope_table needs a 4-byte aligned table");
  if (int rc = check_device()) return rc;
  return hip_status(rope_table_launch(positions, inv_freq, static_cast<uint32_t*>(table), (int)M,
                                      static_cast<hipStream_t>(stream)),
                    "rope_table");
}

int lowbit_w4_qkv_rope_rows(const void* x, const void* w, const void* s, int64_t M, int64_t N, int64_t K,
                            int64_t group, const void* bias, const int64_t* positions, const void* rope_table,
                            void* q_out, void* k_cache, void* v_cache, int64_t Hq, int64_t Hkv, int64_t L,
                            const void* norm_weight, float eps, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_common(x, w, s, q_out, M, N, K, group)) return rc;
  if (M < 1) return fail(LOWBIT_ERR_ROWS, "qkv_rope_rows takes at least one row");
  if (norm_weight && (M > 64 || K > 8192 || !aligned16(norm_weight)))
    return fail(LOWBIT_ERR_ARG, "the fused input norm takes at most 64 rows, K <= 8192 and a 16-byte aligned weight");
  if (!bias || !positions || !rope_table || !k_cache || !v_cache) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (Hq < 1 || Hkv < 1 || Hq % Hkv || L < 1 || N != (Hq + 2 * Hkv) * 128 || !fits_int(L * 128 * Hkv) ||
      !fits_int(M * Hq * 128))
    return fail(LOWBIT_ERR_SHAPE, "qkv_rope: N must be (Hq + 2 Hkv) * 128 with Hkv dividing Hq, L positive");
  if (K % 128 || group % 128) return fail(LOWBIT_ERR_LAYOUT, "the MFMA layout needs K and the group size to be multiples of 128");
  if (int rc = check_mfma_layout_limits(N, K, group, 0)) return rc;
  if (M > 64 && (M + 128) * K * 2 > INT_MAX) return fail(LOWBIT_ERR_SHAPE, "the prefill GEMM takes (M + 128) * K * 2 < 2^31");
  if (!aligned16(rope_table) ||
      ((reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(q_out) | reinterpret_cast<uintptr_t>(k_cache) |
        reinterpret_cast<uintptr_t>(v_cache)) & 7))
    return fail(LOWBIT_ERR_ALIGN, "qkv_rope_rows needs a 16-byte aligned rope table and 8-byte aligned bias, q_out and caches");
  if (workspace && (!aligned16(workspace) || workspace_bytes < kCounterBytes))
    return fail(LOWBIT_ERR_ARG, "the workspace must be 16-byte aligned and hold at least %zu bytes", kCounterBytes);
  if (int rc = check_device()) return rc;
  GemvArgs a{static_cast<const f16*>(x), static_cast<const uint8_t*>(w), static_cast<const f16*>(s), static_cast<f16*>(q_out),
             (int)M, (int)N, (int)K, (int)group, static_cast<hipStream_t>(stream)};
  a.epi.mode = kEpiRopeQKV;
  a.epi.aux = static_cast<const f16*>(bias);
  a.epi.rope = RopeArgs{positions, nullptr, static_cast<const uint32_t*>(rope_table), static_cast<f16*>(q_out),
                        static_cast<f16*>(k_cache), static_cast<f16*>(v_cache), (int)Hq, (int)Hkv, (int)L};
  a.norm_w = static_cast<const f16*>(norm_weight);
  a.eps = eps;
  if (M <= 64) return hip_status(gemm_mfma_launch(a, 0, workspace, workspace ? workspace_bytes : 0), "w4_qkv_rope_rows");
  return hip_status(gemm_prefill_launch(a, workspace, workspace ? workspace_bytes : 0), "w4_qkv_rope_rows");
}

// One token's attention followed by its output projection, the merge of the attention's key partitions done in the
// projection's prologue (shared by the int4 and fp16-weight entry points below; w4: scales given, else fp16 weights)
static int attention_linear_impl(const void* q, const void* k_cache, const void* v_cache, const int64_t* positions, int64_t Hq,
                          int64_t Hkv, int64_t L, int64_t max_keys, float scale, const void* w, const void* s, void* y,
                          int64_t N, int64_t group, int epilogue, const void* aux, void* workspace,
                          size_t workspace_bytes, void* stream, const char* what) {
  if (!q || !k_cache || !v_cache || !positions || !w || !y || !workspace) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (Hq < 1 || Hkv < 1 || Hq % Hkv || L < 1 || !fits_int(L * 128 * Hkv))
    return fail(LOWBIT_ERR_SHAPE, "%s: Hq, Hkv (dividing Hq), L must be positive", what);
  const int64_t g = Hq / Hkv, K = Hq * 128;
  if (!(g == 1 || g == 2 || g == 4 || g == 6 || g == 7 || g == 8))
    return fail(LOWBIT_ERR_SHAPE, "%s takes 1, 2, 4, 6, 7 or 8 query heads per KV head", what);
  if (Hq > 32) return fail(LOWBIT_ERR_SHAPE, "%s takes at most 32 query heads (x of at most 4096)", what);
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(w))
    return fail(LOWBIT_ERR_ALIGN, "%s needs 16-byte aligned q, caches and weights", what);
  const size_t need = kAttnCounterBytes + (size_t)Hq * kAttnRec * 4;
  if (!aligned16(workspace) || workspace_bytes < need)
    return fail(LOWBIT_ERR_ARG, "%s: the workspace must be 16-byte aligned and hold at least %zu bytes", what, need);
  if (N < 1 || !fits_int(N)) return fail(LOWBIT_ERR_SHAPE, "%s: N must be positive", what);
  if (s) {
    if (group % 128 || group < 128 || K % group) return fail(LOWBIT_ERR_LAYOUT, "%s: the group must be a multiple of 128 dividing K", what);
    if (int rc = check_mfma_layout_limits(N, K, group, 1)) return rc;
  }
  if (epilogue < LOWBIT_EPI_STORE || epilogue > LOWBIT_EPI_SILU_MUL) return fail(LOWBIT_ERR_ARG, "unknown epilogue");
  if ((epilogue == LOWBIT_EPI_BIAS || epilogue == LOWBIT_EPI_RESIDUAL) && !aux)
    return fail(LOWBIT_ERR_ARG, "the bias and residual epilogues need aux");
  if (epilogue == LOWBIT_EPI_SILU_MUL && (N % 16 || (reinterpret_cast<uintptr_t>(y) & 7)))
    return fail(LOWBIT_ERR_SHAPE, "silu-mul needs N (gate and up rows) a multiple of 16 and an 8-byte aligned y");
  if (int rc = check_device()) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  f16* xbuf = reinterpret_cast<f16*>(ws + kAttnCounterBytes);   // the attention's output when it runs unsplit
  int parts = 1;
  hipError_t e = attention_partials_launch(static_cast<const f16*>(q), static_cast<const f16*>(k_cache),
                                           static_cast<const f16*>(v_cache), positions, xbuf, (int)Hq, (int)Hkv, (int)L,
                                           (int)std::max<int64_t>(1, std::min(max_keys, L)), scale, workspace,
                                           workspace_bytes, &parts, st);
  if (e != hipSuccess) return hip_status(e, what);
  GemvArgs a{xbuf, static_cast<const uint8_t*>(w), s ? static_cast<const f16*>(s) : xbuf, static_cast<f16*>(y), 1,
             (int)N, (int)K, s ? (int)group : (int)K, st};
  a.epi.mode = epilogue;
  a.epi.aux = static_cast<const f16*>(aux);
  if (parts > 1) {
    a.epi.attn_part = reinterpret_cast<const float*>(ws + kAttnCounterBytes);
    a.epi.attn_parts = parts;
  }
  return hip_status(s ? gemv_mfma_layout_launch(a, 0) : gemv_f16w_launch(a), what);
}

int lowbit_attention(const void* q, const void* k_cache, const void* v_cache, const int64_t* positions, void* out,
                     int64_t M, int64_t Hq, int64_t Hkv, int64_t L, int64_t max_keys, float scale, void* workspace,
                     size_t workspace_bytes, void* stream) {
  if (!q || !k_cache || !v_cache || !positions || !out) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (M < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || L < 1 || !fits_int(M * Hkv) || !fits_int(L * 128 * Hkv))
    return fail(LOWBIT_ERR_SHAPE, "attention: M, Hq, Hkv (dividing Hq), L must be positive");
  const int64_t g = Hq / Hkv;
  if (!(g == 1 || g == 2 || g == 4 || g == 6 || g == 7 || g == 8))
    return fail(LOWBIT_ERR_SHAPE, "attention takes 1, 2, 4, 6, 7 or 8 query heads per KV head");
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache)) return fail(LOWBIT_ERR_ALIGN, "attention needs 16-byte aligned q and caches");
  if (workspace && (!aligned16(workspace) || workspace_bytes < kAttnCounterBytes))
    return fail(LOWBIT_ERR_ARG, "the attention workspace must be 16-byte aligned and hold at least %zu bytes",
                kAttnCounterBytes);
  if (int rc = check_device()) return rc;
  return hip_status(attention_launch(static_cast<const f16*>(q), static_cast<const f16*>(k_cache),
                                     static_cast<const f16*>(v_cache), positions, static_cast<f16*>(out), (int)M,
                                     (int)Hq, (int)Hkv, (int)L, (int)std::max<int64_t>(1, std::min(max_keys, L)), scale,
                                     workspace, workspace ? workspace_bytes : 0, static_cast<hipStream_t>(stream)),
                    "attention");
}

int lowbit_w4_attention_linear(const void* q, const void* k_cache, const void* v_cache, const int64_t* positions,
                               int64_t Hq, int64_t Hkv, int64_t L, int64_t max_keys, float scale, const void* w,
                               const void* s, void* y, int64_t N, int64_t group, int epilogue, const void* aux,
                               void* workspace, size_t workspace_bytes, void* stream) {
  if (!s) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  return attention_linear_impl(q, k_cache, v_cache, positions, Hq, Hkv, L, max_keys, scale, w, s, y, N, group, epilogue,
                               aux, workspace, workspace_bytes, stream, "w4_attention_linear");
}

int lowbit_f16_attention_linear(const void* q, const void* k_cache, const void* v_cache, const int64_t* positions,
                                int64_t Hq, int64_t Hkv, int64_t L, int64_t max_keys, float scale, const void* w,
                                void* y, int64_t N, int epilogue, const void* aux, void* workspace,
                                size_t workspace_bytes, void* stream) {
  return attention_linear_impl(q, k_cache, v_cache, positions, Hq, Hkv, L, max_keys, scale, w, nullptr, y, N, 0,
                               epilogue, aux, workspace, workspace_bytes, stream, "f16_attention_linear");
}

int lowbit_f16_gemv(const void* x, const void* w, void* y, int64_t M, int64_t N, int64_t K, void* stream) {
  if (!x || !w || !y) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (M < 1 || M > 64) return fail(LOWBIT_ERR_ROWS, "the fp16 GEMV takes 1..64 rows");
  if (N < 1 || K < 8 || K % 8 || !fits_int(N) || (int64_t)16 * K * 2 > INT_MAX || M * K * 2 > INT_MAX)
    return fail(LOWBIT_ERR_SHAPE, "the fp16 GEMV takes K % 8 == 0");
  if ((M > 16 || M * K * 2 > 65536) && K % 128)
    return fail(LOWBIT_ERR_SHAPE, "the fp16 GEMV takes K % 128 == 0 beyond 16 rows or M * K * 2 > 65536");
  if (!aligned16(x) || !aligned16(w)) return fail(LOWBIT_ERR_ALIGN, "x and w must be 16-byte aligned");
  if (int rc = check_device()) return rc;
  return hip_status(gemv_f16_launch(static_cast<const f16*>(x), static_cast<const f16*>(w), static_cast<f16*>(y), (int)M,
                                    (int)N, (int)K, static_cast<hipStream_t>(stream)),
                    "f16_gemv");
}

int lowbit_f16_gemv_pick(const void* x, const void* w, void* y, int64_t N, int64_t K, void* workspace,
                         size_t workspace_bytes, int64_t* tokens, int64_t* positions, int64_t* out_tokens,
                         int64_t out_capacity, int32_t* out_count, const void* embed, void* h_out, void* stream) {
  if (!x || !w || !y || !workspace || !tokens) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (!out_tokens != !out_count || !embed != !h_out)
    return fail(LOWBIT_ERR_ARG, "out_tokens goes with out_count, embed with h_out");
  if (out_count && (out_capacity < 0 || !fits_int(out_capacity)))
    return fail(LOWBIT_ERR_SHAPE, "f16_gemv_pick: out_capacity must be a non-negative 32-bit count");
  if (embed && (!aligned16(embed) || !aligned16(h_out)))
    return fail(LOWBIT_ERR_ALIGN, "f16_gemv_pick: embed and h_out must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(out_tokens) & 7) || (reinterpret_cast<uintptr_t>(out_count) & 3))
    return fail(LOWBIT_ERR_ALIGN, "f16_gemv_pick needs naturally aligned out_tokens and out_count");
  if (N < 1 || K < 8 || K % 8 || !fits_int(N) || K * 2 > 65536)
    return fail(LOWBIT_ERR_SHAPE, "the fp16 GEMV takes K % 8 == 0 and K * 2 <= 65536");
  if (!aligned16(x) || !aligned16(w)) return fail(LOWBIT_ERR_ALIGN, "x and w must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(workspace) | reinterpret_cast<uintptr_t>(tokens) |
       reinterpret_cast<uintptr_t>(positions)) & 7)
    return fail(LOWBIT_ERR_ALIGN, "f16_gemv_pick needs an 8-byte aligned workspace, tokens and positions");
  const size_t need = (size_t)8 * head_pick_parts((int)N);
  if (workspace_bytes < need)
    return fail(LOWBIT_ERR_ARG, "f16_gemv_pick needs a workspace of at least %zu bytes for N = %lld", need,
                (long long)N);
  if (int rc = check_device()) return rc;
  return hip_status(head_pick_launch(static_cast<const f16*>(x), static_cast<const f16*>(w), static_cast<f16*>(y),
                                     (int)N, (int)K, static_cast<uint64_t*>(workspace), tokens, positions, out_tokens,
                                     (int)out_capacity, out_count, static_cast<const f16*>(embed),
                                     static_cast<f16*>(h_out), static_cast<hipStream_t>(stream)),
                    "f16_gemv_pick");
}

int lowbit_hbm_read(const void* src, int64_t bytes, void* sink, int64_t blocks, void* stream) {
  if (!src || !sink) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (bytes < 16 || bytes % 16) return fail(LOWBIT_ERR_SHAPE, "hbm_read: bytes must be a positive multiple of 16");
  if (blocks < 1 || blocks > 65536) return fail(LOWBIT_ERR_SHAPE, "hbm_read: blocks must be 1..65536");
  if (!aligned16(src) || reinterpret_cast<uintptr_t>(sink) % 4) return fail(LOWBIT_ERR_ALIGN, "hbm_read needs a 16-byte aligned source");
  if (int rc = check_device()) return rc;
  return hip_status(hbm_read_launch(src, (size_t)bytes, static_cast<uint32_t*>(sink), (int)blocks,
                                    static_cast<hipStream_t>(stream)),
                    "hbm_read");
}

int lowbit_hbm_copy(const void* src, void* dst, int64_t bytes, int64_t blocks, void* stream) {
  if (!src || !dst) return fail(LOWBIT_ERR_ARG, "null pointer argument");
  if (bytes < 16 || bytes % 16) return fail(LOWBIT_ERR_SHAPE, "hbm_copy: bytes must be a positive multiple of 16");
  if (blocks < 1 || blocks > 65536) return fail(LOWBIT_ERR_SHAPE, "hbm_copy: blocks must be 1..65536");
  if (!aligned16(src) || !aligned16(dst)) return fail(LOWBIT_ERR_ALIGN, "hbm_copy needs 16-byte aligned buffers");
  if (int rc = check_device()) return rc;
  return hip_status(hbm_copy_launch(src, dst, (size_t)bytes, (int)blocks, static_cast<hipStream_t>(stream)), "hbm_copy");
}

}  // extern "C"
