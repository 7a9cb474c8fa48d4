// Device-side building blocks shared by the gfx950 W4A16 kernels: vector types, the exact nibble decode, wave64
// reductions (DPP + readlane, no LDS), buffer-resource loads and the launch helper.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace lowbit {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 0x6400 is 1024.0 in fp16, where the mantissa step is exactly 1: (0x6400 | u) reads as 1024 + u for a nibble in
// bits 0..3, and as 1024 + 16 u for a nibble in bits 4..7.
constexpr uint32_t kMagic = 0x64006400u;

__device__ __forceinline__ f16x2 as_f16x2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t as_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// A 32-bit word in v3 nibble order (slots 0..7 hold k0, k2, k4, k6, k1, k3, k5, k7) -> four fp16 pairs holding the
// signed values u - 8 exactly: p[0] = (k0, k1), p[1] = (k2, k3), p[2] = (k4, k5), p[3] = (k6, k7).
// Pairs 1 and 3 sit in bits 4..7 of each half, so (1024 + 16 u) / 16 - 72 = u - 8 (one fused step, exact) saves the
// shift the low-nibble pairs would need. For a canonical word the same code yields (k0,k4), (k1,k5), (k2,k6), (k3,k7).
__device__ __forceinline__ void decode_word(uint32_t w, f16x2 p[4]) {
  const f16x2 m1032 = {(f16)-1032.0f, (f16)-1032.0f};
  const f16x2 m72 = {(f16)-72.0f, (f16)-72.0f};
  const f16x2 inv16 = {(f16)0.0625f, (f16)0.0625f};
  const uint32_t w8 = w >> 8;
  p[0] = as_f16x2((w & 0x000F000Fu) | kMagic) + m1032;
  p[1] = as_f16x2((w & 0x00F000F0u) | kMagic) * inv16 + m72;
  p[2] = as_f16x2((w8 & 0x000F000Fu) | kMagic) + m1032;
  p[3] = as_f16x2((w8 & 0x00F000F0u) | kMagic) * inv16 + m72;
}

// The decode's bit masks (scalar registers) and magic number (one vector register). gfx9 VOP3 instructions take no
// literal operand and at most one scalar one, so with literal constants the compiler emits each (w & mask) | magic
// as an AND and an OR; with the mask in an SGPR and the magic in a VGPR it is one v_and_or_b32, for one VGPR. Create
// once per kernel, outside the loops (the empty asm hides the constants from constant folding).
struct DecodeRegs {
  uint32_t lo, hi, magic;
};
__device__ __forceinline__ uint32_t in_vgpr(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ uint32_t in_sgpr(uint32_t v) {
  asm volatile("" : "+s"(v));
  return v;
}
__device__ __forceinline__ DecodeRegs decode_regs() {
  return DecodeRegs{in_sgpr(0x000F000Fu), in_sgpr(0x00F000F0u), in_vgpr(kMagic)};
}

// A v3 word as an MFMA A fragment: the eight fp16 values u - 8 (exact) for k0 .. k7 in k order, pairs as in
// decode_word: four v_and_or_b32, two packed adds, two packed FMAs and one shift.
__device__ __forceinline__ f16x8 decode_word_a(uint32_t w, const DecodeRegs& c) {
  const f16x2 m1032 = {(f16)-1032.0f, (f16)-1032.0f};
  const f16x2 m72 = {(f16)-72.0f, (f16)-72.0f};
  const f16x2 inv16 = {(f16)0.0625f, (f16)0.0625f};
  const uint32_t w8 = w >> 8;
  const f16x2 p0 = as_f16x2((w & c.lo) | c.magic) + m1032;
  const f16x2 p1 = as_f16x2((w & c.hi) | c.magic) * inv16 + m72;
  const f16x2 p2 = as_f16x2((w8 & c.lo) | c.magic) + m1032;
  const f16x2 p3 = as_f16x2((w8 & c.hi) | c.magic) * inv16 + m72;
  return __builtin_bit_cast(f16x8, u32x4{as_u32(p0), as_u32(p1), as_u32(p2), as_u32(p3)});
}

__device__ __forceinline__ float dot2(f16x2 a, f16x2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

// Subnormal decode for dot products: a nibble alone in the mantissa of an fp16 half (exponent 0) is the subnormal
// u * 2^-24 (bits 0..3) or u * 2^-20 (bits 4..7), which v_dot2_f32_f16 multiplies exactly (fp16 denormals are on).
// For a v3 word: lo[0] = (k0, k1), lo[1] = (k4, k5) scaled 2^-24; hi[0] = (k2, k3), hi[1] = (k6, k7) scaled 2^-20.
// The offset 8 is removed by subtracting the same dot2 sequence run on nibbles 8 (see the GEMV), so runs of zero
// weights cancel exactly.
__device__ __forceinline__ void decode_word_subnormal(uint32_t w, f16x2 lo[2], f16x2 hi[2]) {
  const uint32_t w8 = w >> 8;
  lo[0] = as_f16x2(w & 0x000F000Fu);
  hi[0] = as_f16x2(w & 0x00F000F0u);
  lo[1] = as_f16x2(w8 & 0x000F000Fu);
  hi[1] = as_f16x2(w8 & 0x00F000F0u);
}

template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}
constexpr int kQuadSwap1 = 0xB1;       // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kQuadSwap2 = 0x4E;       // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kRowHalfMirror = 0x141;  // lane ^ 7 inside 8 lanes
constexpr int kRowMirror = 0x140;      // lane ^ 15 inside 16 lanes

template <int kV>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {   // value of lane kV of each quad
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kV | (kV << 2) | (kV << 4) | (kV << 6), 0xF, 0xF, false);
}

// sum over the 4 lanes of a quad; every lane of the quad gets the total
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp<kQuadSwap1>(v);
  v += dpp<kQuadSwap2>(v);
  return v;
}

// sum over the 16 lanes of each row; every lane of the row gets the row's total
__device__ __forceinline__ float row_sum(float v) {
  v = quad_sum(v);
  v += dpp<kRowHalfMirror>(v);   // quads are uniform, so lane ^ 7 reaches the other quad of the 8
  v += dpp<kRowMirror>(v);       // 8-lane groups are uniform, lane ^ 15 reaches the other half of the row
  return v;
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// sum over all 64 lanes (all lanes must be active); the result is wave-uniform. The four rows are combined through
// v_readlane in a fixed order, so the sum is deterministic. (permlane16/32_swap with both operands the same value is
// miscompiled by this toolchain -- both results are taken from one register -- so it is not used for this.)
__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kQuadSwap1>(v));
  v = fmaxf(v, dpp<kQuadSwap2>(v));
  v = fmaxf(v, dpp<kRowHalfMirror>(v));
  v = fmaxf(v, dpp<kRowMirror>(v));
  return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}

// Raw buffer resource over [base, base + bytes): loads at offsets at or past `bytes` return zeros and touch no
// memory, so tails and idle lanes need no branch around the load (0x00020000: the gfx9 raw-buffer dword 3).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
constexpr int kOutOfRange = 0x7FFFFFF0;    // a buffer offset past any resource this library builds
constexpr int kNonTemporal = 2;            // gfx94x/gfx950 cache policy bit: streamed, no reuse expected
__device__ __forceinline__ u32x4 buffer_load16_nt(__amdgpu_buffer_rsrc_t rsrc, int offset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, kNonTemporal));
}
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, int offset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, 0));
}
__device__ __forceinline__ uint16_t buffer_load2(__amdgpu_buffer_rsrc_t rsrc, int offset) {
  return __builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(rsrc, offset, 0, 0));
}
// non-temporal 2-byte load: for the GEMV's group scales, read once per call like the weights (measured on MI355X:
// 0.14-0.25 us per launch sooner than a default-policy load, which the staging barrier waits for)
__device__ __forceinline__ uint16_t buffer_load2_nt(__amdgpu_buffer_rsrc_t rsrc, int offset) {
  return __builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(rsrc, offset, 0, kNonTemporal));
}

// Split-K partial sums handed from one workgroup to another: buffer stores and loads with the sc1 cache-policy bit,
// which on gfx950 makes each access coherent across the XCDs' L2 caches by itself (the LLVM AMDGPU memory model
// implements relaxed agent-scope atomic stores and loads as exactly these accesses, 4 or 8 bytes wide; here 16). So
// once a writer has waited for its stores' acknowledgements, its arrival can be counted with a relaxed atomic: no
// release (an L2 write-back in every split workgroup) and no acquire (an L2 invalidate in the last one).
constexpr int kAgentCoherent = 16;         // gfx94x/gfx950 cache policy bit sc1
__device__ __forceinline__ void store_partial4(__amdgpu_buffer_rsrc_t r, int offset, const f32x4& v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, offset, 0, kAgentCoherent);
}
__device__ __forceinline__ void store_partial(__amdgpu_buffer_rsrc_t r, int offset, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, offset, 0, kAgentCoherent);
}
__device__ __forceinline__ f32x4 load_partial4(__amdgpu_buffer_rsrc_t r, int offset) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, kAgentCoherent));
}
__device__ __forceinline__ float load_partial(__amdgpu_buffer_rsrc_t r, int offset) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, offset, 0, kAgentCoherent));
}
// The K split's fixup: the sum of the S partials of four outputs at byte offsets off(0) .. off(S - 1), added in split
// order. The loads go out in batches of 8 before the first add: a loop that adds each partial as it loads it waits one
// memory round trip per split (measured on MI355X: 3.0 us of a 12 us launch at S = 8). `lanes` < 4: only the first
// `lanes` outputs exist, loaded and added one by one.
template <typename Off>
__device__ __forceinline__ f32x4 sum_partials4(__amdgpu_buffer_rsrc_t r, int S, int lanes, Off off) {
  f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < S; s0 += 8) {
    if (lanes == 4) {
      f32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = load_partial4(r, s0 + u < S ? off(s0 + u) : kOutOfRange);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s0 + u < S) sum += v[u];
    } else {
      float v[8][4];
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[u][e] = load_partial(r, s0 + u < S && e < lanes ? off(s0 + u) + 4 * e : kOutOfRange);
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (s0 + u < S && e < lanes) sum[e] += v[u][e];
    }
  }
  return sum;
}

// ---- direct-to-LDS loads (gfx950: 16 bytes per lane) ----
// The LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}
// One wave-load straight into LDS: lane l's 16 bytes at buffer offset `voffset` land at LDS byte `lds` + 16 l (M0
// carries the wave-uniform `lds`). Written as inline asm, so the compiler neither inserts waits for it nor holds LDS
// accesses back behind it: the caller counts these loads itself (lds_wait_read16, lds_wait_barrier). Vector-memory
// operations of one wave complete in issue order, so "at most N outstanding" means everything but the newest N has
// landed; a load of the compiler's issued later only makes such a wait longer, never short. m0 is otherwise unused
// by the kernels that call this (gfx9 LDS instructions do not read it).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, int voffset, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voffset), "s"(r),
               "s"(lds)
               : "memory", "m0");
}
__device__ __forceinline__ void dma16_nt(__amdgpu_buffer_rsrc_t r, int voffset, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds" ::"v"(voffset), "s"(r),
               "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop
// Wait until at most N of this wave's vector-memory operations are outstanding, then read 16 bytes at LDS byte
// `addr`. The read and its own wait sit in the same statement, so the value is complete when the statement ends and
// no instruction the compiler schedules can use it earlier.
template <int N>
__device__ __forceinline__ u32x4 lds_wait_read16(uint32_t addr) {
  u32x4 v;
  asm volatile("s_waitcnt vmcnt(%1)\n\tds_read_b128 %0, %2\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "n"(N), "v"(addr)
               : "memory");
  return v;
}
// Workgroup barrier once at most N of this wave's vector-memory operations are outstanding and its LDS accesses are
// done: direct-to-LDS loads older than the newest N are then visible to every wave. No cache write-back or invalidate
// (the compiler's __syncthreads would also drain every load in flight).
template <int N>
__device__ __forceinline__ void lds_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ u32x4 load_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x4 load16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// ---- output epilogues (the modes are listed with struct Epilogue in kernels.hpp) ----

// y value for one output of the store / bias / residual modes
__device__ __forceinline__ f16 epi_value(int mode, const f16* __restrict__ aux, float acc, int m, int n, int N) {
  const f16 v = (f16)acc;
  if (mode == 1) return v + aux[n];
  if (mode == 2) return aux[(size_t)m * N + n] + v;
  return v;
}

// epi_value with its bias or residual element a already loaded (the same arithmetic)
__device__ __forceinline__ f16 epi_apply(int mode, f16 a, float acc) {
  const f16 v = (f16)acc;
  if (mode == 1) return v + a;
  if (mode == 2) return a + v;
  return v;
}

// RoPE of one dim pair (d, d + 64) at position p as transformers computes it for fp16 models: angle =
// fp32(p * inv_freq[d]), cos and sin in fp32 rounded to fp16, x * cos + rotate_half(x) * sin with each product and
// the sum rounded to fp16 (no contraction)
__device__ __forceinline__ void rope_rotate(f16 x1, f16 x2, f16 c, f16 s, f16& o1, f16& o2) {
#pragma clang fp contract(off)
  o1 = (f16)(x1 * c) + (f16)(-x2 * s);
  o2 = (f16)(x2 * c) + (f16)(x1 * s);
}

// the fp16 cos and sin of the angle p * inv_f (fp32), as rope_pair rounds them
__device__ __forceinline__ void rope_cos_sin(int64_t p, float inv_f, f16& c, f16& s) {
#pragma clang fp contract(off)
  const float ang = (float)p * inv_f;
  c = (f16)cosf(ang);
  s = (f16)sinf(ang);
}

__device__ __forceinline__ void rope_pair(f16 x1, f16 x2, int64_t p, float inv_f, f16& o1, f16& o2) {
  f16 c, s;
  rope_cos_sin(p, inv_f, c, s);
  rope_rotate(x1, x2, c, s, o1, o2);
}

// row of head dim d (< 64: the first of the pair) in the RoPE-permuted q|k|v layout: tile d / 8, rows 0..7 hold dims
// 8 t .. 8 t + 7 and rows 8..15 their partners 64 + 8 t ..
__device__ __forceinline__ int rope_row(int d) { return 16 * (d >> 3) + (d & 7); }

// silu(g) * u with the rounding of the torch ops it replaces: g and u rounded to fp16, silu evaluated in fp32 as
// g / (1 + exp(-g)) and rounded, the product rounded
__device__ __forceinline__ f16 silu_mul(float g, float u) {
  const float g16 = (float)(f16)g;
  const f16 s = (f16)(g16 / (1.0f + expf(-g16)));
  return (f16)((float)s * (float)(f16)u);
}

// Bind kernel arguments to scalar registers at the kernel's start. Kernel arguments are read through the scalar cache,
// which is cold at every launch (a few hundred ns per round trip); the compiler otherwise fetches each argument at its
// first use, so a prologue whose later addresses depend on later arguments waits for two or three round trips before
// its main loads go out. Naming them all here issues every fetch before the first wait.
template <typename T>
__device__ __forceinline__ void arg_in_sgpr(const T& v) {
  asm volatile("" ::"s"(v));
}
template <typename... T>
__device__ __forceinline__ void args_in_sgprs(const T&... v) {
  (arg_in_sgpr(v), ...);
}

__device__ __forceinline__ float shfl_down32(float v) {     // lane l gets lane l + 32 (lanes 32..63 get their own)
  return __shfl_down(v, 32, 64);
}

// Launch on `stream` and report the launch status.
template <typename... KArgs, typename... Args>
inline hipError_t launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t shmem, hipStream_t stream,
                         Args... args) {
  kernel<<<grid, block, shmem, stream>>>(static_cast<KArgs>(args)...);
  return hipGetLastError();
}

// Raise a kernel's dynamic LDS limit above the default 64 KiB (gfx950 has 160 KB per CU).
template <typename... KArgs>
inline hipError_t allow_lds(void (*kernel)(KArgs...), size_t bytes) {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)bytes);
}

}  // namespace lowbit
