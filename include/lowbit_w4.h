/* lowbit_w4.h -- C ABI of liblowbit_w4.so, the gfx950 W4A16 kernel library.
 *
 * Format (reference lowbit/quant.py:1-35): a weight W [N, K] is stored as symmetric int4, one fp16 scale per group of
 * G consecutive values along K (G % 32 == 0, K % G == 0), the nibble u = q + 8 two per byte, low nibble = even k.
 * Three byte layouts of the packed tensor [N, K/2] exist:
 *   LOWBIT_LAYOUT_CANONICAL  row-major bytes as quantized (reference "canonical", lowbit/quant.py:7-8);
 *   LOWBIT_LAYOUT_V3         canonical with each 32-bit word in the nibble order [k0,k2,k4,k6,k1,k3,k5,k7]
 *                            (reference interleave_for_gpu, lowbit/quant.py:55-64);
 *   LOWBIT_LAYOUT_MFMA       this library's gfx950 device layout, the one copy a model keeps and the counterpart of
 *                            the reference's "mma" layout (lowbit/quant.py:67-78): 16-row tiles; inside tile t, the
 *                            128-k chunk c holds rows_t x 64 bytes (row r at offset 64 r), words in v3 order.
 *                            Needs K % 128 == 0 and G % 128 == 0.
 * Scales are always float16 [N, K/G], row-major.
 *
 * Conventions. Pointers are device pointers unless the function name says host. x, y and scales are IEEE binary16
 * (passed as void*). `stream` is a hipStream_t (NULL = the default stream). Every entry point validates its
 * arguments first and returns LOWBIT_OK (0) or a status code; lowbit_last_error() returns the message of the last
 * failure on the calling thread (the same wording as the reference's TORCH_CHECK messages). No entry point
 * allocates device memory: outputs are owned by the caller, so every launch can be captured into a hipGraph.
 * Launches are asynchronous on `stream`.
 */
#ifndef LOWBIT_W4_H
#define LOWBIT_W4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  LOWBIT_OK = 0,
  LOWBIT_ERR_ARG = 1,      /* a NULL pointer, a bad enum value, a non-positive size */
  LOWBIT_ERR_GROUP = 2,    /* group size not positive / not a multiple of 32, or K not a multiple of it */
  LOWBIT_ERR_SHAPE = 3,    /* inconsistent sizes */
  LOWBIT_ERR_ALIGN = 4,    /* x / w not 16-byte aligned */
  LOWBIT_ERR_ROWS = 5,     /* M outside the kernel's range */
  LOWBIT_ERR_VERSION = 6,  /* unknown kernel version */
  LOWBIT_ERR_LAYOUT = 7,   /* the MFMA layout needs K % 128 == 0 and G % 128 == 0 */
  LOWBIT_ERR_TUNING = 8,   /* rows_per_wave / row_tiles not in the allowed set */
  LOWBIT_ERR_HIP = 9,      /* a HIP runtime call or launch failed */
  LOWBIT_ERR_DEVICE = 10   /* the current device is not gfx950 */
};

enum { LOWBIT_LAYOUT_CANONICAL = 0, LOWBIT_LAYOUT_V3 = 1, LOWBIT_LAYOUT_MFMA = 2, LOWBIT_LAYOUT_NV_MMA = 3 };
enum { LOWBIT_DTYPE_F32 = 0, LOWBIT_DTYPE_F16 = 1, LOWBIT_DTYPE_BF16 = 2 };

/* Message of the last failed call on this thread ("" if none). */
const char* lowbit_last_error(void);
/* Short name of a status code. */
const char* lowbit_strerror(int status);
/* Library version string. */
const char* lowbit_version(void);

/* Process-wide launch-shape override of the MFMA-layout kernels, for tuning sweeps. waves_per_group: the M <= 8
 * GEMV's waves per workgroup (0 = automatic, else 1, 2, 4, 8 or 16; clamped to what the register budget allows); for
 * the prefill GEMM the tile shape (1: 64 activation rows / 4 waves, 2: 64 / 8 waves, 4: 128 / 4 waves, 8: 128 / 8
 * waves, which is never built and falls back to 4 waves). ring: chunk slots in flight per wave (0 = automatic, else
 * 2, 3, 4 or 8: the GEMV uses 4 or 8, 8 only for M <= 2; the MFMA GEMM 2, 3 or 4; the prefill GEMM 2 or 3, and 4 =
 * 2 with a two-chunk activation lookahead). k_splits: workgroups the MFMA and prefill GEMMs split K over
 * (0 = automatic, 1..32; bounded by the workspace and by K / 128); for the M <= 8 GEMV, workgroups sharing one
 * 16-row tile (1, 2 or 4, owning 16, 8 or 4 rows each; honoured with one tile per wave, K / 128 a multiple of it and
 * no silu-mul or RoPE epilogue, which pair rows r and r + 8; other values leave the GEMV's choice automatic).
 * Affects later launches only. No counterpart in the reference (its launch shapes were compile-time template
 * choices). */
int lowbit_set_launch_override(int waves_per_group, int ring, int k_splits);

/* Process-wide choice of where the M = 1 v6 GEMV keeps its weight ring, for tuning sweeps and tests: 0 = automatic;
 * -1 = in registers (4 slots per wave); 4, 8, 12 or 16 = that many 1 KB slots per wave in LDS, filled by
 * direct-to-LDS loads (fewer when the workgroup's LDS would not fit a CU). The sums are formed in the same order
 * either way, so the results are identical bit for bit. Affects later launches only. No counterpart in the
 * reference. */
int lowbit_set_gemv_lds_ring(int slots);

/* Process-wide choice of the MFMA GEMM's workgroup order when K is split across workgroups, for tuning sweeps and
 * tests: 0 = automatic; 1 = row groups fastest; 2 = splits fastest (the workgroups of one split, which read the same
 * slice of x, share an XCD). The split partials are added in split order either way, so the results are identical
 * bit for bit. Affects later launches only. No counterpart in the reference. */
int lowbit_set_gemm_order(int order);

/* Process-wide choice of the MFMA GEMM's structure (lowbit_w4_gemm_mfma, lowbit_w4_linear_fused for M >= 2), for
 * tuning sweeps and tests: 0 = automatic; 1 = row groups of 64 or 128 weight rows sharing staged activations, K split
 * across workgroups on narrow layers; 2 = one 16-row tile per workgroup, its waves splitting K (M <= 32 only; larger M
 * keeps row groups). Results of the two differ only in fp32 summation order. Affects later launches only. No
 * counterpart in the reference. */
int lowbit_set_gemm_kernel(int kernel);

/* Process-wide choice of the MFMA GEMM's tile-waves per K-group in its row-group structure, for tuning sweeps and
 * tests: 0 = automatic; 3, 4, 5, 6 or 8 (all but 4 with one 16-row tile per wave and 2 ring slots; 3 with up to 4
 * K-groups at M <= 32, else 2, 5, 6 and 8 with at most 2; with row_tiles = 2 the GEMM keeps 4). Each tile is computed the same way whatever the count, so the results are
 * identical bit for bit. Affects later launches only. No counterpart in the reference. */
int lowbit_set_gemm_tile_waves(int tile_waves);

/* y[M, N] (fp16) = x[M, K] (fp16) . dequant(W)^T, 1 <= M <= 8.
 * Replaces the reference's w4_gemv (csrc/w4_gemv.cu:454-484) and, through it, ops.gemv(version in 1..4, 6)
 * (lowbit/ops.py:67-78). version 1 or 2: w in the canonical layout; 3 or 4: v3 layout; 6: the MFMA layout (needs
 * K % 128 == 0 and G % 128 == 0). rows_per_wave: 0 = chosen from N and M, else 1, 2 or 4 (versions 1-4: output
 * rows per wave; version 6: 16-row tiles per wave). fp32 accumulation. */
int lowbit_w4_gemv(const void* x, const void* w, const void* s, void* y, int64_t M, int64_t N, int64_t K, int64_t group,
                   int version, int rows_per_wave, void* stream);

/* Workspace of lowbit_w4_gemm_mfma: LOWBIT_WORKSPACE_COUNTER_BYTES of arrival counters, which must be zero before
 * the first call and which every call leaves zero, then fp32 partial sums. LOWBIT_WORKSPACE_BYTES lets every shape
 * with M * N <= 65536 split K the full 32 ways; a smaller workspace splits less. */
#define LOWBIT_WORKSPACE_COUNTER_BYTES 16384
#define LOWBIT_WORKSPACE_BYTES (LOWBIT_WORKSPACE_COUNTER_BYTES + (16u << 20))

/* y[M, N] (fp16) = x[M, K] . dequant(W)^T on the MFMA layout with fp16 MFMA (fp32 accumulate), 1 <= M <= 64.
 * Replaces the reference's w4_gemm_tc (csrc/w4_gemv.cu:486-515), i.e. ops.gemv(version 5) (lowbit/ops.py:75-76).
 * row_tiles: 0 = automatic, else 1, 2 or 4 sixteen-row tiles per wave. workspace (device memory, 16-byte aligned,
 * see above; may be NULL): lets narrow N split K across workgroups; the partial sums are added in a fixed order,
 * so a given shape, workspace size and override give the same bits on every call. Calls that share a workspace must not run concurrently (one stream per workspace). The workspace argument
 * has no counterpart in the reference, whose extension allocated nothing beyond the output. */
int lowbit_w4_gemm_mfma(const void* x, const void* w, const void* s, void* y, int64_t M, int64_t N, int64_t K,
                        int64_t group, int row_tiles, void* workspace, size_t workspace_bytes, void* stream);

/* Size of the device scratch lowbit_w4_gemm_mfma_noalloc uses in place of a workspace: the same as
 * LOWBIT_WORKSPACE_BYTES (16 KiB of arrival counters + 16 MiB of fp32 partial sums). */
#define LOWBIT_NOALLOC_SCRATCH_BYTES LOWBIT_WORKSPACE_BYTES

/* lowbit_w4_gemm_mfma with no workspace argument and no allocation of any kind: for callers that cannot call
 * hipMalloc (code under hipGraph capture, tight serving loops, harnesses that forbid allocation). No counterpart in
 * the reference. The caller passes inputs and outputs; the split-K workspace is a file-scope device array of
 * LOWBIT_NOALLOC_SCRATCH_BYTES in the library, one per GPU, held until the process ends and found with
 * hipGetSymbolAddress on the first call on each device. The launch plan is the one lowbit_w4_gemm_mfma makes with a
 * workspace of that size, so the two give the same bits for the same shape and override. Sizes: 1 <= M <= 64 as
 * lowbit_w4_gemm_mfma; the partial sums of a K split take S * M * N * 4 bytes and the planner lowers S to what the
 * scratch holds (M * N <= 131072 keeps the full 32-way split), and a plan that would still not fit is refused with
 * LOWBIT_ERR_SHAPE. Every call on a GPU shares that GPU's scratch, which keeps the last call's contents: the arrival
 * counters are cleared by a kernel before first use and every call leaves them zero. Calls that overlap on one GPU
 * (concurrent streams, or graphs replayed concurrently) race on the scratch and give wrong results: serialize them. */
int lowbit_w4_gemm_mfma_noalloc(const void* x, const void* w, const void* s, void* y, int64_t M, int64_t N, int64_t K,
                                int64_t group, int row_tiles, void* stream);

/* out[N, K] (fp16) = (u - 8) * scale rounded once to fp16, from the canonical (mfma_layout = 0) or the MFMA layout
 * (mfma_layout = 1). Both give the same bits. Replaces the reference's w4_dequant (csrc/w4_gemv.cu:517-540), i.e.
 * ops.dequant (lowbit/ops.py:126-135). */
int lowbit_w4_dequant(const void* w, const void* s, void* out, int64_t N, int64_t K, int64_t group, int mfma_layout,
                      void* stream);

/* GPU quantizer: W [N, K] (float32, float16 or bfloat16 by w_dtype) -> packed canonical u8 [N, K/2] + fp16 scales
 * [N, K/G]. clip_grid (HOST array of n_clip floats, may be NULL with n_clip = 0): per group, try
 * scale = f16(f32(amax * a) / 7) for each a and keep the strictly smallest squared error (first wins ties); with
 * no grid the result is bit-identical to the canonical absmax quantizer. Replaces the reference's
 * ops.quantize_w4_gpu (lowbit/ops.py:81-116), which is torch code there. n_clip <= 64. */
int lowbit_w4_quantize(const void* w, int w_dtype, void* packed, void* scales, int64_t N, int64_t K, int64_t group,
                       const float* clip_grid, int n_clip, void* stream);

/* Device relayout of packed weights: src canonical [N, K/2] -> dst in `layout` (LOWBIT_LAYOUT_V3 or
 * LOWBIT_LAYOUT_MFMA; dst must not alias src). Replaces the host-side numpy interleave + copy the reference does in
 * W4Weight (lowbit/ops.py:42-44, quant.interleave_for_gpu / interleave_for_mma). */
int lowbit_w4_relayout(const void* src, void* dst, int64_t N, int64_t K, int layout, void* stream);

/* ---- decode-step fusions (no counterpart in the reference's extension; they replace the torch modules around the
 * projections of a Qwen2 decoder layer, so that a graph-captured decode step issues ~9 launches per layer) ---- */

#define LOWBIT_EPI_STORE 0     /* y = fp16(acc) */
#define LOWBIT_EPI_BIAS 1      /* y = fp16(acc) + aux[n]                     (aux: bias [N]) */
#define LOWBIT_EPI_RESIDUAL 2  /* y = aux[m][n] + fp16(acc)                  (aux: residual [M][N]; may equal y) */
#define LOWBIT_EPI_SILU_MUL 3  /* rows interleaved 8 gate / 8 up per 16-row tile; y [M][N/2] = silu(gate) * up */

/* A W4A16 projection on the MFMA layout with its consumer fused into the store: 1 <= M <= 64 (M = 1 runs the GEMV,
 * otherwise the MFMA GEMM; workspace as for lowbit_w4_gemm_mfma). Each mode rounds as the unfused torch ops do
 * (the projection to fp16 first; silu in fp32 then fp16, the product fp16), so results equal the unfused sequence
 * (nn.Linear bias add of the reference's W4Linear, lowbit/model.py:25-26; the residual add and silu(gate) * up of
 * transformers' Qwen2 layer). norm_weight (may be NULL; 16-byte aligned; K <= 16384 at M = 1, K <= 8192 at M >= 2): project
 * lowbit_rmsnorm(x, norm_weight, eps) instead of x, the norm computed in the kernel's prologue with lowbit_rmsnorm's
 * per-element arithmetic; for 2..64 rows each row's sum of squares is also added in lowbit_rmsnorm's order (the same
 * bits as lowbit_rmsnorm followed by the projection), for one row in the GEMV's own order (1 / RMS may differ from
 * lowbit_rmsnorm's in its last bit). */
int lowbit_w4_linear_fused(const void* x, const void* w, const void* s, void* y, int64_t M, int64_t N, int64_t K,
                           int64_t group, int epilogue, const void* aux, const void* norm_weight, float eps,
                           void* workspace, size_t workspace_bytes, void* stream);

/* Prefill GEMM, any M >= 1 (meant for M > 64): y [M, N] = x [M, K] . dequant(W)^T on the MFMA layout (K and group
 * multiples of 128), reading the int4 weights directly, with the same epilogues as lowbit_w4_linear_fused. Replaces
 * the reference's prefill path, dequantize to fp16 + cuBLAS (lowbit/ops.py:126-135,163-178): the weights multiplied
 * are exactly the dequantized fp16 values. The workspace (optional, as for lowbit_w4_gemm_mfma: counters zeroed before
 * the first call and left zero) lets K split across workgroups when the tiles alone do not fill the GPU; partial sums
 * take S * M * N * 4 bytes after the counters, and the split count is lowered to what fits. Requires
 * (M + 128) * K * 2 < 2^31. */
int lowbit_w4_gemm_prefill(const void* x, const void* w, const void* s, void* y, int64_t M, int64_t N, int64_t K,
                           int64_t group, int epilogue, const void* aux, void* workspace, size_t workspace_bytes,
                           void* stream);

/* out[M][H] = weight * fp16(x / sqrt(mean(x^2) + eps)) (fp16 in/out, fp32 statistics; transformers Qwen2RMSNorm). */
int lowbit_rmsnorm(const void* x, const void* weight, void* out, int64_t M, int64_t H, float eps, void* stream);

/* RoPE (rotate-half, head_dim 128, angle = positions[m] * inv_freq[i] in fp32) on the q and k heads of a fused qkv
 * projection output [M][(Hq + 2 Hkv) * 128]; rotated q -> q_out [M][Hq][128]; rotated k and v -> k_cache, v_cache
 * [Hkv][L][128] at row positions[m] (device int64; rows outside 0..L-1 are not written). permuted != 0: qkv holds
 * each head's 128 values in the RoPE-permuted order of lowbit_w4_qkv_rope (row 16 (d / 8) + d % 8 for dim d < 64,
 * that row + 8 for dim d + 64). */
int lowbit_rope_kv(const void* qkv, const int64_t* positions, const float* inv_freq, void* q_out, void* k_cache,
                   void* v_cache, int64_t M, int64_t Hq, int64_t Hkv, int64_t L, int permuted, void* stream);

/* One decode token's q|k|v projection with RoPE and the cache write fused into its store (no counterpart in the
 * reference; it replaces lowbit_w4_linear_fused(LOWBIT_EPI_BIAS) followed by lowbit_rope_kv). The weight's rows are
 * permuted per 128-row head so that 16-row tile j holds dims 8 j .. 8 j + 7 and 64 + 8 j .. 64 + 8 j + 7 (rope_kv's
 * permuted layout); bias [N] in the same order. x [1, K]: the layer input, normalized first when norm_weight is given
 * (RMSNorm, as lowbit_w4_linear_fused). q -> q_out [Hq][128]; k, v -> k_cache / v_cache [Hkv][L][128] at row
 * positions[0] (device int64; outside 0..L-1 nothing is written). The same bits as the unfused pair. */
int lowbit_w4_qkv_rope(const void* x, const void* w, const void* s, int64_t N, int64_t K, int64_t group,
                       const void* bias, const void* norm_weight, float eps, const int64_t* positions,
                       const float* inv_freq, void* q_out, void* k_cache, void* v_cache, int64_t Hq, int64_t Hkv,
                       int64_t L, void* stream);

/* lowbit_w4_linear_fused for one row over an fp16 weight w [N, K] (row-major, 16-byte aligned; K % 128 == 0, at
 * most 16384): the W4A16 decode's fp16 comparator, with the same kernel structure, epilogues (store, bias, residual,
 * silu-mul on 8 / 8 interleaved rows) and fused input RMSNorm, so that the two differ only in the weight bytes they
 * stream. fp16 products summed in fp32. No counterpart in the reference, whose fp16 baseline is cuBLAS through
 * F.linear (bench/e2e.py:84-147). */
int lowbit_f16_linear_fused(const void* x, const void* w, void* y, int64_t N, int64_t K, int epilogue,
                            const void* aux, const void* norm_weight, float eps, void* stream);

/* lowbit_w4_qkv_rope over an fp16 q|k|v weight [N, K] in the same RoPE-permuted row order: the fp16 comparator of the
 * fused decode's first projection. No counterpart in the reference. */
int lowbit_f16_qkv_rope(const void* x, const void* w, int64_t N, int64_t K, const void* bias, const void* norm_weight,
                        float eps, const int64_t* positions, const float* inv_freq, void* q_out, void* k_cache,
                        void* v_cache, int64_t Hq, int64_t Hkv, int64_t L, void* stream);

/* The RoPE factors of a step (no counterpart in the reference; the angles of lowbit_rope_kv evaluated once per step
 * instead of once per head and layer): table [M][64] of fp16 pairs (cos, sin) of positions[m] * inv_freq[i] (fp32
 * angle, cos and sin in fp32 rounded to fp16, as lowbit_rope_kv computes them). */
int lowbit_rope_table(const int64_t* positions, const float* inv_freq, void* table, int64_t M, void* stream);

/* lowbit_w4_qkv_rope for M >= 1 tokens (a multi-token step or a prompt; no counterpart in the reference; it replaces
 * lowbit_w4_linear_fused / lowbit_w4_gemm_prefill with LOWBIT_EPI_BIAS followed by lowbit_rope_kv). x [M, K] is
 * the layer input, normalized here when norm_weight is given (RMSNorm(x) * norm_weight with lowbit_rmsnorm's
 * arithmetic, each row's 1 / RMS over all of K; up to 64 rows, K <= 8192, the weight 16-byte aligned; NULL: x is
 * already normalized); token m's q -> q_out [M][Hq][128], its k and v -> the caches' row positions[m];
 * rope_table is lowbit_rope_table's output for these positions. Up to 64 rows run the MFMA GEMM, more the prefill
 * GEMM; the workspace is that kernel's (as lowbit_w4_gemm_mfma or lowbit_w4_gemm_prefill; NULL = no K split). The
 * same bits as the unfused pair; more than 64 rows require (M + 128) * K * 2 < 2^31; the table 16-byte aligned,
 * bias, q_out and the caches 8-byte aligned. */
int lowbit_w4_qkv_rope_rows(const void* x, const void* w, const void* s, int64_t M, int64_t N, int64_t K,
                            int64_t group, const void* bias, const int64_t* positions, const void* rope_table,
                            void* q_out, void* k_cache, void* v_cache, int64_t Hq, int64_t Hkv, int64_t L,
                            const void* norm_weight, float eps,
                            void* workspace, size_t workspace_bytes, void* stream);

/* Causal GQA attention: out[M][Hq * 128] for queries q [M][Hq][128] at positions[m] over cache rows 0..positions[m]
 * (at most L); scores scaled by `scale`, softmax and P.V in fp32. Cache rows past the largest position of the call
 * are never read into a result (they may hold anything, NaN included); rows up to it must be finite, since a
 * multi-token step reads whole 32-key blocks up to the largest position of the rows it groups. max_keys: an upper bound on positions[m] + 1 over
 * the calls that will run (sizes the launch; a captured graph keeps it; keys past it are still attended, by the last
 * key partition). Hq / Hkv in {1, 2, 4, 6, 7, 8}. workspace (optional, 16-byte aligned, at least 4096 bytes, no
 * initial contents needed; its first 4096 bytes are not used -- version 0.2 kept arrival counters there and needed
 * them zero): when there are too few (token, head group) blocks to fill the GPU and max_keys >= 512, the keys are
 * split into partitions whose fp32 partial softmax sums (blocks x partitions x (2 + 128) x 4 bytes after the first
 * 4096, at most workspace_bytes; steps with at least 32 query rows per KV head: 16-row tiles x partitions x
 * (2 + 128) x 4) a second launch merges in partition order; the same bits on every call for a given launch. NULL = no
 * split. Calls that overlap on one workspace race. */
int lowbit_attention(const void* q, const void* k_cache, const void* v_cache, const int64_t* positions, void* out,
                     int64_t M, int64_t Hq, int64_t Hkv, int64_t L, int64_t max_keys, float scale, void* workspace,
                     size_t workspace_bytes, void* stream);

/* One decoded token's attention and its output projection in two launches: y [1, N] = epilogue(attn [1, Hq * 128] .
 * W^T) with attn what lowbit_attention computes for M = 1 (the same q, caches, positions, max_keys and scale), W the
 * int4 MFMA-layout weight [N, Hq * 128] with its scales (group: a multiple of 128) or, for the _f16_ variant, an fp16
 * weight [N, Hq * 128] row-major; epilogue and aux as in lowbit_w4_linear_fused (aux may be y for the residual). The
 * attention keeps at most 8 key partitions and leaves their partial softmax sums in the workspace; the projection's
 * prologue merges them into its x in partition order, the attention's own merge, so y has the bits of lowbit_attention
 * (with a workspace that holds at most the same partitions) followed by lowbit_w4_linear_fused / lowbit_f16_linear_fused
 * at M = 1 -- one launch fewer, and the attention output never written. Hq <= 32, Hq / Hkv in {1, 2, 4, 6, 7, 8};
 * workspace required: 16-byte aligned, at least 4096 + Hq * 132 * 4 bytes, no initial contents (the partials, P x Hq
 * x 132 x 4 bytes, follow its first 4096). No counterpart in the reference (its decoder runs torch attention, then
 * W4Linear); it serves the fused decoder's one-token step. */
int lowbit_w4_attention_linear(const void* q, const void* k_cache, const void* v_cache, const int64_t* positions,
                               int64_t Hq, int64_t Hkv, int64_t L, int64_t max_keys, float scale, const void* w,
                               const void* s, void* y, int64_t N, int64_t group, int epilogue, const void* aux,
                               void* workspace, size_t workspace_bytes, void* stream);
int lowbit_f16_attention_linear(const void* q, const void* k_cache, const void* v_cache, const int64_t* positions,
                                int64_t Hq, int64_t Hkv, int64_t L, int64_t max_keys, float scale, const void* w,
                                void* y, int64_t N, int epilogue, const void* aux, void* workspace,
                                size_t workspace_bytes, void* stream);

/* fp16 GEMV for the tied fp16 lm_head of a decode step (or the last row of a prefill): y [M, N] = fp16(x [M, K] . W^T)
 * with W fp16 [N, K] row-major, fp32 accumulation, 1 <= M <= 64, K % 8 == 0 (K % 128 == 0 beyond 16 rows or where
 * M * K * 2 > 65536), x and W 16-byte
 * aligned. No counterpart in the reference (its head is torch.nn.functional.linear, cuBLAS); it replaces that call
 * in the fused decoder, where hipBLASLt streams the 622 MB Qwen2.5-3B head at ~3 TB/s. */
int lowbit_f16_gemv(const void* x, const void* w, void* y, int64_t M, int64_t N, int64_t K, void* stream);

/* lowbit_f16_gemv for one row followed by the greedy pick and its feedback (replaces the reference harness's
 * lg.argmax(-1) and the copy that feeds the pick back as the next step's input, bench/e2e.py:93-95): y [1, N] as
 * lowbit_f16_gemv writes it, then tokens[0] = the index of the largest of y as torch.argmax picks it (the first of
 * equal maxima, -0 equal to +0, a NaN above every number) and positions[0] += 1 (positions may be NULL); with
 * out_tokens and out_count (both or neither), out_tokens[*out_count] = the pick while *out_count < out_capacity, then
 * *out_count += 1; with embed (the tied embedding [N, K], 16-byte aligned) and h_out (both or neither), h_out [K] =
 * the pick's embedding row, the next step's input (replaces the reference harness's embedding lookup of the fed-back
 * token). Two launches, no allocation and no memset, so a decode step may capture it; workspace (8-byte aligned) holds
 * a 64-bit key per head workgroup, 8 * ceil(N / 8) bytes, and needs no initial contents. */
int lowbit_f16_gemv_pick(const void* x, const void* w, void* y, int64_t N, int64_t K, void* workspace,
                         size_t workspace_bytes, int64_t* tokens, int64_t* positions, int64_t* out_tokens,
                         int64_t out_capacity, int32_t* out_count, const void* embed, void* h_out, void* stream);

/* ---- HBM bandwidth probes (the measured peak that kernel bandwidths are quoted against) ----
 * The reference measures its peak with a torch device copy and a torch sum over 256 MiB (bench/gpu_run.py:133-141);
 * these are streaming kernels of this library for the same two figures. hbm_read reads `bytes` (a multiple of 16,
 * 16-byte aligned source) with 16-byte loads over `blocks` workgroups of 256 threads and writes at most one 32-bit
 * word to `sink`; hbm_copy copies `bytes` from src to dst. */
int lowbit_hbm_read(const void* src, int64_t bytes, void* sink, int64_t blocks, void* stream);
int lowbit_hbm_copy(const void* src, void* dst, int64_t bytes, int64_t blocks, void* stream);

/* ---- host-side format functions (CPU memory, no GPU needed); counterparts of lowbit/quant.py ---- */

/* quant.quantize_w4 (lowbit/quant.py:23-35): w float32 [N, K] -> packed [N, K/2], scales fp16 bits [N, K/G]. */
int lowbit_host_quantize(const float* w, uint8_t* packed, uint16_t* scales, int64_t N, int64_t K, int64_t group);
/* quant.unpack_w4 (lowbit/quant.py:38-44): packed [N, K/2] (canonical) -> int8 [N, K] in -8..7. */
int lowbit_host_unpack(const uint8_t* packed, int8_t* out, int64_t N, int64_t K);
/* quant.dequantize_w4 (lowbit/quant.py:47-51): float32 [N, K] = (u - 8) * scale. */
int lowbit_host_dequantize(const uint8_t* packed, const uint16_t* scales, float* out, int64_t N, int64_t K,
                           int64_t group);
/* quant.interleave_for_gpu / interleave_for_mma (lowbit/quant.py:55-78) and this library's MFMA layout:
 * canonical src [N, K/2] -> dst in layout (V3, NV_MMA = the reference's m16n8k8 fragment order, or MFMA). */
int lowbit_host_relayout(const uint8_t* src, uint8_t* dst, int64_t N, int64_t K, int layout);
/* quant.gemv_reference (lowbit/quant.py:81-84): y float64 [M, N] = x float64 [M, K] . dequant(W)^T. */
int lowbit_host_gemv_reference(const double* x, const uint8_t* packed, const uint16_t* scales, double* y, int64_t M,
                               int64_t N, int64_t K, int64_t group);

#ifdef __cplusplus
}
#endif

#endif /* LOWBIT_W4_H */
