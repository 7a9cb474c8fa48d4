"""PyTorch side of the gfx950 kernels: hold quantized weights on the GPU and dispatch decode vs prefill.

Same public surface and semantics as the reference's lowbit/ops.py (names, arguments, defaults, row limits, error
types and messages); every kernel call goes to liblowbit_w4.so through `ext()`. There is no CPU or torch fallback
for a kernel: without the built library, `ext()` raises.

Kernel versions keep the reference's numbering (lowbit/ops.py:57-59):
  1, 2  GEMV on the canonical layout (one gfx950 kernel serves both)       M <= 8
  3, 4  GEMV on the v3 layout (one gfx950 kernel serves both)              M <= 8
  5     MFMA skinny GEMM on the device ("mma") layout                      M <= 64
  6     bandwidth GEMV on the device ("mma") layout, the M = 1 decode path M <= 8
"""
import torch

from . import _native

_EXT = None


def ext():
    """The native extension object (w4_gemv, w4_gemm_tc, w4_dequant, w4_quantize, w4_relayout), loaded once.
    Reference lowbit/ops.py:12-18 (there a JIT nvcc build; here the in-tree hipcc build)."""
    global _EXT
    if _EXT is None:
        _EXT = _native.NativeExt()
    return _EXT


LAYOUTS = ("canonical", "v3", "mma")


def _to_device_u8(a, device):
    t = a if isinstance(a, torch.Tensor) else torch.from_numpy(a)
    return t.to(device=device, dtype=torch.uint8).contiguous()


def _to_device_f16(a, device):
    t = a if isinstance(a, torch.Tensor) else torch.from_numpy(a)
    if t.dtype != torch.float16:
        raise ValueError("scales must be float16")
    return t.to(device=device).contiguous()


class W4Weight:
    """One linear layer's weight in the lowbit.quant format, on the GPU (reference lowbit/ops.py:24-54).
    `layouts` picks which copies to keep: canonical (v1, v2, dequantize), v3 (v3, v4), mma = the gfx950 device layout
    (v5, v6, dequantize; needs K and the group size to be multiples of 128). None = every layout this shape supports;
    a model keeps ("mma",). Prefill dequantizes, so one of canonical / mma must be kept.

    `packed` / `scales` may be numpy arrays or tensors (CPU or CUDA) in the canonical layout; the v3 and mma copies
    are produced on the GPU by the native relayout kernel (no host round trip)."""

    def __init__(self, packed, scales, group, layouts=None, device="cuda"):
        self.group = group
        self.n, self.k = packed.shape[0], packed.shape[1] * 2
        mma_ok = self.k % 128 == 0 and group % 128 == 0
        if layouts is None:
            layouts = LAYOUTS if mma_ok else ("canonical", "v3")
        if not set(layouts) <= set(LAYOUTS):
            raise ValueError(f"unknown layout in {layouts}; choose from {LAYOUTS}")
        if "mma" in layouts and not mma_ok:
            raise ValueError(f"the mma layout needs K and the group size to be multiples of 128 (K={self.k}, G={group})")
        if "canonical" not in layouts and "mma" not in layouts:
            raise ValueError("keep the canonical or the mma layout: prefill dequantizes from one of them")
        if device == "cuda" or (isinstance(device, torch.device) and device.type == "cuda" and device.index is None):
            device = torch.device("cuda", torch.cuda.current_device())
        canonical = _to_device_u8(packed, device)
        self.scales = _to_device_f16(scales, device)
        e = ext()
        self.packed_v3 = e.w4_relayout(canonical, _native.LAYOUT_V3) if "v3" in layouts else None
        self.packed_mma = e.w4_relayout(canonical, _native.LAYOUT_MFMA) if "mma" in layouts else None
        self.packed = canonical if "canonical" in layouts else None

    @classmethod
    def from_float(cls, w, group=128, layouts=None):
        """Quantize on the GPU (native quantizer, bit-identical to quant.quantize_w4) and keep `layouts`."""
        packed, scales = quantize_w4_gpu(w, group)
        return cls(packed, scales, group, layouts, device=packed.device)

    def nbytes(self):
        """Bytes of one copy of the weight (packed values + scales), whatever layouts are kept."""
        return self.n * self.k // 2 + self.scales.numel() * 2


def pick_rows(n, m):
    """Rows per wave the row-major GEMVs (v1-v4) use when rows_per_warp = 0 (mirror of the native choice)."""
    return 4 if n >= 512 else 2 if m >= 4 else 1


# the layout each kernel version reads, and the most rows it takes (reference lowbit/ops.py:57-59)
NEEDS = {1: "packed", 2: "packed", 3: "packed_v3", 4: "packed_v3", 5: "packed_mma", 6: "packed_mma"}
MAX_ROWS = {1: 8, 2: 8, 3: 8, 4: 8, 5: 64, 6: 8}


def gemv(x, wq, version=4, rows_per_warp=0):
    """x [M, K] fp16 -> [M, N] fp16. v1-v4, v6: M <= 8 (rows_per_warp: rows per wave for v1-v4, 16-row tiles per
    wave for v6; 0 = chosen from N and M); v5: MFMA, M <= 64 (rows_per_warp = 16-row tiles per wave, 1/2/4, 0 =
    chosen). v5 and v6 read the same device layout (packed_mma), so a model needs only that copy."""
    if version not in NEEDS:
        raise ValueError(f"version must be one of {sorted(NEEDS)}")
    if getattr(wq, NEEDS[version]) is None:
        raise ValueError(f"v{version} reads {NEEDS[version]}, which this W4Weight does not keep")
    if version == 5:
        return ext().w4_gemm_tc(x.contiguous(), wq.packed_mma, wq.scales, wq.group, rows_per_warp)
    w = wq.packed_mma if version == 6 else wq.packed_v3 if version >= 3 else wq.packed
    return ext().w4_gemv(x.contiguous(), w, wq.scales, wq.group, version, rows_per_warp)


def quantize_w4_gpu(w, group=128, clip_grid=None, rows_per_pass=2048):
    """Same format and, with clip_grid=None, the same bits as quant.quantize_w4, computed by the native GPU
    quantizer. clip_grid, e.g. (1.0, 0.975, ..., 0.75): per group, try scale = fp16(fp32(amax * a) / 7) for each a
    and keep the strictly smallest squared weight error (ties keep the earlier a). A CPU input moves to the GPU
    `rows_per_pass` rows at a time. Returns (packed uint8 [N, K/2], scales fp16 [N, K/G]) on the GPU.
    Reference lowbit/ops.py:81-116."""
    n, k = w.shape
    if k % group or group % 32:
        raise ValueError(f"K={k} must be a multiple of the group size {group}, itself a multiple of 32")
    w = w.detach()
    if w.is_cuda:
        return ext().w4_quantize(w, group, clip_grid)
    dev = torch.device("cuda", torch.cuda.current_device())
    packed = torch.empty(n, k // 2, dtype=torch.uint8, device=dev)
    scales = torch.empty(n, k // group, dtype=torch.float16, device=dev)
    for r0 in range(0, n, rows_per_pass):
        p, s = ext().w4_quantize(w[r0:r0 + rows_per_pass].to(dev), group, clip_grid)
        packed[r0:r0 + rows_per_pass] = p
        scales[r0:r0 + rows_per_pass] = s
    return packed, scales


def dequantize_w4_gpu(packed, scales, group=128):
    """fp16 [N, K]: (u - 8) * scale rounded once to fp16, from canonical packed weights (what the dequantize kernel
    writes). CUDA tensors run the native dequant kernel; CPU tensors use the library's host code (same bits).
    Reference lowbit/ops.py:119-123."""
    if packed.is_cuda:
        return ext().w4_dequant(packed.contiguous(), scales.contiguous(), group)
    from . import quant
    return torch.from_numpy(quant.dequantize_w4(packed.numpy(), scales.numpy(), group)).half()


def dequant(wq, layout=None):
    """fp16 W [N, K] from the canonical or the mma copy (None: canonical when kept). Both give the same bits."""
    if layout is None:
        layout = "canonical" if wq.packed is not None else "mma"
    if layout == "canonical" and wq.packed is not None:
        return ext().w4_dequant(wq.packed, wq.scales, wq.group)
    if layout == "mma" and wq.packed_mma is not None:
        return ext().w4_dequant(wq.packed_mma, wq.scales, wq.group, True)
    raise ValueError(f"cannot dequantize from the {layout} layout: not kept")


# version 0 (auto) picks by batch size and layer width. The structure is the reference's (lowbit/ops.py:137-160):
# the v6 GEMV up to AUTO_GEMV_ROWS rows; the MFMA kernel (v5) up to AUTO_V5_ROWS rows on every layer and up to
# AUTO_V5_WIDE_ROWS rows on layers with N >= AUTO_WIDE_N; dequantize + BLAS beyond. The constants come from MI355X
# sweeps (graph-timed, weights cycled through >= 1 GiB, M in 1..64 on the Qwen2.5-1.5B/3B/7B projections): from M = 2
# to 64 the MFMA kernel beats dequantize + hipBLASLt 2-6x and fp16 hipBLASLt on every shape, so the v5 width split of
# the reference's rule (which came from a T4) no longer matters. The GEMV, which spends ALU per activation row, keeps
# M = 2 and 3 on layers narrower than AUTO_GEMV_NARROW_N with K <= AUTO_GEMV_MAX_K (11008 x 2048, M = 2: 6.7 us vs
# 11.5; q / o / k / v: 3.5-3.9 vs 3.8-4.6 us); wider layers and longer K go to v5 from M = 2 (2048 x 11008, M = 2: 7.0
# vs 6.6 us). With AUTO_GEMV_NARROW_ROWS = AUTO_GEMV_ROWS the rule is exactly the reference's.
AUTO_GEMV_ROWS, AUTO_V5_ROWS, AUTO_V5_WIDE_ROWS, AUTO_WIDE_N = 1, 64, 64, 3072
AUTO_GEMV_NARROW_ROWS, AUTO_GEMV_NARROW_N, AUTO_GEMV_MAX_K = 3, 8192, 16384
# Beyond the MFMA kernel's rows (prefill), a weight on the mma layout goes to the int4-direct prefill GEMM (prefill())
# when K >= AUTO_PREFILL_MIN_K, when M <= AUTO_PREFILL_ROWS, or when M <= AUTO_PREFILL_NARROW_ROWS on a small layer
# (N and K <= AUTO_PREFILL_NARROW); everything else dequantizes (4.4-4.8 TB/s) and calls BLAS. From the MI355X sweep at
# M = 128, 256, 512, 2048 on the Qwen2.5-3B / 7B projections (int4 vs dequantize + hipBLASLt, us): every layer up to
# 512 rows (3B merged gate|up 26.3 vs 45.9 at 128, 72.6 vs 75.9 at 512; 3B down 26.0 vs 38.3 at 128, 49.0 vs 58.4 at
# 512; 7B gate|up 97.8 vs 100.8 at 512), the attention-sized 3B layers up to 2048 rows (o 29.2 vs 31.7, q|k|v 36.9 vs
# 36.6 at 2048) and the long-K 7B down at every M (47 vs 109 at 128, 119 vs 203 at 512, 345 vs 395 at 2048);
# dequantize + hipBLASLt keeps the wide and long layers at 2048 rows (3B gate|up 190 vs 261, 3B down 107 vs 134).
AUTO_PREFILL_MIN_K, AUTO_PREFILL_ROWS = 16384, 512
AUTO_PREFILL_NARROW, AUTO_PREFILL_NARROW_ROWS = 4096, 2048


def gemm_chunked(x, wq, chunk=64):
    """Many rows through v5 in 64-row slices (no fp16 weight copy is written)."""
    return torch.cat([gemv(x[i:i + chunk], wq, 5) for i in range(0, x.shape[0], chunk)])


def auto_version(m, wq):
    """The kernel linear() uses for m rows, or None for dequantize + BLAS. Weights without the mma layout (K or the
    group size not a multiple of 128) use v4 / v2 up to 8 rows."""
    if wq.packed_mma is not None:
        if m <= AUTO_GEMV_ROWS or (m <= AUTO_GEMV_NARROW_ROWS and wq.n < AUTO_GEMV_NARROW_N and wq.k <= AUTO_GEMV_MAX_K):
            return 6
        return 5 if m <= (AUTO_V5_WIDE_ROWS if wq.n >= AUTO_WIDE_N else AUTO_V5_ROWS) else None
    if m <= 8:
        return 4 if wq.packed_v3 is not None else 2 if wq.packed is not None else None
    return None


def prefill(x, wq):
    """x [M, K] times an mma-layout weight with the int4-direct prefill GEMM (any M; fp32 accumulation of exactly the
    dequantized fp16 weights, as dequantize + BLAS computes)."""
    if wq.packed_mma is None:
        raise ValueError("the prefill GEMM reads packed_mma, which this W4Weight does not keep")
    return ext().w4_gemm_prefill(x.contiguous(), wq.packed_mma, wq.scales, wq.group)


def prefill_path(m, wq):
    """True when linear() sends m rows to the int4 prefill GEMM rather than dequantize + BLAS (auto routing only)."""
    if auto_version(m, wq) is not None or wq.packed_mma is None:
        return False
    return (wq.k >= AUTO_PREFILL_MIN_K or m <= AUTO_PREFILL_ROWS
            or (m <= AUTO_PREFILL_NARROW_ROWS and wq.n <= AUTO_PREFILL_NARROW and wq.k <= AUTO_PREFILL_NARROW))


def linear(x, wq, max_gemv_rows=8, version=0, bias=None):
    """Decode (few rows): an INT4 kernel (v6 GEMV for one row, v5 MFMA beyond). Prefill (many rows): dequantize, then
    the fp16 BLAS GEMM (hipBLASLt under PyTorch-ROCm), or the int4 prefill GEMM where prefill_path says (K >=
    AUTO_PREFILL_MIN_K at any M, every layer up to AUTO_PREFILL_ROWS rows, layers with N and K <= AUTO_PREFILL_NARROW
    up to AUTO_PREFILL_NARROW_ROWS rows). version 0 = auto; a fixed version runs up to min(max_gemv_rows, its row
    limit) rows (v5: 64), and dequantize + BLAS above.
    bias ([N], optional; not in the reference's signature; used in fp16 on x's device on every route): y =
    fp16(x W^T) + bias in fp16, the rounding of the reference's linear() followed by `+ bias`; the v5, one-row v6 and prefill kernels add it in their store (no extra
    launch), multi-row v6 and dequantize + BLAS with a separate add."""
    m = x.shape[0]
    if m == 0:
        return x.new_empty(0, wq.n)
    if bias is not None:                      # one bias for every route: fp16 [N] on x's device
        if bias.numel() != wq.n:
            raise ValueError(f"bias must hold N={wq.n} values, got shape {list(bias.shape)}")
        bias = bias.reshape(wq.n).to(device=x.device, dtype=torch.float16).contiguous()
    if version == 0:
        v = auto_version(m, wq)
    elif version in MAX_ROWS:
        v = version if m <= (MAX_ROWS[5] if version == 5 else min(max_gemv_rows, MAX_ROWS[version])) else None
    else:
        raise ValueError(f"version must be 0 (auto) or one of {sorted(MAX_ROWS)}")
    # the fused entry runs the GEMV for one row and the MFMA kernel for more: fuse the bias where that is the kernel
    # the unbiased call would run, so linear(bias=b) stays linear() + b bit for bit
    if bias is not None and (v == 5 or (v == 6 and m == 1)):
        return ext().w4_linear_fused(x.contiguous(), wq.packed_mma, wq.scales, wq.group, _native.EPI_BIAS, bias)
    if v is not None:
        y = gemv(x, wq, v)
    elif version == 0 and prefill_path(m, wq):
        if bias is not None:
            return ext().w4_gemm_prefill(x.contiguous(), wq.packed_mma, wq.scales, wq.group, _native.EPI_BIAS, bias)
        y = prefill(x, wq)
    else:
        y = torch.nn.functional.linear(x, dequant(wq, "mma" if wq.packed_mma is not None else "canonical"))
    return y.add_(bias) if bias is not None else y
