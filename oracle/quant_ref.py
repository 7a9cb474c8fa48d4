"""CPU oracle for the W4A16 path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker or as the timed CPU baseline. The product (lowbit-kernels_amd/lowbit) never imports it.

It restates, in numpy, the reference's format and CPU arithmetic for the W4A16 linear:
  * the format (reference lowbit/quant.py:1-84): symmetric int4, one fp16 scale per G-group along K, two nibbles
    per byte, low nibble = even k; the v3 word order and the mma (NVIDIA m16n8k8) regroup; the fp64 GEMV;
  * the GPU quantizer's clip search (reference lowbit/ops.py:81-116), restated in float32 numpy;
  * the fp16 dequant rule, rounded once (reference lowbit/ops.py:119-123, csrc/w4_gemv.cu:296-310);
  * the harness's error metric and known answers (reference bench/gpu_run.py:144-159,177,231-245).
It also states this build's own gfx950 device layout (`interleave_for_mfma`), which has no reference
counterpart, so that tests can check the device relayout byte for byte.

How each function is pinned (tests/test_oracle.py): the reference's known-answer tests
(tests/test_quant.py:24-30,71-76,96-108), closed-form invariants (error <= half a step, permutation, range),
brute force on tiny inputs, and the committed fixtures in tests/golden/. The clip search has no reference
vector: it is pinned by invariants only (chosen scale is a grid candidate, its error is minimal within fp32
summation tolerance, ties keep the earliest candidate, an empty grid reproduces absmax bit for bit).
"""
import numpy as np

QMIN, QMAX, OFFSET = -8, 7, 8          # reference lowbit/quant.py:20

# nibble slot s of a little-endian 32-bit word holds value k0 + SLOT_TO_K[s] (reference lowbit/quant.py:54-55)
SLOT_TO_K = np.array([0, 2, 4, 6, 1, 3, 5, 7])
# byte 16t + s of a 64-byte chunk holds canonical byte 4s + t (reference lowbit/quant.py:67-68)
MMA_BYTE_ORDER = np.array([4 * s + t for t in range(4) for s in range(16)])

# the harness's clip grid 1.00, 0.975, ..., 0.75 (reference bench/e2e.py:30)
CLIP_GRID = tuple(round(1.0 - 0.025 * i, 3) for i in range(11))
# normalized max error bound (reference bench/gpu_run.py:179,245)
REL_BOUND = 3e-3


def quantize_w4(w, group=128):
    """W [N, K] -> (packed u8 [N, K/2], scales f16 [N, K/G]). Reference lowbit/quant.py:23-35."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % group or group % 32:
        raise ValueError(f"K={k} must be a multiple of the group size {group}, itself a multiple of 32")
    g = w.reshape(n, k // group, group)
    amax = np.abs(g).max(axis=2)
    scale = (amax / np.float32(QMAX)).astype(np.float16)         # fp32 division, then one rounding to fp16
    scale[scale == 0] = np.float16(1.0)
    q = np.clip(np.rint(g / scale.astype(np.float32)[..., None]), QMIN, QMAX).astype(np.int8)
    u = (q.reshape(n, k) + OFFSET).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8), scale


def unpack_w4(packed):
    """packed u8 [N, K/2] -> int8 [N, K] in -8..7. Reference lowbit/quant.py:38-44."""
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty((packed.shape[0], packed.shape[1] * 2), dtype=np.int8)
    out[:, 0::2] = (packed & 0x0F).astype(np.int8) - OFFSET
    out[:, 1::2] = (packed >> 4).astype(np.int8) - OFFSET
    return out


def dequantize_w4(packed, scales, group=128):
    """(u - 8) * scale in float32, exact. Reference lowbit/quant.py:47-51."""
    q = unpack_w4(packed).astype(np.float32)
    n, k = q.shape
    return (q.reshape(n, k // group, group) * np.asarray(scales, np.float32)[..., None]).reshape(n, k)


def dequantize_w4_f16(packed, scales, group=128):
    """The fp16 weights every dequant kernel must write: the exact product rounded once to fp16.
    Reference lowbit/ops.py:119-123 (fp32 product, .half()) and bench/gpu_run.py:217-224 (== fp64 rounded)."""
    return dequantize_w4(packed, scales, group).astype(np.float16)


def interleave_for_gpu(packed):
    """Canonical -> v3 word order. Reference lowbit/quant.py:58-64."""
    u = unpack_w4(packed) + OFFSET
    n, k = u.shape
    words = u.reshape(n, k // 8, 8)[:, :, SLOT_TO_K].reshape(n, k).astype(np.uint8)
    return (words[:, 0::2] | (words[:, 1::2] << 4)).astype(np.uint8)


def interleave_for_mma(packed):
    """Canonical -> the NVIDIA m16n8k8 fragment layout (chunk regroup, then v3 order). Reference
    lowbit/quant.py:71-78."""
    packed = np.asarray(packed, dtype=np.uint8)
    n, half_k = packed.shape
    if half_k % 64:
        raise ValueError(f"K={2 * half_k} must be a multiple of 128 for the tensor-core layout")
    regrouped = packed.reshape(n, half_k // 64, 64)[:, :, MMA_BYTE_ORDER].reshape(n, half_k)
    return interleave_for_gpu(regrouped)


def interleave_for_mfma(packed):
    """Canonical -> this build's gfx950 device layout (no reference counterpart; stated here so tests can check the
    device relayout). Rows form 16-row tiles (the last tile holds N % 16 rows when N is not a multiple of 16).
    Tile t starts at byte 16 t K/2. Inside it, 128-k chunk c occupies rows_t * 64 bytes at offset c * rows_t * 64,
    and row r of the tile holds that chunk's 64 canonical bytes at offset 64 r, each 32-bit word in v3 order.
    So one 1 KB block is 16 rows x 128 k, and a 16-byte piece is 32 consecutive k of one row."""
    packed = np.asarray(packed, dtype=np.uint8)
    n, half_k = packed.shape
    if half_k % 64:
        raise ValueError(f"K={2 * half_k} must be a multiple of 128 for the MFMA layout")
    v3 = interleave_for_gpu(packed)
    out = np.empty(n * half_k, dtype=np.uint8)
    chunks = half_k // 64
    for t0 in range(0, n, 16):
        rows = min(16, n - t0)
        tile = v3[t0:t0 + rows].reshape(rows, chunks, 64).transpose(1, 0, 2)     # [chunk, row, 64 B]
        out[t0 * half_k:(t0 + rows) * half_k] = tile.reshape(-1)
    return out.reshape(n, half_k)


def gemv_reference(x, packed, scales, group=128):
    """y = x_f64 @ dequant_f64^T. Reference lowbit/quant.py:81-84."""
    w = dequantize_w4(packed, scales, group).astype(np.float64)
    return np.asarray(x, np.float64) @ w.T


def quantize_w4_clip(w, group=128, clip_grid=None):
    """Restatement of the GPU quantizer with the per-group clip search, reference lowbit/ops.py:81-116, in float32:
    for each grid value a, sc = f16(f32(amax * a) / 7) (a == 1: f16(amax / 7)); sc == 0 -> 1;
    q = clamp(round_half_even(g / sc), -8, 7); err = sum((q * sc - g)^2) in float32; a candidate replaces the best
    only when strictly better. clip_grid=None reproduces quantize_w4 bit for bit.
    Returns (packed, scales, chosen grid index [N, K/G], errs [len(grid), N, K/G] float32)."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % group or group % 32:
        raise ValueError(f"K={k} must be a multiple of the group size {group}, itself a multiple of 32")
    g = w.reshape(n, k // group, group)
    amax = np.abs(g).max(axis=2)
    grid = tuple(clip_grid) if clip_grid else (1.0,)
    best_s = best_q = best_e = None
    best_i = np.zeros(amax.shape, np.int32)
    errs = []
    for i, a in enumerate(grid):
        num = amax * np.float32(a) if a != 1.0 else amax
        sc = (num.astype(np.float32) / np.float32(QMAX)).astype(np.float16)
        sc[sc == 0] = np.float16(1.0)
        scf = sc.astype(np.float32)[..., None]
        q = np.clip(np.rint(g / scf), QMIN, QMAX).astype(np.float32)
        err = ((q * scf - g) ** 2).sum(-1, dtype=np.float32)
        errs.append(err)
        if best_e is None:
            best_s, best_q, best_e = sc, q, err
        else:
            better = err < best_e
            best_s = np.where(better, sc, best_s)
            best_q = np.where(better[..., None], q, best_q)
            best_i = np.where(better, i, best_i)
            best_e = np.minimum(err, best_e)
    u = (best_q.reshape(n, k) + OFFSET).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8), best_s, best_i, np.stack(errs)


def rel_err(y, ref):
    """max|y - ref| / RMS(ref), the harness's metric (reference bench/gpu_run.py:177,231-243)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.sqrt(np.mean(ref ** 2))
    return float(np.abs(y - ref).max() / scale) if ref.size else 0.0


# known answers of the overflow regression (reference bench/gpu_run.py:144-159): q = 7 everywhere (byte 0xFF),
# scale 2^-10, one group of K = 128, N = 16; x = 4096 gives 3584 and x = -8192 gives -7168, within 2
OVERFLOW_CASE = {"k": 128, "n": 16, "byte": 0xFF, "scale": 2.0 ** -10, "answers": ((4096.0, 3584.0), (-8192.0, -7168.0)),
                 "tol": 2.0}


def dequantize_w4_torch(packed, scales, group=128):
    """The reference's torch dequantize (lowbit/ops.py:119-123), restated for the CPU baseline: each nibble as a float32
    u - 8, times its group's scale in float32, rounded once to fp16 -> torch fp16 [N, K]. Runs on torch's CPU kernels
    (all of torch's threads), as the reference's CPU path does; bit-identical to dequantize_w4_f16."""
    import torch
    p = torch.as_tensor(np.ascontiguousarray(packed))
    s = torch.as_tensor(np.ascontiguousarray(scales))
    n, half_k = p.shape
    u = torch.empty(n, 2 * half_k, dtype=torch.float32)
    u[:, 0::2] = p & 0xF
    u[:, 1::2] = p >> 4
    u -= OFFSET
    return (u.view(n, -1, group) * s.float().unsqueeze(-1)).view(n, 2 * half_k).half()


def cpu_torch_linear(x16, packed, scales, group=128):
    """One layer of the reference's CPU torch path after quantization: dequantize_w4_torch, then
    torch.nn.functional.linear on fp16 (reference lowbit/ops.py:119-123,178)."""
    import torch
    return torch.nn.functional.linear(torch.as_tensor(x16), dequantize_w4_torch(packed, scales, group))
