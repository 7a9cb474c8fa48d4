"""Weight-only INT4 format: the public host-side functions of the reference's lowbit/quant.py, same names and
semantics, computed by the native library's host code (lowbit_host_* in liblowbit_format.so, a HIP-free build of
the same functions liblowbit_w4.so exports), bit for bit. No GPU stack is needed to pack weights.

Format (reference lowbit/quant.py:1-17): for an nn.Linear weight W [N, K], one fp16 scale per group of G values
along K, scale = fp16(max|W_group| / 7) (an all-zero group gets 1.0), q = clamp(round_half_even(W / scale), -8, 7),
stored as the nibble u = q + 8, two per byte, low nibble = even k ("canonical").

Layouts of the same bytes:
  * interleave_for_gpu: every 32-bit word in the nibble order [k0, k2, k4, k6, k1, k3, k5, k7] ("v3");
  * interleave_for_mma: the reference's NVIDIA m16n8k8 fragment order (kept for compatibility; no kernel here reads
    it);
  * interleave_for_mfma: this library's gfx950 device layout, the one copy a model keeps (W4Weight's "mma" copy):
    16-row tiles; inside tile t the 128-k chunk c holds rows_t x 64 bytes, row r at offset 64 r, words in v3 order,
    so one 1 KB block is 16 rows x 128 k and lane l of a wave reads 32 consecutive k of one row in one 16-byte load.
"""
import numpy as np

from . import _native

QMIN, QMAX, OFFSET = -8, 7, 8
# nibble slot s (0..7, bit 4s of a little-endian 32-bit word) holds value k0 + SLOT_TO_K[s]
SLOT_TO_K = np.array([0, 2, 4, 6, 1, 3, 5, 7])
# byte position 16t + s of a 64-byte chunk holds canonical byte 4s + t (the reference's m16n8k8 order)
MMA_BYTE_ORDER = np.array([4 * s + t for t in range(4) for s in range(16)])


def _check(rc):
    _native.check(rc, _native.host_lib())


def _u8(packed):
    return np.ascontiguousarray(np.asarray(packed, dtype=np.uint8))


def quantize_w4(w, group=128):
    """W [N, K] float -> (packed uint8 [N, K//2], scales float16 [N, K//group])."""
    w = np.ascontiguousarray(np.asarray(w, dtype=np.float32))
    if w.ndim != 2:
        raise ValueError("W must be 2-D [N, K]")
    n, k = w.shape
    if k % group or group % 32:
        raise ValueError(f"K={k} must be a multiple of the group size {group}, itself a multiple of 32")
    packed = np.empty((n, k // 2), dtype=np.uint8)
    scales = np.empty((n, k // group), dtype=np.float16)
    _check(_native.host_lib().lowbit_host_quantize(_native.np_ptr(w), _native.np_ptr(packed), _native.np_ptr(scales),
                                                     n, k, group))
    return packed, scales


def unpack_w4(packed):
    """packed uint8 [N, K//2] -> signed int8 values [N, K] in -8..7."""
    packed = _u8(packed)
    out = np.empty((packed.shape[0], packed.shape[1] * 2), dtype=np.int8)
    _check(_native.host_lib().lowbit_host_unpack(_native.np_ptr(packed), _native.np_ptr(out), packed.shape[0],
                                                   packed.shape[1] * 2))
    return out


def dequantize_w4(packed, scales, group=128):
    """-> float32 [N, K], exactly what a kernel should multiply by."""
    packed = _u8(packed)
    scales = np.ascontiguousarray(np.asarray(scales, dtype=np.float16))
    n, k = packed.shape[0], packed.shape[1] * 2
    out = np.empty((n, k), dtype=np.float32)
    _check(_native.host_lib().lowbit_host_dequantize(_native.np_ptr(packed), _native.np_ptr(scales),
                                                       _native.np_ptr(out), n, k, group))
    return out


def _relayout(packed, layout):
    packed = _u8(packed)
    out = np.empty_like(packed)
    _check(_native.host_lib().lowbit_host_relayout(_native.np_ptr(packed), _native.np_ptr(out), packed.shape[0],
                                                     packed.shape[1] * 2, layout))
    return out


def interleave_for_gpu(packed):
    """Canonical packed [N, K//2] -> the v3 layout. Bytes per row are unchanged."""
    return _relayout(packed, _native.LAYOUT_V3)


def interleave_for_mma(packed):
    """Canonical packed [N, K//2] -> the reference's m16n8k8 fragment layout. K must be a multiple of 128."""
    packed = _u8(packed)
    if packed.shape[1] % 64:
        raise ValueError(f"K={2 * packed.shape[1]} must be a multiple of 128 for the tensor-core layout")
    return _relayout(packed, _native.LAYOUT_NV_MMA)


def interleave_for_mfma(packed):
    """Canonical packed [N, K//2] -> the gfx950 device layout the kernels read. K must be a multiple of 128."""
    packed = _u8(packed)
    if packed.shape[1] % 64:
        raise ValueError(f"K={2 * packed.shape[1]} must be a multiple of 128 for the MFMA layout")
    return _relayout(packed, _native.LAYOUT_MFMA)


def gemv_reference(x, packed, scales, group=128):
    """y[m, n] = sum_k x[m, k] * dequant(W)[n, k], in float64 for a tight reference."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float64))
    packed = _u8(packed)
    scales = np.ascontiguousarray(np.asarray(scales, dtype=np.float16))
    if x.ndim == 1:
        x = x[None]
    m, k = x.shape
    n = packed.shape[0]
    if packed.shape[1] * 2 != k:
        raise ValueError("x [M, K] and packed [N, K/2] disagree on K")
    y = np.empty((m, n), dtype=np.float64)
    _check(_native.host_lib().lowbit_host_gemv_reference(_native.np_ptr(x), _native.np_ptr(packed),
                                                           _native.np_ptr(scales), _native.np_ptr(y), m, n, k, group))
    return y
