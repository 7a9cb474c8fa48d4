"""ctypes binding of liblowbit_w4.so (include/lowbit_w4.h) and the torch-facing `ext()` object.

`NativeExt` keeps the three functions of the reference's pybind11 module (csrc/w4_gemv.cu:542-550) with the same
keyword names and defaults: w4_gemv(x, w, s, group, version, rows_per_warp=0), w4_gemm_tc(x, w, s, group,
row_tiles=0), w4_dequant(w, s, group, mma_layout=False). Like the reference they check the tensors, allocate the
output with torch.empty on the input's device, launch on that device's current stream and raise RuntimeError on any
refusal (the reference's TORCH_CHECK messages). There is no fallback: without the built library every call raises.
"""
import ctypes
import os
import pathlib

LIB_NAME = "liblowbit_w4.so"
LIB_PATH = pathlib.Path(__file__).resolve().parent / LIB_NAME
# the host format functions alone (lowbit_host_*, lowbit_last_error, lowbit_strerror), built with g++: no HIP
FORMAT_LIB_PATH = pathlib.Path(__file__).resolve().parent / "liblowbit_format.so"

LAYOUT_CANONICAL, LAYOUT_V3, LAYOUT_MFMA, LAYOUT_NV_MMA = 0, 1, 2, 3
EPI_STORE, EPI_BIAS, EPI_RESIDUAL, EPI_SILU_MUL = 0, 1, 2, 3
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2

_LIB = None
_FORMAT_LIB = None

_i64, _int, _vp = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
SIGNATURES = {
    "lowbit_last_error": ([], ctypes.c_char_p),
    "lowbit_strerror": ([_int], ctypes.c_char_p),
    "lowbit_version": ([], ctypes.c_char_p),
    "lowbit_set_launch_override": ([_int, _int, _int], _int),
    "lowbit_set_gemm_kernel": ([_int], _int),
    "lowbit_set_gemv_lds_ring": ([_int], _int),
    "lowbit_set_gemm_order": ([_int], _int),
    "lowbit_set_gemm_tile_waves": ([_int], _int),
    "lowbit_w4_gemv": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _int, _vp], _int),
    "lowbit_w4_gemm_mfma": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, ctypes.c_size_t, _vp], _int),
    "lowbit_w4_gemm_mfma_noalloc": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp], _int),
    "lowbit_w4_dequant": ([_vp, _vp, _vp, _i64, _i64, _i64, _int, _vp], _int),
    "lowbit_w4_quantize": ([_vp, _int, _vp, _vp, _i64, _i64, _i64, ctypes.POINTER(ctypes.c_float), _int, _vp], _int),
    "lowbit_w4_relayout": ([_vp, _vp, _i64, _i64, _int, _vp], _int),
    "lowbit_w4_linear_fused": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _vp, ctypes.c_float, _vp,
                                ctypes.c_size_t, _vp], _int),
    "lowbit_w4_gemm_prefill": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _vp, ctypes.c_size_t, _vp],
                               _int),
    "lowbit_rmsnorm": ([_vp, _vp, _vp, _i64, _i64, ctypes.c_float, _vp], _int),
    "lowbit_rope_kv": ([_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp], _int),
    "lowbit_w4_qkv_rope": ([_vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _vp, _i64,
                            _i64, _i64, _vp], _int),
    "lowbit_rope_table": ([_vp, _vp, _vp, _i64, _vp], _int),
    "lowbit_w4_qkv_rope_rows": ([_vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                 _i64, _vp, ctypes.c_float, _vp, ctypes.c_size_t, _vp], _int),
    "lowbit_attention": ([_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _vp, ctypes.c_size_t,
                          _vp], _int),
    "lowbit_f16_gemv": ([_vp, _vp, _vp, _i64, _i64, _i64, _vp], _int),
    "lowbit_f16_gemv_pick": ([_vp, _vp, _vp, _i64, _i64, _vp, ctypes.c_size_t, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp],
                             _int),
    "lowbit_w4_attention_linear": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _vp, _vp, _vp, _i64,
                                    _i64, _int, _vp, _vp, ctypes.c_size_t, _vp], _int),
    "lowbit_f16_attention_linear": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _vp, _vp, _i64, _int,
                                     _vp, _vp, ctypes.c_size_t, _vp], _int),
    "lowbit_f16_linear_fused": ([_vp, _vp, _vp, _i64, _i64, _int, _vp, _vp, ctypes.c_float, _vp], _int),
    "lowbit_f16_qkv_rope": ([_vp, _vp, _i64, _i64, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                             _i64, _vp], _int),
    "lowbit_hbm_read": ([_vp, _i64, _vp, _i64, _vp], _int),
    "lowbit_hbm_copy": ([_vp, _vp, _i64, _i64, _vp], _int),
    "lowbit_host_quantize": ([_vp, _vp, _vp, _i64, _i64, _i64], _int),
    "lowbit_host_unpack": ([_vp, _vp, _i64, _i64], _int),
    "lowbit_host_dequantize": ([_vp, _vp, _vp, _i64, _i64, _i64], _int),
    "lowbit_host_relayout": ([_vp, _vp, _i64, _i64, _int], _int),
    "lowbit_host_gemv_reference": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64], _int),
}


def lib():
    """The loaded library (loaded once). Raises RuntimeError if it has not been built."""
    global _LIB
    if _LIB is None:
        path = pathlib.Path(os.environ.get("LOWBIT_LIB", LIB_PATH))
        if not path.exists():
            raise RuntimeError(f"{path} is not built: run `python lowbit-kernels_amd/build.py` (hipcc, gfx950)")
        handle = ctypes.CDLL(str(path))
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes, fn.restype = args, res
        _LIB = handle
    return _LIB


HOST_FUNCTIONS = ("lowbit_last_error", "lowbit_strerror", "lowbit_host_quantize", "lowbit_host_unpack",
                  "lowbit_host_dequantize", "lowbit_host_relayout", "lowbit_host_gemv_reference")


def host_lib():
    """The HIP-free host format library (loaded once), which lowbit.quant uses: packing weights needs no GPU stack.
    Raises RuntimeError if it has not been built."""
    global _FORMAT_LIB
    if _FORMAT_LIB is None:
        path = pathlib.Path(os.environ.get("LOWBIT_FORMAT_LIB", FORMAT_LIB_PATH))
        if not path.exists():
            raise RuntimeError(f"{path} is not built: run `python lowbit-kernels_amd/build.py`")
        handle = ctypes.CDLL(str(path))
        for name in HOST_FUNCTIONS:
            fn = getattr(handle, name)
            fn.argtypes, fn.restype = SIGNATURES[name]
        _FORMAT_LIB = handle
    return _FORMAT_LIB


def check(rc, library=None):
    """Raise RuntimeError with the library's message for a non-zero status (`library`: the one that returned it,
    the kernel library by default)."""
    if rc != 0:
        l = library if library is not None else lib()
        msg = l.lowbit_last_error().decode() or l.lowbit_strerror(rc).decode()
        raise RuntimeError(msg)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def np_ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


class _DeviceGuard:
    """Make `device` current for the duration of a call (what the reference's CUDAGuard does), cheaply when it
    already is."""

    def __init__(self, device):
        import torch
        self.torch = torch
        self.index = device.index if device.index is not None else torch.cuda.current_device()
        self.prev = None

    def __enter__(self):
        cur = self.torch.cuda.current_device()
        if cur != self.index:
            self.prev = cur
            self.torch.cuda.set_device(self.index)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            self.torch.cuda.set_device(self.prev)
        return False


def _stream(device):
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


WORKSPACE_COUNTER_BYTES = 16384
WORKSPACE_BYTES = WORKSPACE_COUNTER_BYTES + (16 << 20)     # LOWBIT_WORKSPACE_BYTES
PREFILL_WORKSPACE_BYTES = WORKSPACE_COUNTER_BYTES + (64 << 20)
ATTENTION_WORKSPACE_BYTES = 4 << 20
PICK_WORKSPACE_BYTES = 1 << 20          # the greedy pick's keys: 8 bytes per 8 head rows
_WORKSPACES = {}
_CAPTURE_STREAMS = {}


def capture_stream(device):
    """One side stream per device on which the decoders warm up and capture their graphs. Workspaces are keyed by
    stream, so warming up on the stream that is then captured creates every workspace before capture (no allocation
    or fill kernel lands in a graph), and later captures reuse them. Graphs captured on it share those workspaces,
    so they must not be replayed concurrently (replay them on one stream)."""
    import torch
    index = device.index if device.index is not None else torch.cuda.current_device()
    s = _CAPTURE_STREAMS.get(index)
    if s is None:
        s = torch.cuda.Stream(device=torch.device("cuda", index))
        _CAPTURE_STREAMS[index] = s
    return s


def workspace(device, stream, nbytes=WORKSPACE_BYTES, tag=""):
    """A GEMM workspace of `nbytes` for (device, stream): zeroed once, kept for the life of the process (a graph
    captured on the stream keeps using it), so calls on one stream never race on it and never reallocate it. The
    skinny GEMM and the prefill GEMM each have their own (WORKSPACE_BYTES, PREFILL_WORKSPACE_BYTES); `tag` keeps a
    buffer of another kind apart from them whatever its size."""
    import torch
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream.value, nbytes, tag)
    ws = _WORKSPACES.get(key)
    if ws is None:
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def _check_epilogue(epilogue, aux, m, n, device):
    """aux must match what the kernels read: bias [N] or residual [M, N], fp16, contiguous, on x's GPU (the C ABI
    cannot check its size)."""
    import torch
    if epilogue not in (EPI_STORE, EPI_BIAS, EPI_RESIDUAL, EPI_SILU_MUL):
        raise RuntimeError("unknown epilogue")
    if epilogue in (EPI_BIAS, EPI_RESIDUAL):
        if aux is None:
            raise RuntimeError("the bias and residual epilogues need aux")
        if aux.dtype != torch.float16 or not aux.is_contiguous() or aux.device != device:
            raise RuntimeError("aux must be a contiguous float16 tensor on the same GPU")
        if epilogue == EPI_BIAS and aux.numel() != n:
            raise RuntimeError(f"bias must hold N={n} values, got {aux.numel()}")
        if epilogue == EPI_RESIDUAL and (aux.dim() != 2 or tuple(aux.shape) != (m, n)):
            raise RuntimeError(f"the residual must be [M, N] = [{m}, {n}], got {list(aux.shape)}")


def _need(t, name, dtype, shape, device):
    """t must be a contiguous tensor of `dtype` and `shape` on `device` (the kernels index it by that shape)."""
    if t is None or t.dtype != dtype or not t.is_contiguous() or t.device != device or tuple(t.shape) != tuple(shape):
        got = "None" if t is None else f"{t.dtype} {list(t.shape)} on {t.device}"
        raise RuntimeError(f"{name} must be a contiguous {dtype} tensor of shape {list(shape)} on {device}, got {got}")


def _check_norm(norm, k, device):
    """The fused input norm's weight: fp16 [K], contiguous, on x's GPU."""
    import torch
    if norm is None:
        return
    nw = norm[0]
    if nw.dtype != torch.float16 or not nw.is_contiguous() or nw.device != device or nw.numel() != k:
        raise RuntimeError(f"the norm weight must be a contiguous float16 [K={k}] tensor on the same GPU")


def _check_tensors(x, w, s, group):
    """The tensor-metadata half of the reference's check() (csrc/w4_gemv.cu:312-325); sizes are checked natively."""
    import torch
    if not (x.is_cuda and w.is_cuda and s.is_cuda):
        raise RuntimeError("tensors must be on the GPU")
    if w.device != x.device or s.device != x.device:
        raise RuntimeError("x, w and scales must be on the same GPU")
    if group <= 0:
        raise RuntimeError("group size must be positive")
    if x.dtype != torch.float16 or s.dtype != torch.float16 or w.dtype != torch.uint8:
        raise RuntimeError("x and scales must be float16, packed weights uint8")
    if not (x.is_contiguous() and w.is_contiguous() and s.is_contiguous()):
        raise RuntimeError("tensors must be contiguous")
    if x.dim() != 2 or w.dim() != 2 or s.dim() != 2:
        raise RuntimeError("x [M,K], w [N,K/2], scales [N,K/G]")
    k = x.shape[1]
    if group % 32 or k % group:
        raise RuntimeError("K must be a multiple of the group size, itself a multiple of 32")
    if w.shape[1] * 2 != k or s.shape[0] != w.shape[0] or s.shape[1] != k // group:
        raise RuntimeError("shape mismatch")


class NativeExt:
    """The reference's extension surface (w4_gemv / w4_gemm_tc / w4_dequant) on the gfx950 library."""

    def __init__(self):
        self.lib = lib()

    def w4_gemv(self, x, w, s, group, version, rows_per_warp=0):
        import torch
        _check_tensors(x, w, s, group)
        m, n = x.shape[0], w.shape[0]
        y = torch.empty((m, n), dtype=torch.float16, device=x.device)
        with _DeviceGuard(x.device):
            check(self.lib.lowbit_w4_gemv(ptr(x), ptr(w), ptr(s), ptr(y), m, n, x.shape[1], group, int(version),
                                          int(rows_per_warp), _stream(x.device)))
        return y

    def w4_gemm_tc(self, x, w, s, group, row_tiles=0):
        import torch
        _check_tensors(x, w, s, group)
        m, n = x.shape[0], w.shape[0]
        y = torch.empty((m, n), dtype=torch.float16, device=x.device)
        with _DeviceGuard(x.device):
            st = _stream(x.device)
            ws = workspace(x.device, st)
            check(self.lib.lowbit_w4_gemm_mfma(ptr(x), ptr(w), ptr(s), ptr(y), m, n, x.shape[1], group, int(row_tiles),
                                               ptr(ws), ws.numel(), st))
        return y

    def w4_gemm_tc_noalloc(self, x, w, s, group, row_tiles=0):
        """w4_gemm_tc through lowbit_w4_gemm_mfma_noalloc: the library's own device scratch instead of a workspace
        (same bits). Only the output is allocated here; calls on one GPU must not overlap."""
        import torch
        _check_tensors(x, w, s, group)
        m, n = x.shape[0], w.shape[0]
        y = torch.empty((m, n), dtype=torch.float16, device=x.device)
        with _DeviceGuard(x.device):
            check(self.lib.lowbit_w4_gemm_mfma_noalloc(ptr(x), ptr(w), ptr(s), ptr(y), m, n, x.shape[1], group,
                                                       int(row_tiles), _stream(x.device)))
        return y

    def w4_dequant(self, w, s, group, mma_layout=False):
        import torch
        if not (w.is_cuda and s.is_cuda and w.device == s.device):
            raise RuntimeError("packed weights and scales must be on the same GPU")
        if w.dtype != torch.uint8 or s.dtype != torch.float16:
            raise RuntimeError("packed weights uint8, scales float16")
        if w.dim() != 2 or s.dim() != 2 or group <= 0:
            raise RuntimeError("w [N,K/2], scales [N,K/G], positive group size")
        if not (w.is_contiguous() and s.is_contiguous()):
            raise RuntimeError("packed weights must be contiguous and 16-byte aligned")
        n, k = w.shape[0], w.shape[1] * 2
        if group % 32 or k % group or s.shape[0] != n or s.shape[1] != k // group:
            raise RuntimeError("shape mismatch")
        out = torch.empty((n, k), dtype=torch.float16, device=w.device)
        with _DeviceGuard(w.device):
            check(self.lib.lowbit_w4_dequant(ptr(w), ptr(s), ptr(out), n, k, group, 1 if mma_layout else 0,
                                             _stream(w.device)))
        return out

    # ---- beyond the reference's three functions: the device quantizer and relayout ----

    def w4_quantize(self, w, group, clip_grid=None):
        """Device quantizer: W [N, K] (float32 / float16 / bfloat16, CUDA) -> (packed canonical, scales fp16)."""
        import torch
        dtypes = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}
        if not w.is_cuda or w.dim() != 2:
            raise RuntimeError("the GPU quantizer takes a 2-D CUDA tensor")
        if w.dtype not in dtypes:
            w = w.float()
        w = w.contiguous()
        n, k = w.shape
        packed = torch.empty((n, k // 2), dtype=torch.uint8, device=w.device)
        scales = torch.empty((n, k // group if group > 0 else 0), dtype=torch.float16, device=w.device)
        grid = [float(a) for a in clip_grid] if clip_grid else []
        arr = (ctypes.c_float * max(1, len(grid)))(*grid)
        with _DeviceGuard(w.device):
            check(self.lib.lowbit_w4_quantize(ptr(w), dtypes[w.dtype], ptr(packed), ptr(scales), n, k, group, arr,
                                              len(grid), _stream(w.device)))
        return packed, scales

    def w4_relayout(self, packed, layout):
        """canonical packed [N, K/2] (CUDA) -> a new tensor in LAYOUT_V3 or LAYOUT_MFMA."""
        import torch
        if not packed.is_cuda or packed.dtype != torch.uint8 or packed.dim() != 2:
            raise RuntimeError("packed weights must be a 2-D uint8 CUDA tensor")
        packed = packed.contiguous()
        out = torch.empty_like(packed)
        with _DeviceGuard(packed.device):
            check(self.lib.lowbit_w4_relayout(ptr(packed), ptr(out), packed.shape[0], packed.shape[1] * 2, int(layout),
                                              _stream(packed.device)))
        return out

    # ---- decode-step fusions (lowbit_w4_linear_fused, lowbit_rmsnorm, lowbit_rope_kv, lowbit_attention) ----

    def w4_linear_fused(self, x, w, s, group, epilogue, aux=None, out=None, norm=None):
        """x [M, K] (M <= 64) times the MFMA-layout weight with the epilogue fused into the store; returns y
        ([M, N], or [M, N / 2] for EPI_SILU_MUL). `out` may be given (for EPI_RESIDUAL it may be `aux` itself).
        norm = (weight, eps): project RMSNorm(x) * weight instead of x, normalized in the kernel (K <= 16384 for one
        row; K <= 8192 for 2..64 rows, with lowbit_rmsnorm's bits)."""
        import torch
        _check_tensors(x, w, s, group)
        m, n = x.shape[0], w.shape[0]
        cols = n // 2 if epilogue == EPI_SILU_MUL else n
        y = out if out is not None else torch.empty((m, cols), dtype=torch.float16, device=x.device)
        if y.shape != (m, cols) or y.dtype != torch.float16 or not y.is_contiguous() or y.device != x.device:
            raise RuntimeError("out must be a contiguous float16 [M, N] (or [M, N/2] for silu-mul) tensor")
        _check_epilogue(epilogue, aux, m, n, x.device)
        _check_norm(norm, x.shape[1], x.device)
        with _DeviceGuard(x.device):
            st = _stream(x.device)
            ws = workspace(x.device, st)
            nw, eps = norm if norm is not None else (None, 0.0)
            check(self.lib.lowbit_w4_linear_fused(ptr(x), ptr(w), ptr(s), ptr(y), m, n, x.shape[1], group,
                                                  int(epilogue), ptr(aux) if aux is not None else None,
                                                  ptr(nw) if nw is not None else None, float(eps), ptr(ws),
                                                  ws.numel(), st))
        return y

    def w4_gemm_prefill(self, x, w, s, group, epilogue=EPI_STORE, aux=None, out=None):
        """x [M, K] (any M, meant for M > 64) times the MFMA-layout weight, int4 read directly, with the epilogue
        fused into the store; returns y ([M, N], or [M, N / 2] for EPI_SILU_MUL)."""
        import torch
        _check_tensors(x, w, s, group)
        m, n = x.shape[0], w.shape[0]
        cols = n // 2 if epilogue == EPI_SILU_MUL else n
        y = out if out is not None else torch.empty((m, cols), dtype=torch.float16, device=x.device)
        if y.shape != (m, cols) or y.dtype != torch.float16 or not y.is_contiguous() or y.device != x.device:
            raise RuntimeError("out must be a contiguous float16 [M, N] (or [M, N/2] for silu-mul) tensor")
        _check_epilogue(epilogue, aux, m, n, x.device)
        with _DeviceGuard(x.device):
            st = _stream(x.device)
            ws = workspace(x.device, st, PREFILL_WORKSPACE_BYTES)
            check(self.lib.lowbit_w4_gemm_prefill(ptr(x), ptr(w), ptr(s), ptr(y), m, n, x.shape[1], group,
                                                  int(epilogue), ptr(aux) if aux is not None else None, ptr(ws),
                                                  ws.numel(), st))
        return y

    def rmsnorm(self, x, weight, eps, out=None):
        import torch
        if not x.is_cuda or x.dim() != 2:
            raise RuntimeError("rmsnorm takes a 2-D CUDA tensor x [M, H]")
        _need(x, "x", torch.float16, x.shape, x.device)
        _need(weight, "the norm weight", torch.float16, (x.shape[1],), x.device)
        y = out if out is not None else torch.empty_like(x)
        _need(y, "out", torch.float16, x.shape, x.device)
        with _DeviceGuard(x.device):
            check(self.lib.lowbit_rmsnorm(ptr(x), ptr(weight), ptr(y), x.shape[0], x.shape[1], float(eps),
                                          _stream(x.device)))
        return y

    def _check_rope(self, m, positions, inv_freq, q_out, k_cache, v_cache, hq, hkv, device):
        import torch
        if k_cache.dim() != 3:
            raise RuntimeError("the caches must be [Hkv, L, 128]")
        _need(positions, "positions", torch.int64, (m,), device)
        _need(inv_freq, "inv_freq", torch.float32, (64,), device)
        _need(q_out, "q_out", torch.float16, (m, hq, 128), device)
        _need(k_cache, "k_cache", torch.float16, (hkv, k_cache.shape[1], 128), device)
        _need(v_cache, "v_cache", torch.float16, tuple(k_cache.shape), device)

    def rope_kv(self, qkv, positions, inv_freq, q_out, k_cache, v_cache, hq, hkv, permuted=False):
        import torch
        if not qkv.is_cuda or qkv.dim() != 2:
            raise RuntimeError("qkv must be a 2-D CUDA tensor [M, (Hq + 2 Hkv) 128]")
        _need(qkv, "qkv", torch.float16, (qkv.shape[0], (hq + 2 * hkv) * 128), qkv.device)
        self._check_rope(qkv.shape[0], positions, inv_freq, q_out, k_cache, v_cache, hq, hkv, qkv.device)
        with _DeviceGuard(qkv.device):
            check(self.lib.lowbit_rope_kv(ptr(qkv), ptr(positions), ptr(inv_freq), ptr(q_out), ptr(k_cache),
                                          ptr(v_cache), qkv.shape[0], hq, hkv, k_cache.shape[1], int(bool(permuted)),
                                          _stream(qkv.device)))

    def w4_qkv_rope(self, x, w, s, group, bias, positions, inv_freq, q_out, k_cache, v_cache, hq, hkv, norm=None):
        """One token: the RoPE-permuted q|k|v projection (+ bias, RoPE, cache write) into q_out [1, Hq, 128] and
        the caches [Hkv, L, 128]; norm = (weight, eps) normalizes x first."""
        import torch
        _check_tensors(x, w, s, group)
        if x.shape[0] != 1:
            raise RuntimeError("w4_qkv_rope takes one row")
        if w.shape[0] != (hq + 2 * hkv) * 128:
            raise RuntimeError("the q|k|v weight must have (Hq + 2 Hkv) * 128 rows")
        _need(bias, "bias", torch.float16, (w.shape[0],), x.device)
        _check_norm(norm, x.shape[1], x.device)
        self._check_rope(1, positions, inv_freq, q_out, k_cache, v_cache, hq, hkv, x.device)
        nw, eps = norm if norm is not None else (None, 0.0)
        with _DeviceGuard(x.device):
            check(self.lib.lowbit_w4_qkv_rope(ptr(x), ptr(w), ptr(s), w.shape[0], x.shape[1], group, ptr(bias),
                                              ptr(nw) if nw is not None else None, float(eps), ptr(positions),
                                              ptr(inv_freq), ptr(q_out), ptr(k_cache), ptr(v_cache), hq, hkv,
                                              k_cache.shape[1], _stream(x.device)))

    def rope_table(self, positions, inv_freq, out=None):
        """The RoPE factors of a step: int32 [M, 64], each the fp16 pair (cos, sin) of positions[m] * inv_freq[i], as
        lowbit_rope_kv evaluates them (w4_qkv_rope_rows reads it)."""
        import torch
        m = positions.shape[0]
        _need(positions, "positions", torch.int64, (m,), positions.device)
        _need(inv_freq, "inv_freq", torch.float32, (64,), positions.device)
        t = out if out is not None else torch.empty(m, 64, dtype=torch.int32, device=positions.device)
        _need(t, "out", torch.int32, (m, 64), positions.device)
        with _DeviceGuard(positions.device):
            check(self.lib.lowbit_rope_table(ptr(positions), ptr(inv_freq), ptr(t), m, _stream(positions.device)))
        return t

    def w4_qkv_rope_rows(self, x, w, s, group, bias, positions, table, q_out, k_cache, v_cache, hq, hkv, norm=None):
        """M tokens: the RoPE-permuted q|k|v projection of the input x [M, K] (+ bias, RoPE, cache write) into q_out
        [M, Hq, 128] and the caches [Hkv, L, 128] at rows positions[m]; table = rope_table(positions, ...) (the MFMA
        GEMM up to 64 rows, the prefill GEMM beyond, each with its own workspace). norm = (weight, eps), up to 64 rows and
        K <= 8192: project RMSNorm(x) * weight, normalized in the GEMM (lowbit_rmsnorm's bits); otherwise x is the
        normalized input."""
        import torch
        _check_tensors(x, w, s, group)
        m = x.shape[0]
        _check_norm(norm, x.shape[1], x.device)
        if w.shape[0] != (hq + 2 * hkv) * 128:
            raise RuntimeError("the q|k|v weight must have (Hq + 2 Hkv) * 128 rows")
        _need(bias, "bias", torch.float16, (w.shape[0],), x.device)
        _need(table, "table", torch.int32, (m, 64), x.device)
        if k_cache.dim() != 3:
            raise RuntimeError("the caches must be [Hkv, L, 128]")
        _need(positions, "positions", torch.int64, (m,), x.device)
        _need(q_out, "q_out", torch.float16, (m, hq, 128), x.device)
        _need(k_cache, "k_cache", torch.float16, (hkv, k_cache.shape[1], 128), x.device)
        _need(v_cache, "v_cache", torch.float16, tuple(k_cache.shape), x.device)
        with _DeviceGuard(x.device):
            st = _stream(x.device)
            ws = workspace(x.device, st, WORKSPACE_BYTES if m <= 64 else PREFILL_WORKSPACE_BYTES)
            nw, eps = norm if norm is not None else (None, 0.0)
            check(self.lib.lowbit_w4_qkv_rope_rows(ptr(x), ptr(w), ptr(s), m, w.shape[0], x.shape[1], group, ptr(bias),
                                                   ptr(positions), ptr(table), ptr(q_out), ptr(k_cache), ptr(v_cache),
                                                   hq, hkv, k_cache.shape[1], ptr(nw) if nw is not None else None,
                                                   float(eps), ptr(ws), ws.numel(), st))

    def attention(self, q, k_cache, v_cache, positions, out, hq, hkv, max_keys, scale, split=True):
        """split=False runs one block per (token, head group), without the key partitions and their workspace."""
        import torch
        if not q.is_cuda or q.dim() != 3 or k_cache.dim() != 3:
            raise RuntimeError("q [M, Hq, 128] and the caches [Hkv, L, 128] must be CUDA tensors")
        m = q.shape[0]
        _need(q, "q", torch.float16, (m, hq, 128), q.device)
        _need(k_cache, "k_cache", torch.float16, (hkv, k_cache.shape[1], 128), q.device)
        _need(v_cache, "v_cache", torch.float16, tuple(k_cache.shape), q.device)
        _need(positions, "positions", torch.int64, (m,), q.device)
        _need(out, "out", torch.float16, (m, hq * 128), q.device)
        with _DeviceGuard(q.device):
            st = _stream(q.device)
            ws = workspace(q.device, st, ATTENTION_WORKSPACE_BYTES) if split else None
            check(self.lib.lowbit_attention(ptr(q), ptr(k_cache), ptr(v_cache), ptr(positions), ptr(out), q.shape[0],
                                            hq, hkv, k_cache.shape[1], int(max_keys), float(scale),
                                            ptr(ws) if ws is not None else None, ws.numel() if ws is not None else 0,
                                            st))

    def _attention_linear(self, q, k_cache, v_cache, positions, hq, hkv, max_keys, scale, w, s, group, epilogue, aux,
                          out):
        import torch
        if not q.is_cuda or q.dim() != 3 or k_cache.dim() != 3:
            raise RuntimeError("q [1, Hq, 128] and the caches [Hkv, L, 128] must be CUDA tensors")
        _need(q, "q", torch.float16, (1, hq, 128), q.device)
        _need(k_cache, "k_cache", torch.float16, (hkv, k_cache.shape[1], 128), q.device)
        _need(v_cache, "v_cache", torch.float16, tuple(k_cache.shape), q.device)
        _need(positions, "positions", torch.int64, (1,), q.device)
        k = hq * 128
        if s is not None:
            _check_tensors(torch.empty((1, k), dtype=torch.float16, device=q.device), w, s, group)
        elif w.dtype != torch.float16 or w.dim() != 2 or w.shape[1] != k or not w.is_contiguous() or w.device != q.device:
            raise RuntimeError("w must be a contiguous float16 [N, Hq * 128] tensor on q's GPU")
        n = w.shape[0]
        cols = n // 2 if epilogue == EPI_SILU_MUL else n
        y = out if out is not None else torch.empty((1, cols), dtype=torch.float16, device=q.device)
        _need(y, "out", torch.float16, (1, cols), q.device)
        _check_epilogue(epilogue, aux, 1, n, q.device)
        with _DeviceGuard(q.device):
            st = _stream(q.device)
            ws = workspace(q.device, st, ATTENTION_WORKSPACE_BYTES)
            common = (ptr(q), ptr(k_cache), ptr(v_cache), ptr(positions), hq, hkv, k_cache.shape[1], int(max_keys),
                      float(scale))
            aux_p = ptr(aux) if aux is not None else None
            if s is not None:
                check(self.lib.lowbit_w4_attention_linear(*common, ptr(w), ptr(s), ptr(y), n, group, int(epilogue), aux_p,
                                                          ptr(ws), ws.numel(), st))
            else:
                check(self.lib.lowbit_f16_attention_linear(*common, ptr(w), ptr(y), n, int(epilogue), aux_p, ptr(ws),
                                                           ws.numel(), st))
        return y

    def w4_attention_linear(self, q, k_cache, v_cache, positions, hq, hkv, max_keys, scale, w, s, group, epilogue,
                            aux=None, out=None):
        """One token's attention (as attention(), at most 8 key partitions) followed by the int4 projection with its
        epilogue, the partitions merged in the projection's prologue (lowbit_w4_attention_linear): y [1, N] (or
        [1, N / 2] for EPI_SILU_MUL); `out` may be `aux` for the residual."""
        return self._attention_linear(q, k_cache, v_cache, positions, hq, hkv, max_keys, scale, w, s, group, epilogue,
                                      aux, out)

    def f16_attention_linear(self, q, k_cache, v_cache, positions, hq, hkv, max_keys, scale, w, epilogue, aux=None,
                             out=None):
        """w4_attention_linear over an fp16 weight W [N, Hq * 128] (lowbit_f16_attention_linear)."""
        return self._attention_linear(q, k_cache, v_cache, positions, hq, hkv, max_keys, scale, w, None, 0, epilogue,
                                      aux, out)

    def f16_gemv(self, x, w, out=None):
        """fp16 x [M <= 16, K] times fp16 W [N, K]^T -> fp16 [M, N] (fp32 accumulation)."""
        import torch
        if not (x.is_cuda and w.is_cuda and x.device == w.device):
            raise RuntimeError("x and w must be on the same GPU")
        if x.dtype != torch.float16 or w.dtype != torch.float16 or not (x.is_contiguous() and w.is_contiguous()):
            raise RuntimeError("x and w must be contiguous float16")
        if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
            raise RuntimeError("x [M, K] and w [N, K]")
        y = out if out is not None else torch.empty((x.shape[0], w.shape[0]), dtype=torch.float16, device=x.device)
        _need(y, "out", torch.float16, (x.shape[0], w.shape[0]), x.device)
        with _DeviceGuard(x.device):
            check(self.lib.lowbit_f16_gemv(ptr(x), ptr(w), ptr(y), x.shape[0], w.shape[0], x.shape[1],
                                           _stream(x.device)))
        return y

    def f16_gemv_pick(self, x, w, tokens, positions=None, out=None, out_tokens=None, out_count=None, embed=None,
                      h_out=None):
        """f16_gemv for one row, then the greedy pick on the GPU: tokens[0] = argmax of the logits (torch.argmax's
        choice among equal maxima and NaNs), positions[0] += 1 (int64, or None); returns the logits [1, N].
        out_tokens (int64) with out_count (int32 [1]): out_tokens[out_count] = the pick while out_count <
        out_tokens.numel(), then out_count += 1. embed ([N, K] fp16) with h_out ([1, K] fp16): h_out = embed[pick]."""
        import torch
        if x.dim() != 2 or x.shape[0] != 1:
            raise RuntimeError("f16_gemv_pick takes one row x [1, K]")
        if not (x.is_cuda and w.is_cuda and x.device == w.device):
            raise RuntimeError("x and w must be on the same GPU")
        if x.dtype != torch.float16 or w.dtype != torch.float16 or not (x.is_contiguous() and w.is_contiguous()):
            raise RuntimeError("x and w must be contiguous float16")
        if w.dim() != 2 or x.shape[1] != w.shape[1]:
            raise RuntimeError("x [1, K] and w [N, K]")
        for name, t in (("tokens", tokens), ("positions", positions)):   # element 0 is written
            if t is not None and (t.dtype != torch.int64 or not t.is_contiguous() or t.device != x.device or t.numel() < 1):
                raise RuntimeError(f"{name} must be a contiguous int64 tensor of at least one element on {x.device}")
        if (out_tokens is None) != (out_count is None) or (embed is None) != (h_out is None):
            raise RuntimeError("out_tokens goes with out_count, embed with h_out")
        if out_tokens is not None:
            if out_tokens.dtype != torch.int64 or not out_tokens.is_contiguous() or out_tokens.device != x.device:
                raise RuntimeError(f"out_tokens must be a contiguous int64 tensor on {x.device}")
            _need(out_count, "out_count", torch.int32, (1,), x.device)
        if embed is not None:
            _need(embed, "embed", torch.float16, tuple(w.shape), x.device)
            _need(h_out, "h_out", torch.float16, (1, x.shape[1]), x.device)
        n = w.shape[0]
        y = out if out is not None else torch.empty((1, n), dtype=torch.float16, device=x.device)
        _need(y, "out", torch.float16, (1, n), x.device)
        with _DeviceGuard(x.device):
            st = _stream(x.device)
            ws = workspace(x.device, st, max(PICK_WORKSPACE_BYTES, 8 * (-(-n // 8))), tag="pick")
            opt = lambda t: ptr(t) if t is not None else None
            check(self.lib.lowbit_f16_gemv_pick(ptr(x), ptr(w), ptr(y), n, x.shape[1], ptr(ws), ws.numel(), ptr(tokens),
                                                opt(positions), opt(out_tokens),
                                                out_tokens.numel() if out_tokens is not None else 0, opt(out_count),
                                                opt(embed), opt(h_out), st))
        return y

    def _check_f16_weight(self, x, w):
        import torch
        if not (x.is_cuda and w.is_cuda and x.device == w.device):
            raise RuntimeError("x and w must be on the same GPU")
        if x.dtype != torch.float16 or w.dtype != torch.float16 or not (x.is_contiguous() and w.is_contiguous()):
            raise RuntimeError("x and w must be contiguous float16")
        if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1] or x.shape[0] != 1:
            raise RuntimeError("x [1, K] and w [N, K]")

    def f16_linear_fused(self, x, w, epilogue, aux=None, out=None, norm=None):
        """One row x [1, K] times an fp16 weight W [N, K]^T with the epilogue fused into the store (the W4A16 fused
        GEMV's comparator: same kernel structure and epilogues, fp16 weight bytes); returns y ([1, N], or [1, N / 2]
        for EPI_SILU_MUL). norm = (weight, eps): project RMSNorm(x) * weight instead of x."""
        import torch
        self._check_f16_weight(x, w)
        n = w.shape[0]
        cols = n // 2 if epilogue == EPI_SILU_MUL else n
        y = out if out is not None else torch.empty((1, cols), dtype=torch.float16, device=x.device)
        _need(y, "out", torch.float16, (1, cols), x.device)
        _check_epilogue(epilogue, aux, 1, n, x.device)
        _check_norm(norm, x.shape[1], x.device)
        nw, eps = norm if norm is not None else (None, 0.0)
        with _DeviceGuard(x.device):
            check(self.lib.lowbit_f16_linear_fused(ptr(x), ptr(w), ptr(y), n, x.shape[1], int(epilogue),
                                                   ptr(aux) if aux is not None else None,
                                                   ptr(nw) if nw is not None else None, float(eps), _stream(x.device)))
        return y

    def f16_qkv_rope(self, x, w, bias, positions, inv_freq, q_out, k_cache, v_cache, hq, hkv, norm=None):
        """w4_qkv_rope over an fp16 q|k|v weight in the same RoPE-permuted row order."""
        import torch
        self._check_f16_weight(x, w)
        if w.shape[0] != (hq + 2 * hkv) * 128:
            raise RuntimeError("the q|k|v weight must have (Hq + 2 Hkv) * 128 rows")
        _need(bias, "bias", torch.float16, (w.shape[0],), x.device)
        _check_norm(norm, x.shape[1], x.device)
        self._check_rope(1, positions, inv_freq, q_out, k_cache, v_cache, hq, hkv, x.device)
        nw, eps = norm if norm is not None else (None, 0.0)
        with _DeviceGuard(x.device):
            check(self.lib.lowbit_f16_qkv_rope(ptr(x), ptr(w), w.shape[0], x.shape[1], ptr(bias),
                                               ptr(nw) if nw is not None else None, float(eps), ptr(positions),
                                               ptr(inv_freq), ptr(q_out), ptr(k_cache), ptr(v_cache), hq, hkv,
                                               k_cache.shape[1], _stream(x.device)))

    # ---- bandwidth probes (lowbit_hbm_read, lowbit_hbm_copy) ----
    def hbm_read(self, buf, sink, blocks):
        """Stream every byte of the contiguous CUDA tensor `buf` (nbytes a multiple of 16) through `blocks`
        workgroups; `sink` is a CUDA int32 tensor the kernel may write one word to."""
        with _DeviceGuard(buf.device):
            check(self.lib.lowbit_hbm_read(ptr(buf), buf.numel() * buf.element_size(), ptr(sink), int(blocks),
                                           _stream(buf.device)))

    def hbm_copy(self, src, dst, blocks):
        if src.numel() * src.element_size() != dst.numel() * dst.element_size():
            raise RuntimeError("hbm_copy: src and dst must have the same size in bytes")
        with _DeviceGuard(src.device):
            check(self.lib.lowbit_hbm_copy(ptr(src), ptr(dst), src.numel() * src.element_size(), int(blocks),
                                           _stream(src.device)))
