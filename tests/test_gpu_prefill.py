"""The prefill GEMM (lowbit_w4_gemm_prefill, int4 read directly, M > 64) on the GPU, through the C ABI:
* within the reference's bound of the fp64 product on the oracle's quantized weights (bench/gpu_run.py:229-245), on
  shapes with ragged M and N, narrow N that splits K, and long K;
* the fp16 rounding of the fp64 product of the dequantized fp16 weights, up to fp32 summation noise (the kernel
  multiplies exactly the dequantized values);
* epilogues: bias and residual equal the unfused kernel plus the torch add bit for bit, silu-mul within 1 ulp;
* K splits change only the fp32 summation order; zero weights give exact zeros; repeated calls give the same bits."""
import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from lowbit import _native, ops
from oracle import quant_ref as R

from test_gpu_kernels import bound, make_weight, rel

pytestmark = pytest.mark.gpu


def prefill(x, wq, epilogue=_native.EPI_STORE, aux=None, out=None):
    return ops.ext().w4_gemm_prefill(x, wq.packed_mma, wq.scales, wq.group, epilogue, aux, out)


def assert_rounds(y, ref):
    """|y - ref| <= half an fp16 ulp of ref + 2^-16 RMS(ref) (the fp32 accumulation of fp16 products, K <= 2^15)."""
    a = ref.abs().clamp_min(2.0 ** -14)
    ulp = torch.exp2(torch.floor(torch.log2(a)) - 10)
    allowed = 0.5 * ulp + ref.pow(2).mean().sqrt() * 2.0 ** -16
    over = (y.double() - ref).abs() - allowed
    assert float(over.max()) <= 0, float(((y.double() - ref).abs() / ulp).max())


def ulps(a, b):
    return int((a.view(torch.int16).int() - b.view(torch.int16).int()).abs().max())


@pytest.mark.parametrize("k,n,m", [(256, 512, 65), (1024, 2560, 130), (2048, 1000, 200), (11008, 2048, 128),
                                   (384, 4096, 1000), (2048, 22016, 512), (18944, 256, 96), (128, 16, 1)])
def test_prefill_against_fp64(cuda, k, n, m):
    wq, ref_w, *_, gen = make_weight(k, n, 7 * k + n, layouts=("mma",), sd=0.02)
    x = torch.randn(m, k, generator=gen).half().cuda()
    y = prefill(x, wq)
    ref = x.double() @ ref_w.t()
    assert y.shape == (m, n) and y.dtype == torch.float16
    assert rel(y, ref) < bound(x, ref_w, ref), (k, n, m)
    # the kernel multiplies exactly the dequantized fp16 weights: y is the fp16 rounding of their fp64 product, up to
    # half an fp16 ulp plus fp32 summation noise
    ref16 = x.double() @ ops.dequant(wq, "mma").double().t()
    assert_rounds(y, ref16)
    assert torch.equal(prefill(x, wq), y)                   # same bits on every call


@pytest.mark.parametrize("k,n", [(2048, 2560), (11008, 2048), (1536, 17920)])
def test_prefill_epilogues(cuda, k, n):
    wq, _, *_, gen = make_weight(k, n, k + 3 * n, layouts=("mma",), sd=0.05)
    bias = (torch.randn(n, generator=gen) * 0.5).half().cuda()
    for m in (65, 200, 512):
        x = torch.randn(m, k, generator=gen).half().cuda()
        plain = prefill(x, wq)
        assert torch.equal(prefill(x, wq, _native.EPI_BIAS, bias), plain + bias), m
        res = torch.randn(m, n, generator=gen).half().cuda()
        want = res + plain
        assert torch.equal(prefill(x, wq, _native.EPI_RESIDUAL, res), want), m
        prefill(x, wq, _native.EPI_RESIDUAL, res, out=res)  # in place
        assert torch.equal(res, want), m
        gu = plain.view(m, -1, 2, 8)
        silu = (F.silu(gu[:, :, 0]) * gu[:, :, 1]).reshape(m, -1)
        got = prefill(x, wq, _native.EPI_SILU_MUL)
        assert ulps(got, silu) <= 1 and float((got != silu).float().mean()) < 0.01, m


def test_prefill_splits_only_reorder_the_sum(cuda):
    wq, ref_w, *_, gen = make_weight(11008, 2048, 99, layouts=("mma",), sd=0.02)
    x = torch.randn(300, 11008, generator=gen).half().cuda()
    ref = x.double() @ ref_w.t()
    outs = []
    try:
        for sp in (1, 2, 3, 8, 16):
            _native.lib().lowbit_set_launch_override(0, 0, sp)
            outs.append(prefill(x, wq))
    finally:
        _native.lib().lowbit_set_launch_override(0, 0, 0)
    ref16 = x.double() @ ops.dequant(wq, "mma").double().t()
    for y in outs:
        assert rel(y, ref) < bound(x, ref_w, ref)
        assert_rounds(y, ref16)


def test_prefill_zero_weights_and_tiny_activations(cuda):
    k, n, m = 512, 384, 96
    packed = np.full((n, k // 2), 0x88, np.uint8)               # u = 8 everywhere: W = 0
    scales = np.ones((n, k // 128), np.float16)
    wq = ops.W4Weight(packed, scales, 128, ("mma",))
    x = torch.randn(m, k).half().cuda() * 1000
    assert int(torch.count_nonzero(prefill(x, wq))) == 0
    wq2, ref_w, *_, gen = make_weight(k, n, 5, layouts=("mma",), sd=0.02)
    x = torch.randn(m, k, generator=gen).half().cuda()
    x[2, ::7] = 300.0
    x[5] = torch.randn(k, generator=gen).half().cuda() * 1e-5      # partly subnormal fp16
    y = prefill(x, wq2)
    ref = x.double() @ ref_w.t()
    assert rel(y, ref) < bound(x, ref_w, ref)
    # row 5's outputs are fp16 subnormals: they must be the rounding of the exact product (products of subnormal
    # activations are exact in the fp32 accumulation)
    ref16 = x.double() @ ops.dequant(wq2, "mma").double().t()
    assert_rounds(y[5:6], ref16[5:6])
    assert_rounds(y[2:3], ref16[2:3])


def test_prefill_refuses_bad_arguments(cuda):
    wq, *_ = make_weight(256, 64, 1, layouts=("mma",))
    x = torch.randn(100, 256).half().cuda()
    lib = _native.lib()
    y = torch.empty(100, 64, dtype=torch.half, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = (x.data_ptr(), wq.packed_mma.data_ptr(), wq.scales.data_ptr(), y.data_ptr())
    assert lib.lowbit_w4_gemm_prefill(*args, 100, 64, 256, 128, 7, None, None, 0, st) == 1
    assert lib.lowbit_w4_gemm_prefill(*args, 100, 64, 256, 128, _native.EPI_BIAS, None, None, 0, st) == 1
    assert lib.lowbit_w4_gemm_prefill(*args, 100, 64, 192, 64, 0, None, None, 0, st) == 7
    assert lib.lowbit_w4_gemm_prefill(*args, 0, 64, 256, 128, 0, None, None, 0, st) == 5
    assert lib.lowbit_w4_gemm_prefill(*args, 70000, 64, 16384, 128, 0, None, None, 0, st) == 3
    assert lib.lowbit_w4_gemm_prefill(*args, 100, 64, 256, 128, 0, None, ctypes.c_void_p(4104), 1 << 20, st) == 1


@pytest.mark.parametrize("k,n,m", [(2048, 2560, 200), (11008, 1000, 130)])
def test_prefill_every_launch_shape(cuda, k, n, m):
    """Each tile shape / pipeline depth the override can select (including the ones that fall back to a buildable
    variant) gives the exact rounding of the dequantized product."""
    wq, ref_w, *_, gen = make_weight(k, n, k + n + m, layouts=("mma",), sd=0.02)
    x = torch.randn(m, k, generator=gen).half().cuda()
    ref16 = x.double() @ ops.dequant(wq, "mma").double().t()
    try:
        for waves in (1, 2, 4, 8):
            for ring in (2, 3, 4):
                for sp in (0, 1, 3):
                    _native.lib().lowbit_set_launch_override(waves, ring, sp)
                    assert_rounds(prefill(x, wq), ref16)
    finally:
        _native.lib().lowbit_set_launch_override(0, 0, 0)


@pytest.mark.parametrize("k,n,m,g", [(512, 4096, 130, 256), (1024, 1000, 200, 512), (18944, 512, 100, 256)])
def test_prefill_group_sizes(cuda, k, n, m, g):
    """Groups spanning several 128-k chunks (one scale per 2 or 4 chunks), with K splits whose boundaries fall inside
    a group on the long-K case."""
    wq, ref_w, *_, gen = make_weight(k, n, k + n + g, group=g, layouts=("mma",), sd=0.02)
    x = torch.randn(m, k, generator=gen).half().cuda()
    y = prefill(x, wq)
    ref = x.double() @ ref_w.t()
    assert rel(y, ref) < bound(x, ref_w, ref)
    assert_rounds(y, x.double() @ ops.dequant(wq, "mma").double().t())


@pytest.mark.parametrize("k,n,m", [(2048, 2560, 130), (11008, 2048, 130), (896, 4864, 64)])
def test_gemm_chunked_is_v5_in_64_row_slices(cuda, k, n, m):
    """ops.gemm_chunked (reference lowbit/ops.py:145-148): many rows through the MFMA kernel 64 at a time, with no fp16
    weight copy; the same bits as the v5 kernel on each slice, and within the fp64 bound."""
    wq, ref_w, *_, gen = make_weight(k, n, 3 * k + n, layouts=("mma",), sd=0.02)
    x = torch.randn(m, k, generator=gen).half().cuda()
    y = ops.gemm_chunked(x, wq)
    assert tuple(y.shape) == (m, n)
    slices = torch.cat([ops.gemv(x[i:i + 64].contiguous(), wq, 5) for i in range(0, m, 64)])
    assert torch.equal(y, slices)
    ref = x.double() @ ref_w.T
    assert rel(y, ref) <= bound(x, ref_w, ref)
    assert_rounds(y, ref)
