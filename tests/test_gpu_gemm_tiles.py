"""The MFMA GEMM's two structures (lowbit_set_gemm_kernel: 1 = row groups with K split across workgroups, 2 = one
16-row tile per workgroup with its waves splitting K), forced on the same inputs, through the C ABI:
* both within the reference's bound of the fp64 product (bench/gpu_run.py:229-245), on ragged N and M, long K, group
  sizes 128 / 256 / 512 and every wave count of the tile kernel;
* each is the fp16 rounding of the exact product (every (u - 8) x product is exact) up to fp32 accumulation noise
  (half an fp16 ulp plus 2^-16 of the output RMS); so they differ only in summation order:
  within one fp16 ulp of the exact value plus 2^-15 of the output RMS of each other (outputs near zero can sit many of
  their own ulps apart), and give the same bits on every call;
* bias / residual epilogues equal the same kernel's plain result plus the torch add bit for bit, silu-mul is within
  1 ulp of silu(gate) * up from the plain result."""
import pytest
import torch
import torch.nn.functional as F

from lowbit import _native, fused, ops

from test_gpu_kernels import bound, make_weight, rel
from test_gpu_prefill import assert_rounds

pytestmark = pytest.mark.gpu


@pytest.fixture
def restore():
    yield
    _native.check(_native.lib().lowbit_set_gemm_kernel(0))
    _native.check(_native.lib().lowbit_set_launch_override(0, 0, 0))


def use(kernel, waves=0):
    _native.check(_native.lib().lowbit_set_gemm_kernel(kernel))
    _native.check(_native.lib().lowbit_set_launch_override(waves, 0, 0))


def ulps(a, b):
    return int((a.view(torch.int16).int() - b.view(torch.int16).int()).abs().max())


def same_up_to_order(a, b, ref):
    """|a - b| <= one fp16 ulp of |ref| + 2^-15 RMS(ref): two results each within half an ulp + 2^-16 RMS of ref."""
    mag = ref.abs().clamp_min(2.0 ** -14)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 10)
    over = (a.double() - b.double()).abs() - (ulp + ref.pow(2).mean().sqrt() * 2.0 ** -15)
    return float(over.max()) <= 0


@pytest.mark.parametrize("k,n,g", [(11008, 2048, 128), (2048, 200, 128), (1536, 40, 128), (512, 8, 128),
                                   (18944, 256, 256), (1024, 1000, 512), (2048, 4096, 128)])
def test_tile_kernel_against_fp64_and_row_groups(cuda, restore, k, n, g):
    wq, ref_w, *_, gen = make_weight(k, n, 5 * k + n + g, group=g, layouts=("mma",), sd=0.02)
    for m in (1, 2, 3, 8, 16, 17, 32, 33, 48, 49, 64):
        x = torch.randn(m, k, generator=gen).half().cuda()
        ref = x.double() @ ref_w.T
        lim = bound(x, ref_w, ref)
        use(1)
        rows = ops.gemv(x, wq, 5)
        assert rel(rows, ref) <= lim, (k, n, m, "rows")
        assert_rounds(rows, ref)
        for waves in (0, 1, 2, 8):
            if waves > k // 128:
                continue
            use(2, waves)
            y = ops.gemv(x, wq, 5)
            assert rel(y, ref) <= lim, (k, n, m, waves)
            assert_rounds(y, ref)
            assert same_up_to_order(y, rows, ref), (k, n, m, waves)
            assert torch.equal(ops.gemv(x, wq, 5), y), (k, n, m, waves)


@pytest.mark.parametrize("k,n", [(11008, 2048), (2048, 528)])
def test_tile_kernel_epilogues(cuda, restore, k, n):
    ext = ops.ext()
    wq, *_, gen = make_weight(k, n, k + 7 * n, layouts=("mma",), sd=0.05)
    bias = (torch.randn(n, generator=gen) * 0.5).half().cuda()
    use(2)
    for m in (2, 16, 32, 48, 64):
        x = torch.randn(m, k, generator=gen).half().cuda()
        plain = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_STORE)
        assert torch.equal(ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias),
                           plain + bias), m
        res = torch.randn(m, n, generator=gen).half().cuda()
        want = res + plain
        assert torch.equal(ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_RESIDUAL, res), want), m
        gu = plain.view(m, -1, 2, 8)
        silu = (F.silu(gu[:, :, 0]) * gu[:, :, 1]).reshape(m, -1)
        got = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_SILU_MUL)
        assert ulps(got, silu) <= 1 and float((got != silu).float().mean()) < 0.01, m
