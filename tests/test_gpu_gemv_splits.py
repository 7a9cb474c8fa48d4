"""The M <= 8 MFMA-layout GEMV with a 16-row tile split over 2 or 4 workgroups (8 or 4 rows each, a wave-load then
covering 2 or 4 chunks), forced through lowbit_set_launch_override's k_splits, through the C ABI:
* within the reference's bound of the fp64 product (bench/gpu_run.py:229-245) for every split and wave count, on
  ragged N (a last tile of 8 rows, whose second half-tile workgroups have no rows) and M = 1..8;
* a split only reorders the fp32 sums: within one fp16 ulp of the exact value plus 2^-16 of the output RMS of the
  unsplit result;
* bias / residual epilogues and the fused RMSNorm under a split give the same bits as the same split's plain sum plus
  the torch add / the separate norm; silu-mul and RoPE pair rows r and r + 8 of a tile, so they ignore the split."""
import pytest
import torch

from lowbit import _native, ops

from test_gpu_kernels import bound, make_weight, rel

pytestmark = pytest.mark.gpu


def set_split(waves, splits):
    _native.check(_native.lib().lowbit_set_launch_override(waves, 0, splits))


@pytest.fixture
def reset_override():
    yield
    _native.check(_native.lib().lowbit_set_launch_override(0, 0, 0))


def same_up_to_order(a, b, ref):
    """|a - b| <= one fp16 ulp of |ref| + 2^-16 RMS(ref): two fp32 summation orders of the same products."""
    mag = ref.abs().clamp_min(2.0 ** -14)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 10)
    over = (a.double() - b.double()).abs() - (ulp + ref.pow(2).mean().sqrt() * 2.0 ** -16)
    return float(over.max()) <= 0


@pytest.mark.parametrize("k,n", [(1536, 256), (2048, 200), (1024, 40), (512, 8), (11008, 512), (3584, 1000)])
def test_every_split_against_fp64(cuda, reset_override, k, n):
    wq, ref_w, *_, gen = make_weight(k, n, 11 * k + n, layouts=("mma",), sd=0.02)
    kc = k // 128
    for m in (1, 2, 3, 5, 8):
        x = torch.randn(m, k, generator=gen).half().cuda()
        ref = x.double() @ ref_w.T
        lim = bound(x, ref_w, ref)
        set_split(0, 1)
        base = ops.gemv(x, wq, 6)
        assert rel(base, ref) <= lim, (k, n, m)
        for splits in (2, 4):
            if kc % splits:
                continue
            for waves in (0, 1, 2, 4, 8):
                if waves > kc // splits:
                    continue
                set_split(waves, splits)
                y = ops.gemv(x, wq, 6)
                assert rel(y, ref) <= lim, (k, n, m, splits, waves)
                assert same_up_to_order(y, base, ref), (k, n, m, splits, waves)
                assert torch.equal(ops.gemv(x, wq, 6), y)            # same bits on every call


def test_automatic_plan_splits_narrow_layers(cuda, reset_override):
    """The automatic plan (no override) on the narrow decode shapes agrees with the unsplit kernel."""
    for k, n in [(1536, 256), (2048, 256), (2048, 2048), (8960, 1536), (11008, 2048)]:
        wq, ref_w, *_, gen = make_weight(k, n, k + 5 * n, layouts=("mma",), sd=0.02)
        x = torch.randn(1, k, generator=gen).half().cuda()
        ref = x.double() @ ref_w.T
        auto = ops.gemv(x, wq, 6)
        set_split(0, 1)
        base = ops.gemv(x, wq, 6)
        _native.check(_native.lib().lowbit_set_launch_override(0, 0, 0))
        assert rel(auto, ref) <= bound(x, ref_w, ref), (k, n)
        assert same_up_to_order(auto, base, ref), (k, n)


@pytest.mark.parametrize("k,n", [(2048, 2048), (1536, 200)])
def test_split_epilogues_and_norm(cuda, reset_override, k, n):
    from lowbit import fused
    ext = ops.ext()
    wq, *_, gen = make_weight(k, n, 3 * k + n, layouts=("mma",), sd=0.05)
    x = torch.randn(1, k, generator=gen).half().cuda()
    bias = (torch.randn(n, generator=gen) * 0.5).half().cuda()
    nw = (torch.rand(k, generator=gen) + 0.5).half().cuda()
    for splits in (1, 2, 4):
        set_split(0, splits)
        plain = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_STORE)
        assert torch.equal(ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias),
                           plain + bias), splits
        res = torch.randn(1, n, generator=gen).half().cuda()
        want = res + plain
        assert torch.equal(ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_RESIDUAL, res),
                           want), splits
        # the fused norm sums its statistics in another order than lowbit_rmsnorm (and may use more waves): the
        # tolerance of the unsplit fused-norm test
        normed = ext.rmsnorm(x, nw, 1e-6)
        want_n = ext.w4_linear_fused(normed, wq.packed_mma, wq.scales, wq.group, fused.EPI_STORE)
        got_n = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_STORE, norm=(nw, 1e-6))
        assert rel(got_n, want_n.double()) < 2e-3, splits


def test_pair_epilogues_ignore_the_split(cuda, reset_override):
    from lowbit import fused
    ext = ops.ext()
    k, n = 2048, 1024
    wq, *_, gen = make_weight(k, n, 77, layouts=("mma",), sd=0.05)
    x = torch.randn(1, k, generator=gen).half().cuda()
    set_split(0, 1)
    want = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_SILU_MUL)
    for splits in (2, 4):
        set_split(0, splits)
        assert torch.equal(ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_SILU_MUL), want)
