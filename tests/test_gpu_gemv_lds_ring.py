"""The M = 1 v6 GEMV with its weight ring in LDS (direct-to-LDS loads, lowbit_set_gemv_lds_ring) against the same
kernel with the ring in registers, through the C ABI. The two consume the same 1 KB pieces in the same order and
reduce them the same way, so for every (slots, tile split, waves) the outputs must be identical bit for bit -- plain
store, every epilogue (bias, residual, silu-mul, RoPE with the cache write) and the fused RMSNorm -- and within the
reference's bound of the fp64 product (bench/gpu_run.py:229-245). Shapes cover ragged N (a last tile of 8 or 1 rows),
K from one chunk to 148, every wave having no chunk (waves > K / 128), and layers whose LDS holds fewer slots than
asked (the planner lowers them)."""
import pytest
import torch

from lowbit import _native, fused, ops

from test_gpu_kernels import bound, make_weight, rel

pytestmark = pytest.mark.gpu


def set_ring(slots):
    _native.check(_native.lib().lowbit_set_gemv_lds_ring(slots))


def set_shape(waves, splits):
    _native.check(_native.lib().lowbit_set_launch_override(waves, 0, splits))


@pytest.fixture
def reset():
    yield
    set_ring(0)
    set_shape(0, 0)


@pytest.mark.parametrize("k,n", [(128, 1), (1536, 256), (2048, 200), (896, 4864), (11008, 520), (3584, 1000),
                                 (18944, 72)])
def test_lds_ring_equals_register_ring(cuda, reset, k, n):
    wq, ref_w, *_, gen = make_weight(k, n, 5 * k + n, layouts=("mma",), sd=0.02)
    x = torch.randn(1, k, generator=gen).half().cuda()
    ref = x.double() @ ref_w.T
    lim = bound(x, ref_w, ref)
    kc = k // 128
    for splits in (0, 1, 2, 4):
        if splits > 1 and kc % splits:
            continue
        for waves in (0, 1, 4, 16):
            set_shape(waves, splits)
            set_ring(-1)
            want = ops.gemv(x, wq, 6)
            assert rel(want, ref) <= lim, (k, n, splits, waves)
            for slots in (4, 8, 12, 16):
                set_ring(slots)
                got = ops.gemv(x, wq, 6)
                assert torch.equal(got, want), (k, n, splits, waves, slots)
                assert torch.equal(ops.gemv(x, wq, 6), got)         # the same bits on every call


@pytest.mark.parametrize("k,n", [(18944, 3584), (16384, 4096), (18944, 2060)])
def test_automatic_plan_on_long_rows(cuda, reset, k, n):
    """Rows of at least 128 chunks on layers of more than 128 tiles (whole tiles per workgroup) take the LDS ring
    automatically (4 slots, 8 waves): the register ring forced to 8 waves gives the same bits, and both are within the
    bound of the fp64 product (2060 rows: a last tile of 12)."""
    wq, ref_w, *_, gen = make_weight(k, n, 9 * k + n, layouts=("mma",), sd=0.02)
    x = torch.randn(1, k, generator=gen).half().cuda()
    ref = x.double() @ ref_w.T
    auto = ops.gemv(x, wq, 6)
    set_shape(8, 1)
    set_ring(-1)
    want = ops.gemv(x, wq, 6)
    assert torch.equal(auto, want), (k, n)
    assert rel(auto, ref) <= bound(x, ref_w, ref), (k, n)


@pytest.mark.parametrize("k,n", [(2048, 2048), (1536, 208), (8960, 1536)])
def test_lds_ring_epilogues_and_norm(cuda, reset, k, n):
    ext = ops.ext()
    wq, *_, gen = make_weight(k, n, 3 * k + n, layouts=("mma",), sd=0.05)
    x = torch.randn(1, k, generator=gen).half().cuda()
    bias = (torch.randn(n, generator=gen) * 0.5).half().cuda()
    res = torch.randn(1, n, generator=gen).half().cuda()
    nw = (torch.rand(k, generator=gen) + 0.5).half().cuda()
    calls = {
        "store": lambda: ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_STORE),
        "bias": lambda: ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias),
        "residual": lambda: ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_RESIDUAL, res),
        "silu": lambda: ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_SILU_MUL),
        "norm": lambda: ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_STORE, norm=(nw, 1e-6)),
        "norm_silu": lambda: ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_SILU_MUL,
                                                 norm=(nw, 1e-6)),
    }
    for splits in (0, 2):
        set_shape(0, splits)
        for name, call in calls.items():
            set_ring(-1)
            want = call()
            for slots in (4, 16):
                set_ring(slots)
                assert torch.equal(call(), want), (name, splits, slots)


@pytest.mark.parametrize("hq,hkv,k", [(2, 1, 256), (16, 2, 2048)])
def test_lds_ring_qkv_rope(cuda, reset, hq, hkv, k):
    """lowbit_w4_qkv_rope (RMSNorm, q|k|v GEMV, bias, RoPE, cache write) with the LDS ring gives the register ring's
    bits, including a position outside the cache (nothing written)."""
    n, L = (hq + 2 * hkv) * 128, 64
    wq, *_, gen = make_weight(k, n, k + n, layouts=("mma",), sd=0.05)
    ext = ops.ext()
    bias = (torch.randn(n, generator=gen) * 0.5).half().cuda()
    nw = (1 + 0.1 * torch.randn(k, generator=gen)).half().cuda()
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).cuda()
    for p in (0, 37, 64):
        x = (torch.randn(1, k, generator=gen) * 3).half().cuda()
        pos = torch.tensor([p], device="cuda")
        outs = []
        for slots in (-1, 8):
            set_ring(slots)
            q = torch.zeros(1, hq, 128, dtype=torch.half, device="cuda")
            kc = torch.zeros(hkv, L, 128, dtype=torch.half, device="cuda")
            vc = torch.zeros_like(kc)
            ext.w4_qkv_rope(x, wq.packed_mma, wq.scales, wq.group, bias, pos, inv_freq, q, kc, vc, hq, hkv,
                            norm=(nw, 1e-6))
            outs.append((q, kc, vc))
        for a, b in zip(*outs):
            assert torch.equal(a, b), p


def test_lds_ring_under_graph_capture(cuda, reset):
    """Replays of a captured graph of LDS-ring GEMVs over several weights give the eager bits every time."""
    k, n = 2048, 2560
    ws = [make_weight(k, n, 90 + i, layouts=("mma",), sd=0.02)[0] for i in range(3)]
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(4)).half().cuda()
    set_ring(8)
    eager = [ops.gemv(x, w, 6) for w in ws]
    outs = [torch.empty_like(e) for e in eager]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for w, o in zip(ws, outs):
            o.copy_(ops.gemv(x, w, 6))
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for w, o in zip(ws, outs):
            o.copy_(ops.gemv(x, w, 6))
    for _ in range(3):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e)
        ops.gemv(x, ws[0], 6)                                   # eager work between replays
