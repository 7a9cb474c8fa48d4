"""GPU parity of every kernel against the CPU oracle, through the same entry points the reference's harness used
(ops.* and ext().w4_*, i.e. the C ABI). Mirrors the reference's in-benchmark checks (bench/gpu_run.py:144-247):
bit-exact quantize / relayout / dequant, every GEMV and the MFMA GEMM within max(4 x BLAS, 4 x fp16-output floor,
3e-3) of fp64 on the same quantized weights, the overflow known answers, the dispatch matrix, side-stream equality,
refusals, and graph capture."""
import numpy as np
import pytest
import torch

from lowbit import _native, ops
from oracle import quant_ref as R

pytestmark = pytest.mark.gpu

# (name, K, N): the reference's shapes (bench/gpu_run.py:24-31) plus the k/v shapes of the BASELINE sweep
SHAPES = [("qwen0.5b.q_proj", 896, 896), ("qwen0.5b.kv_proj", 896, 128), ("qwen0.5b.gate_up", 896, 4864),
          ("qwen1.5b.kv", 1536, 256), ("qwen3b.q_proj", 2048, 2048), ("qwen3b.down", 11008, 2048)]
EDGE = [("tiny", 128, 1), ("odd_n", 256, 1001), ("odd_n2", 384, 37)]
GROUP = 128


def make_weight(k, n, seed, group=GROUP, layouts=None, sd=1.0):
    g = torch.Generator().manual_seed(seed)
    wf = torch.randn(n, k, generator=g) * sd
    packed, scales = R.quantize_w4(wf.numpy(), group)
    wq = ops.W4Weight(packed, scales, group, layouts)
    ref_w = torch.from_numpy(R.dequantize_w4(packed, scales, group)).double().cuda()
    return wq, ref_w, packed, scales, g


def rel(y, ref):
    return ((y.double() - ref).abs().max() / ref.pow(2).mean().sqrt()).item()


def bound(x, ref_w, ref):
    """max(4 x BLAS error, 4 x fp16-output floor, 3e-3), the reference's acceptance rule (bench/gpu_run.py:229-245)."""
    scale = ref.pow(2).mean().sqrt().item()
    blas = (torch.nn.functional.linear(x, ref_w.half()).double() - ref).abs().max().item() / scale
    floor = (ref.half().double() - ref).abs().max().item() / scale
    return max(4 * blas, 4 * floor, R.REL_BOUND)


# ---------------------------------------------------------------- format kernels, bit for bit

@pytest.mark.parametrize("n,k", [(1, 128), (37, 384), (16, 256), (1001, 256), (4864, 896), (256, 11008)])
def test_device_relayout_matches_the_oracle(cuda, n, k):
    rng = np.random.default_rng(n + k)
    packed, scales = R.quantize_w4(rng.standard_normal((n, k)).astype(np.float32), 128)
    wq = ops.W4Weight(packed, scales, 128)
    assert np.array_equal(wq.packed.cpu().numpy(), packed)
    assert np.array_equal(wq.packed_v3.cpu().numpy(), R.interleave_for_gpu(packed))
    assert np.array_equal(wq.packed_mma.cpu().numpy(), R.interleave_for_mfma(packed))


@pytest.mark.parametrize("n,k,g,sd,dtype", [(64, 512, 128, 0.02, torch.float32), (37, 384, 128, 1.0, torch.float32),
                                            (13, 320, 64, 50.0, torch.float32), (9, 96, 32, 1e-4, torch.float32),
                                            (24, 1024, 256, 0.02, torch.float32), (300, 2048, 128, 0.02, torch.float16),
                                            (40, 768, 128, 3.0, torch.bfloat16), (5, 2048, 1024, 0.02, torch.float32)])
def test_gpu_quantizer_is_bit_exact(cuda, n, k, g, sd, dtype):
    gen = torch.Generator().manual_seed(n * k)
    w = (torch.randn(n, k, generator=gen) * sd).to(dtype)
    w[1 % n, :g] = 0
    packed, scales = ops.quantize_w4_gpu(w.cuda(), g)
    p_ref, s_ref = R.quantize_w4(w.float().numpy(), g)
    assert np.array_equal(packed.cpu().numpy(), p_ref)
    assert np.array_equal(scales.cpu().numpy().view(np.uint16), s_ref.view(np.uint16))
    # a CPU input goes through in row blocks and gives the same bits
    packed2, scales2 = ops.quantize_w4_gpu(w, g, rows_per_pass=7)
    assert torch.equal(packed2, packed) and torch.equal(scales2, scales)


def test_gpu_clip_search_agrees_with_the_oracle(cuda):
    gen = torch.Generator().manual_seed(5)
    w = torch.randn(512, 2048, generator=gen) * 0.02
    packed, scales = ops.quantize_w4_gpu(w.cuda(), 128, R.CLIP_GRID)
    p_ref, s_ref, idx, errs = R.quantize_w4_clip(w.numpy(), 128, R.CLIP_GRID)
    s_gpu = scales.cpu().numpy()
    same = s_gpu.view(np.uint16) == s_ref.view(np.uint16)
    # the fp32 sums run in a different order: a different pick is allowed only on a near-tie
    g = w.numpy().reshape(512, 16, 128).astype(np.float64)
    q_gpu = R.unpack_w4(packed.cpu().numpy()).reshape(512, 16, 128).astype(np.float64)
    e_gpu = ((q_gpu * s_gpu.astype(np.float64)[..., None] - g) ** 2).sum(-1)
    e_best = errs.min(0).astype(np.float64)
    assert np.all(e_gpu[~same] <= e_best[~same] * (1 + 1e-5))
    assert same.mean() > 0.999
    # where the scale agrees, the packed nibbles agree
    rows = same.all(1)
    assert np.array_equal(packed.cpu().numpy()[rows], p_ref[rows])


@pytest.mark.parametrize("n,k,g", [(16, 256, 128), (37, 384, 128), (1001, 256, 128), (13, 320, 64), (9, 96, 32),
                                   (24, 1024, 256), (4864, 896, 128)])
def test_dequant_is_bit_exact_on_both_layouts(cuda, n, k, g):
    rng = np.random.default_rng(n * 7 + k)
    packed, scales = R.quantize_w4(rng.standard_normal((n, k)).astype(np.float32), g)
    want = R.dequantize_w4_f16(packed, scales, g).view(np.uint16)
    wq = ops.W4Weight(packed, scales, g)
    assert np.array_equal(ops.dequant(wq, "canonical").cpu().numpy().view(np.uint16), want)
    if wq.packed_mma is not None:
        assert np.array_equal(ops.dequant(wq, "mma").cpu().numpy().view(np.uint16), want)
    assert np.array_equal(ops.dequantize_w4_gpu(wq.packed, wq.scales, g).cpu().numpy().view(np.uint16), want)


def test_dequant_rounds_once_at_extreme_scales(cuda):
    """Subnormal and near-overflow fp16 results: the product must be rounded exactly once."""
    rng = np.random.default_rng(3)
    n, k = 8, 256
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = np.array([2.0 ** -24, 6.0e-8, 3.1e-5, 6.1e-5, 0.0123, 1.0, 4000.0, 8188.0], np.float16)[:, None]
    scales = np.repeat(scales, k // 128, 1)
    want = R.dequantize_w4_f16(packed, scales, 128).view(np.uint16)
    wq = ops.W4Weight(packed, scales, 128)
    assert np.array_equal(ops.dequant(wq, "canonical").cpu().numpy().view(np.uint16), want)
    assert np.array_equal(ops.dequant(wq, "mma").cpu().numpy().view(np.uint16), want)


def test_golden_fixtures_on_the_gpu(cuda):
    golden = np.load(__import__("pathlib").Path(__file__).resolve().parent / "golden" / "w4_golden.npz")
    for case in sorted({f[:-5] for f in golden.files if f.endswith("_meta")}):
        n, k, g, m, seed = (int(v) for v in golden[f"{case}_meta"])
        packed, scales = ops.quantize_w4_gpu(torch.from_numpy(golden[f"{case}_w"]).cuda(), g)
        assert np.array_equal(packed.cpu().numpy(), golden[f"{case}_packed"]), case
        wq = ops.W4Weight(packed, scales, g)
        assert np.array_equal(ops.dequant(wq).cpu().numpy().view(np.uint16), golden[f"{case}_dequant16"].view(np.uint16))
        x = torch.from_numpy(golden[f"{case}_x"]).cuda()
        ref = torch.from_numpy(golden[f"{case}_y64"]).cuda()
        y = ops.linear(x, wq)
        if ref.abs().max() == 0:                      # an all-zero weight row: the output must be exactly zero
            assert torch.count_nonzero(y) == 0, case
        else:
            assert rel(y, ref) <= R.REL_BOUND, case
        if wq.packed_mma is not None:
            assert np.array_equal(wq.packed_mma.cpu().numpy(), golden[f"{case}_mfma"]), case


# ---------------------------------------------------------------- GEMV / GEMM accuracy

@pytest.mark.parametrize("name,k,n", SHAPES + EDGE)
def test_every_kernel_against_fp64(cuda, name, k, n):
    wq, ref_w, *_ , gen = make_weight(k, n, k * 7 + n)
    for m in list(range(1, 9)) + [12, 16, 33, 64]:
        x = torch.randn(m, k, generator=gen).half().cuda()
        ref = x.double() @ ref_w.T
        lim = bound(x, ref_w, ref)
        versions = [1, 2, 3, 4, 5, 6] if m <= 8 else [5]
        for v in versions:
            for rpw in ((0, 1, 2, 4) if v in (4, 5, 6) else (0,)):
                e = rel(ops.gemv(x, wq, v, rpw), ref)
                assert e <= lim, (name, m, v, rpw, e, lim)


@pytest.mark.parametrize("k,n,g", [(96, 200, 32), (320, 130, 64), (512, 4096, 256), (1024, 3072, 128)])
def test_group_sizes(cuda, k, n, g):
    wq, ref_w, *_, gen = make_weight(k, n, k + n + g, group=g)
    for m in (1, 3, 8):
        x = torch.randn(m, k, generator=gen).half().cuda()
        ref = x.double() @ ref_w.T
        for v in (2, 4) + ((5, 6) if wq.packed_mma is not None else ()):
            assert rel(ops.gemv(x, wq, v), ref) <= bound(x, ref_w, ref), (k, n, g, m, v)


def test_overflow_case_is_exact_for_every_kernel(cuda):
    c = R.OVERFLOW_CASE
    wq = ops.W4Weight(np.full((c["n"], c["k"] // 2), c["byte"], np.uint8), np.full((c["n"], 1), c["scale"], np.float16), c["k"])
    for xv, want in c["answers"]:
        for m in (1, 4, 16):
            x = torch.full((m, c["k"]), xv, dtype=torch.half, device="cuda")
            for v in ((1, 2, 3, 4, 5, 6) if m <= 8 else (5,)):
                y = ops.gemv(x, wq, v).float()
                assert bool(torch.isfinite(y).all()) and float((y - want).abs().max()) <= c["tol"], (xv, m, v)


# ---------------------------------------------------------------- the dispatch matrix (bench/gpu_run.py:162-198)

def test_dispatch_matrix(cuda):
    cases = [("mma_only_g128", 1024, 3072, 128, ("mma",)), ("mma_only_narrow", 1536, 1000, 128, ("mma",)),
             ("canonical_g32", 96, 200, 32, None), ("canonical_g64", 320, 130, 64, None), ("mma_g256", 512, 4096, 256, ("mma",))]
    worst = 0.0
    for name, k, n, g, layouts in cases:
        wq, ref_w, *_, gen = make_weight(k, n, k + n + g, group=g, layouts=layouts)
        for m in (1, 2, 8, 9, 17, 31, 32, 33, 63, 64, 65, 130):
            x = torch.randn(m, k, generator=gen).half().cuda()
            e = rel(ops.linear(x, wq), x.double() @ ref_w.T)
            worst = max(worst, e)
            assert e <= R.REL_BOUND, (name, m, ops.auto_version(m, wq), e)


def test_fixed_versions_past_their_rows_take_the_dequant_route(cuda):
    """A fixed version asked for more rows than it serves (v6: min(max_gemv_rows, 8); v5: 64) runs the dequantize +
    BLAS route: the same bits as F.linear on ops.dequant's fp16 weight, and within the bound of the fp64 product."""
    wq, ref_w, *_, gen = make_weight(768, 320, 41, layouts=("canonical", "mma"))
    w16 = ops.dequant(wq, "mma")
    for version, m, cap in ((6, 9, 16), (6, 5, 4), (5, 65, 8), (2, 12, 8)):
        x = torch.randn(m, 768, generator=gen).half().cuda()
        y = ops.linear(x, wq, max_gemv_rows=cap, version=version)
        assert torch.equal(y, torch.nn.functional.linear(x, w16)), (version, m)
        assert rel(y, x.double() @ ref_w.T) <= R.REL_BOUND, (version, m)


def test_results_do_not_depend_on_the_stream(cuda):
    """Every route gives the same bits on two side streams as on the default stream (the binding launches on the
    current stream and keeps one workspace per stream)."""
    wq, *_, gen = make_weight(2048, 1024, 43, layouts=("mma",))
    xs = [torch.randn(m, 2048, generator=gen).half().cuda() for m in (1, 3, 24, 64, 200)]
    want = [ops.linear(x, wq) for x in xs]
    for side in (torch.cuda.Stream(), torch.cuda.Stream()):
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            got = [ops.linear(x, wq) for x in xs]
        side.synchronize()
        for x, a, b in zip(xs, got, want):
            assert torch.equal(a, b), x.shape[0]


@pytest.mark.parametrize("case", ["scales_on_host", "group_zero", "nine_rows_gemv", "rows_past_v5", "version_7"])
def test_malformed_calls_raise_with_the_reason(cuda, case):
    """The extension refuses malformed calls with RuntimeError naming the problem (the reference's TORCH_CHECKs)."""
    wq = ops.W4Weight.from_float(torch.randn(96, 256))
    x1, x9 = torch.randn(1, 256).half().cuda(), torch.randn(9, 256).half().cuda()
    ext = ops.ext()
    calls = {
        "scales_on_host": (lambda: ext.w4_dequant(wq.packed, wq.scales.cpu(), 128), "same GPU"),
        "group_zero": (lambda: ext.w4_gemv(x1, wq.packed, wq.scales, 0, 1, 0), "group size must be positive"),
        "nine_rows_gemv": (lambda: ext.w4_gemv(x9, wq.packed, wq.scales, 128, 2, 0), "1..8 rows"),
        "rows_past_v5": (lambda: ext.w4_gemm_tc(torch.zeros(65, 256, dtype=torch.half, device="cuda"),
                                                wq.packed_mma, wq.scales, 128), "1..64 rows"),
        "version_7": (lambda: ext.w4_gemv(x1, wq.packed, wq.scales, 128, 7, 0), "version"),
    }
    call, reason = calls[case]
    with pytest.raises(RuntimeError, match=reason):
        call()


def test_graph_capture_replays_match_eager(cuda):
    """Each path captured in a hipGraph (torch.cuda.CUDAGraph), replayed several times with eager work between."""
    wq, ref_w, *_, gen = make_weight(2048, 1536, 77, layouts=("mma",))
    for m in (1, 16, 48, 200):
        x = torch.randn(m, 2048, generator=gen).half().cuda()
        eager = ops.linear(x, wq)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            ops.linear(x, wq)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = ops.linear(x, wq)
        for _ in range(3):
            x.mul_(1.0)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), m
            ops.linear(x, wq)


def test_zero_weights_give_exact_zeros(cuda):
    """Rows whose groups are all zero (scale 1.0, every nibble 8) must produce exactly 0 on every path, also next
    to nonzero rows, for any x -- the GEMV's subnormal decode removes the 8 sum(x) bias exactly."""
    rng = np.random.default_rng(12)
    n, k = 48, 1024
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[::3] = 0.0
    w[1, 128:256] = 0.0
    packed, scales = R.quantize_w4(w, 128)
    wq = ops.W4Weight(packed, scales, 128)
    for m in (1, 2, 5, 8, 16):
        x = torch.from_numpy((rng.standard_normal((m, k)) * 50).astype(np.float16)).cuda()
        for v in ((1, 2, 3, 4, 5, 6) if m <= 8 else (5,)):
            y = ops.gemv(x, wq, v)
            assert torch.count_nonzero(y[:, ::3]) == 0, (m, v)
            ref = torch.from_numpy(R.gemv_reference(x.double().cpu().numpy(), packed, scales, 128)).cuda()
            assert rel(y, ref) <= R.REL_BOUND, (m, v)
