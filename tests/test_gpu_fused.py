"""The decode-step fusions on the GPU, through the C ABI:
* lowbit_w4_linear_fused: the bias and residual epilogues give exactly the unfused result (the same kernel's sum,
  then the torch add); silu-mul equals torch's silu(gate) * up on the unfused outputs; GEMV (M = 1) and MFMA paths,
  with and without the split of K;
* lowbit_rmsnorm and lowbit_rope_kv against transformers' own Qwen2RMSNorm and apply_rotary_pos_emb;
* lowbit_w4_qkv_rope (one row) and lowbit_w4_qkv_rope_rows with lowbit_rope_table (M rows) bit for bit against the
  projection with the bias epilogue followed by lowbit_rope_kv;
* lowbit_attention against an fp32 causal softmax attention;
* FusedQwen2 (fp16 and int4) against the transformers model on the same tokens."""
import math

import pytest
import torch
import torch.nn.functional as F

from lowbit import _native, decode, fused, model as lbmodel, ops

from test_gpu_kernels import make_weight, rel

pytestmark = pytest.mark.gpu


def ulp_diff(a, b):
    return int((a.view(torch.int16).int() - b.view(torch.int16).int()).abs().max())


@pytest.mark.parametrize("k,n", [(1024, 512), (2048, 2560), (11008, 2048), (384, 4096)])
def test_epilogues_equal_the_unfused_ops(cuda, k, n):
    wq, _, *_, gen = make_weight(k, n, k + n, layouts=("mma",), sd=0.05)
    ext = ops.ext()
    bias = (torch.randn(n, generator=gen) * 0.5).half().cuda()
    for m in (1, 3, 16, 40):
        x = torch.randn(m, k, generator=gen).half().cuda()
        plain = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_STORE)
        unfused = ops.gemv(x, wq, 6 if m == 1 else 5)
        assert torch.equal(plain, unfused), m
        assert torch.equal(ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias),
                           plain + bias), m
        res = torch.randn(m, n, generator=gen).half().cuda()
        want = res + plain
        got = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_RESIDUAL, res)
        assert torch.equal(got, want), m
        ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_RESIDUAL, res, out=res)   # in place
        assert torch.equal(res, want), m
        gu = plain.view(m, -1, 2, 8)
        want = (F.silu(gu[:, :, 0]) * gu[:, :, 1]).reshape(m, -1)
        got = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_SILU_MUL)
        assert ulp_diff(got, want) <= 1 and float((got != want).float().mean()) < 0.01, m


@pytest.mark.parametrize("k,n", [(256, 512), (1536, 2048), (2048, 22016), (3584, 4608)])
def test_fused_input_norm_matches_norm_then_projection(cuda, k, n):
    wq, _, *_, gen = make_weight(k, n, 3 * k + n, layouts=("mma",), sd=0.05)
    ext = ops.ext()
    nw = (1 + 0.1 * torch.randn(k, generator=gen)).half().cuda()
    bias = (torch.randn(n, generator=gen) * 0.5).half().cuda()
    for scale in (1.0, 40.0, 1e-3):
        x = (torch.randn(1, k, generator=gen) * scale).half().cuda()
        want = ext.w4_linear_fused(ext.rmsnorm(x, nw, 1e-6), wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias)
        got = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias, norm=(nw, 1e-6))
        assert rel(got, want.double()) < 2e-3, (k, n, scale)
        if n % 16 == 0:
            want = ext.w4_linear_fused(ext.rmsnorm(x, nw, 1e-6), wq.packed_mma, wq.scales, wq.group, fused.EPI_SILU_MUL)
            got = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_SILU_MUL, norm=(nw, 1e-6))
            assert rel(got, want.double()) < 2e-3, (k, n, scale)


@pytest.mark.parametrize("k,n", [(1536, 2048), (2048, 22016), (2048, 2560), (3584, 512), (256, 4096)])
def test_fused_input_norm_on_the_mfma_gemm(cuda, k, n):
    """2 to 64 rows: the MFMA GEMM normalizes its input in its prologue (each row's sum of squares added in
    lowbit_rmsnorm's order, then its two fp16 roundings as the pieces are staged or the fragments built) -- on the
    one-tile and the row-group kernels, with and without a K split -- the same bits as lowbit_rmsnorm followed by the
    same GEMM, rows of very different scale in one call."""
    wq, _, *_, gen = make_weight(k, n, 7 * k + n, layouts=("mma",), sd=0.05)
    ext = ops.ext()
    nw = (1 + 0.1 * torch.randn(k, generator=gen)).half().cuda()
    bias = (torch.randn(n, generator=gen) * 0.5).half().cuda()
    lib = _native.lib()
    try:
        for m in (2, 16, 17, 33, 48, 64):
            rows = torch.randn(m, k, generator=gen) * torch.logspace(-3, 1.6, m).view(m, 1)
            x = rows.half().cuda()
            for kern in (0, 1, 2):
                # the one-tile kernel normalizes up to 48 rows; a normalized input of more goes to row groups (the
                # plan of kernel 1 and the automatic one's when it takes row groups)
                _native.check(lib.lowbit_set_gemm_kernel(1 if m > 48 else kern))
                xn = ext.rmsnorm(x, nw, 1e-6)
                want = ext.w4_linear_fused(xn, wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias)
                want_sm = ext.w4_linear_fused(xn, wq.packed_mma, wq.scales, wq.group, fused.EPI_SILU_MUL) \
                    if n % 16 == 0 else None
                _native.check(lib.lowbit_set_gemm_kernel(kern))
                got = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias, norm=(nw, 1e-6))
                assert torch.equal(got, want), (k, n, m, kern)
                if want_sm is not None:
                    got = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_SILU_MUL,
                                              norm=(nw, 1e-6))
                    assert torch.equal(got, want_sm), (k, n, m, kern)
                assert torch.equal(ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias,
                                                       norm=(nw, 1e-6)), ext.w4_linear_fused(
                    x, wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias, norm=(nw, 1e-6)))
    finally:
        _native.check(lib.lowbit_set_gemm_kernel(0))
    with pytest.raises(RuntimeError):                          # the prefill GEMM has no fused norm
        x2 = torch.randn(65, k, generator=gen).half().cuda()
        ext.w4_linear_fused(x2, wq.packed_mma, wq.scales, wq.group, fused.EPI_STORE, norm=(nw, 1e-6))


@pytest.mark.parametrize("n,k", [(1000, 2048), (4099, 1536), (64, 8), (151936, 2048), (7, 16384), (1001, 384),
                                 (33, 1000)])
def test_f16_gemv_against_fp32(cuda, n, k):
    """The fp16 head GEMV, 1 to 64 rows: the fp16 rounding of the exact product, up to fp32 summation noise (half an
    fp16 ulp plus 2^-16 of the output RMS); up to 8 rows (the dot2 kernel) each row the same bits as that row alone (a
    row's sum does not depend on how many rows share the call), beyond (the MFMA kernel where K % 128 == 0) the same
    bits on every call; more rows than the dot2 kernel holds are refused where K % 128 != 0."""
    g = torch.Generator(device="cuda").manual_seed(n + k)
    w = (torch.randn(n, k, generator=g, device="cuda") * 0.02).half()
    for m in (1, 2, 3, 4, 5, 8, 9, 16, 17, 33, 64):
        if (m > 16 or m * k * 2 > 65536) and k % 128:
            with pytest.raises(RuntimeError, match="K % 128"):
                ops.ext().f16_gemv(torch.zeros(m, k, dtype=torch.half, device="cuda"), w)
            continue
        x = torch.randn(m, k, generator=g, device="cuda").half()
        y = ops.ext().f16_gemv(x, w)
        ref = x.double() @ w.double().t()
        err = (y.double() - ref).abs()
        ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -14))) - 10)
        assert bool((err <= 0.5 * ulp + 2.0 ** -16 * ref.pow(2).mean().sqrt()).all()), (n, k, m)
        if 1 < m <= 8:
            for r in (0, m // 2, m - 1):
                assert torch.equal(y[r:r + 1], ops.ext().f16_gemv(x[r:r + 1].contiguous(), w)), (n, k, m, r)
        assert torch.equal(y, ops.ext().f16_gemv(x, w)), (n, k, m)
    with pytest.raises(RuntimeError, match="1..64 rows"):
        ops.ext().f16_gemv(torch.zeros(65, 128, dtype=torch.half, device="cuda"), torch.zeros(8, 128, dtype=torch.half,
                                                                                               device="cuda"))


def test_rmsnorm_matches_qwen2_rmsnorm(cuda):
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm
    g = torch.Generator().manual_seed(1)
    for h in (256, 1536, 2048, 3584):
        norm = Qwen2RMSNorm(h, eps=1e-6).cuda().half()
        with torch.no_grad():
            norm.weight.copy_((1 + 0.1 * torch.randn(h, generator=g)).half())
        x = (torch.randn(5, h, generator=g) * 3).half().cuda()
        want = norm(x)
        got = ops.ext().rmsnorm(x, norm.weight.detach(), 1e-6)
        assert ulp_diff(got, want) <= 1, h


def test_rope_and_cache_write_match_transformers(cuda):
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
    m = decode.random_model("tiny", seed=2)
    hq, hkv, L = 2, 1, 64
    g = torch.Generator(device="cuda").manual_seed(3)
    pos = torch.tensor([0, 5, 17, 63], device="cuda")
    qkv = torch.randn(4, (hq + 2 * hkv) * 128, generator=g, device="cuda").half()
    q_out = torch.empty(4, hq, 128, dtype=torch.half, device="cuda")
    k_cache = torch.zeros(hkv, L, 128, dtype=torch.half, device="cuda")
    v_cache = torch.zeros_like(k_cache)
    ops.ext().rope_kv(qkv, pos, m.model.rotary_emb.inv_freq.float(), q_out, k_cache, v_cache, hq, hkv)
    cos, sin = m.model.rotary_emb(qkv.view(1, 4, -1), pos.view(1, -1))
    q = qkv[:, :hq * 128].view(1, 4, hq, 128).transpose(1, 2)
    k = qkv[:, hq * 128:(hq + hkv) * 128].view(1, 4, hkv, 128).transpose(1, 2)
    q_ref, k_ref = apply_rotary_pos_emb(q, k, cos, sin)
    assert ulp_diff(q_out, q_ref[0].transpose(0, 1).contiguous()) <= 1
    assert ulp_diff(k_cache[:, pos], k_ref[0]) <= 1
    assert torch.equal(v_cache[:, pos], qkv[:, (hq + hkv) * 128:].view(4, hkv, 128).transpose(0, 1))
    rest = torch.ones(L, dtype=torch.bool, device="cuda")
    rest[pos] = False
    assert int(torch.count_nonzero(k_cache[:, rest])) == 0 and int(torch.count_nonzero(v_cache[:, rest])) == 0


def test_rope_kv_permuted_layout_equals_unpermuted(cuda):
    hq, hkv, L = 16, 2, 96
    g = torch.Generator(device="cuda").manual_seed(8)
    inv_freq = decode.random_model("tiny", seed=2).model.rotary_emb.inv_freq.float()
    pos = torch.tensor([3, 50, 95], device="cuda")
    qkv = torch.randn(3, (hq + 2 * hkv) * 128, generator=g, device="cuda").half()
    perm = fused.rope_permutation(hq + 2 * hkv).cuda()
    outs = []
    for src, permuted in ((qkv, False), (qkv[:, perm].contiguous(), True)):
        q = torch.empty(3, hq, 128, dtype=torch.half, device="cuda")
        kc, vc = torch.zeros(hkv, L, 128, dtype=torch.half, device="cuda"), torch.zeros(hkv, L, 128, dtype=torch.half, device="cuda")
        ops.ext().rope_kv(src, pos, inv_freq, q, kc, vc, hq, hkv, permuted=permuted)
        outs.append((q, kc, vc))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("hq,hkv,k", [(2, 1, 256), (16, 2, 2048), (12, 2, 1536)])
def test_qkv_rope_equals_projection_then_rope(cuda, hq, hkv, k):
    """lowbit_w4_qkv_rope (RMSNorm, q|k|v GEMV, bias, RoPE, cache write in one launch) gives the same bits as the
    fused-norm projection with the bias epilogue followed by lowbit_rope_kv on the permuted layout. RoPE pairs rows
    r and r + 8 of a tile, so the fused kernel never splits a tile over workgroups; the two-step reference is pinned
    to the same unsplit plan (a split would only reorder its fp32 sums)."""
    n, L = (hq + 2 * hkv) * 128, 64
    wq, _, *_, gen = make_weight(k, n, k + n, layouts=("mma",), sd=0.05)
    ext = ops.ext()
    bias = (torch.randn(n, generator=gen) * 0.5).half().cuda()
    nw = (1 + 0.1 * torch.randn(k, generator=gen)).half().cuda()
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).cuda()
    for p in (0, 37, 63, 64):
        x = (torch.randn(1, k, generator=gen) * 3).half().cuda()
        pos = torch.tensor([p], device="cuda")
        caches = []
        for fused_call in (False, True):
            q = torch.zeros(1, hq, 128, dtype=torch.half, device="cuda")
            kc = torch.zeros(hkv, L, 128, dtype=torch.half, device="cuda")
            vc = torch.zeros_like(kc)
            if fused_call:
                ext.w4_qkv_rope(x, wq.packed_mma, wq.scales, wq.group, bias, pos, inv_freq, q, kc, vc, hq, hkv,
                                norm=(nw, 1e-6))
            else:
                _native.check(_native.lib().lowbit_set_launch_override(0, 0, 1))
                try:
                    qkv = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias,
                                              norm=(nw, 1e-6))
                finally:
                    _native.check(_native.lib().lowbit_set_launch_override(0, 0, 0))
                ext.rope_kv(qkv, pos, inv_freq, q, kc, vc, hq, hkv, permuted=True)
            caches.append((q, kc, vc))
        for a, b in zip(*caches):
            assert torch.equal(a, b), p
        if p >= L:                                          # out of the cache: nothing written, q untouched
            assert int(torch.count_nonzero(caches[1][1])) == 0 and int(torch.count_nonzero(caches[1][0])) == 0


def test_rope_table_holds_the_factors_rope_kv_applies(cuda):
    """lowbit_rope_table's (cos, sin) are exactly the factors lowbit_rope_kv multiplies by: with x = 1 and its
    partner 0, rope_kv's rotated pair is (fp16(1 * cos) - fp16(0 * sin), fp16(0 * cos) + fp16(1 * sin)) = (cos, sin)
    bit for bit. Also within an fp16 ulp of torch's fp32 cos and sin (torch's fp32 functions may differ from the
    device library's in the last fp32 bit, which can move an fp16 rounding)."""
    hq, hkv, L = 2, 1, 70000
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).cuda()
    pos = torch.tensor([0, 1, 37, 4095, 32767, 65535, 69999], device="cuda")
    m = pos.shape[0]
    table = ops.ext().rope_table(pos, inv_freq)
    qkv = torch.zeros(m, (hq + 2 * hkv) * 128, dtype=torch.half, device="cuda")
    qkv.view(m, hq + 2 * hkv, 128)[:, :, :64] = 1
    q = torch.zeros(m, hq, 128, dtype=torch.half, device="cuda")
    kc = torch.zeros(hkv, L, 128, dtype=torch.half, device="cuda")
    ops.ext().rope_kv(qkv, pos, inv_freq, q, kc, torch.zeros_like(kc), hq, hkv)
    cs = table.view(torch.int16).view(m, 64, 2).view(torch.half)
    assert torch.equal(cs[:, :, 0], q[:, 0, :64]) and torch.equal(cs[:, :, 1], q[:, 0, 64:])
    ang = pos.float()[:, None] * inv_freq[None, :]
    assert ulp_diff(cs[:, :, 0].contiguous(), torch.cos(ang).half()) <= 1
    assert ulp_diff(cs[:, :, 1].contiguous(), torch.sin(ang).half()) <= 1


@pytest.mark.parametrize("hq,hkv,k", [(2, 1, 256), (16, 2, 2048), (28, 4, 3584)])
@pytest.mark.parametrize("m", [2, 16, 48, 64, 130, 512])
def test_qkv_rope_rows_equal_projection_then_rope(cuda, hq, hkv, k, m):
    """lowbit_w4_qkv_rope_rows (M tokens: q|k|v GEMM, bias, RoPE from the step's table, cache write in one launch;
    the MFMA GEMM up to 64 rows, the prefill GEMM beyond) gives the same bits as the same GEMM with the bias epilogue
    followed by lowbit_rope_kv on the permuted layout, on the automatic plan and with K split in two and four (both
    sides run the same plan; the split fixup pairs rows r and r + 8 of a tile). Tokens at positions outside the
    cache write nothing, their q included."""
    n, L = (hq + 2 * hkv) * 128, 600
    wq, _, *_, gen = make_weight(k, n, 3 * k + n + m, layouts=("mma",), sd=0.05)
    ext = ops.ext()
    bias = (torch.randn(n, generator=gen) * 0.5).half().cuda()
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).cuda()
    x = (torch.randn(m, k, generator=gen) * 3).half().cuda()
    pos = torch.randperm(L, generator=gen)[:m]
    pos[m // 2] = L + 3                                     # one token outside the cache
    pos = pos.cuda()
    table = ext.rope_table(pos, inv_freq)
    for s in (0, 2, 4):
        outs = []
        for fused_call in (False, True):
            q = torch.zeros(m, hq, 128, dtype=torch.half, device="cuda")
            kc = torch.zeros(hkv, L, 128, dtype=torch.half, device="cuda")
            vc = torch.zeros_like(kc)
            _native.check(_native.lib().lowbit_set_launch_override(0, 0, s))
            try:
                if fused_call:
                    ext.w4_qkv_rope_rows(x, wq.packed_mma, wq.scales, wq.group, bias, pos, table, q, kc, vc, hq, hkv)
                elif m <= 64:
                    qkv = ext.w4_linear_fused(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias)
                else:
                    qkv = ext.w4_gemm_prefill(x, wq.packed_mma, wq.scales, wq.group, fused.EPI_BIAS, bias)
            finally:
                _native.check(_native.lib().lowbit_set_launch_override(0, 0, 0))
            if not fused_call:
                ext.rope_kv(qkv, pos, inv_freq, q, kc, vc, hq, hkv, permuted=True)
            outs.append((q, kc, vc))
        for a, b in zip(*outs):
            assert torch.equal(a, b), (m, s)
        assert int(torch.count_nonzero(outs[1][0][m // 2])) == 0
        written = torch.zeros(L, dtype=torch.bool, device="cuda")
        written[pos[pos < L]] = True
        assert int(torch.count_nonzero(outs[1][1][:, ~written])) == 0
        assert int(torch.count_nonzero(outs[1][1][:, written])) > outs[1][1][:, written].numel() * 0.99


@pytest.mark.parametrize("hq,hkv,k,m", [(16, 2, 2048, 16), (16, 2, 2048, 48), (12, 2, 1536, 33), (2, 1, 256, 5)])
def test_qkv_rope_rows_with_the_input_norm(cuda, hq, hkv, k, m):
    """lowbit_w4_qkv_rope_rows with norm_weight (up to 64 rows: the MFMA GEMM normalizes x itself) against
    lowbit_rmsnorm followed by the same call: the same q and cache rows, bit for bit."""
    n, L = (hq + 2 * hkv) * 128, 300
    wq, _, *_, gen = make_weight(k, n, 5 * k + n + m, layouts=("mma",), sd=0.05)
    ext = ops.ext()
    bias = (torch.randn(n, generator=gen) * 0.5).half().cuda()
    nw = (1 + 0.1 * torch.randn(k, generator=gen)).half().cuda()
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).cuda()
    x = (torch.randn(m, k, generator=gen) * 7).half().cuda()
    pos = torch.randperm(L, generator=gen)[:m].cuda()
    table = ext.rope_table(pos, inv_freq)
    outs = []
    for fused_norm in (False, True):
        q = torch.zeros(m, hq, 128, dtype=torch.half, device="cuda")
        kc = torch.zeros(hkv, L, 128, dtype=torch.half, device="cuda")
        vc = torch.zeros_like(kc)
        if fused_norm:
            ext.w4_qkv_rope_rows(x, wq.packed_mma, wq.scales, wq.group, bias, pos, table, q, kc, vc, hq, hkv,
                                 norm=(nw, 1e-6))
        else:
            ext.w4_qkv_rope_rows(ext.rmsnorm(x, nw, 1e-6), wq.packed_mma, wq.scales, wq.group, bias, pos, table, q, kc,
                                 vc, hq, hkv)
        outs.append((q, kc[:, pos], vc[:, pos]))
    for a, b in zip(*outs):
        assert torch.equal(a, b), m
    with pytest.raises(RuntimeError, match="at most 64 rows"):
        x2 = torch.randn(65, k, generator=gen).half().cuda()
        pos2 = torch.arange(65, device="cuda")
        ext.w4_qkv_rope_rows(x2, wq.packed_mma, wq.scales, wq.group, bias, pos2, ext.rope_table(pos2, inv_freq),
                             torch.zeros(65, hq, 128, dtype=torch.half, device="cuda"), kc, vc, hq, hkv,
                             norm=(nw, 1e-6))


@pytest.mark.parametrize("hq,hkv,L,positions", [(16, 2, 1100, [0]), (16, 2, 1100, [767]), (12, 2, 600, [63, 64, 65]),
                                                (28, 4, 300, list(range(200, 248))), (2, 1, 64, [10, 40]),
                                                (16, 2, 4096, [4095]), (28, 4, 2048, [5, 2047]),
                                                (16, 2, 768, list(range(512, 528))), (16, 2, 600, list(range(100, 400))),
                                                (12, 2, 300, list(range(0, 300, 37)))])
def test_attention_against_fp32_softmax(cuda, hq, hkv, L, positions):
    """Decode steps (a few tokens: one block per (token, head group), key partitions merged by a second launch) and
    multi-token steps and prompts (from 32 query rows per KV head: the MFMA kernel, with and without partitions, merged
    the same way). Repeated calls give the same bits, and the workspace's first 4096 bytes are left untouched."""
    g = torch.Generator(device="cuda").manual_seed(hq + L)
    m = len(positions)
    q = torch.randn(m, hq, 128, generator=g, device="cuda").half()
    k_cache = torch.randn(hkv, L, 128, generator=g, device="cuda").half()
    v_cache = torch.randn(hkv, L, 128, generator=g, device="cuda").half()
    pos = torch.tensor(positions, device="cuda")
    scale = 1 / math.sqrt(128)
    grp = hq // hkv
    ref = torch.empty(m, hq, 128, dtype=torch.float32, device="cuda")
    for i, p in enumerate(positions):
        for h in range(hq):
            kk, vv = k_cache[h // grp, :p + 1].float(), v_cache[h // grp, :p + 1].float()
            w = torch.softmax(kk @ q[i, h].float() * scale, 0)
            ref[i, h] = w @ vv
    # one block per (token, head group), and with the keys split into partitions (decode shapes); a max_keys below
    # the real key count still attends every key (the last partition takes the rest)
    for split, max_keys in ((False, L), (True, L), (True, 40)):
        out = torch.empty(m, hq * 128, dtype=torch.half, device="cuda")
        ops.ext().attention(q, k_cache, v_cache, pos, out, hq, hkv, max_keys, scale, split=split)
        assert rel(out.view(m, hq, 128), ref.double()) < 3e-3, (split, max_keys)
        again = torch.empty_like(out)
        ops.ext().attention(q, k_cache, v_cache, pos, again, hq, hkv, max_keys, scale, split=split)
        assert torch.equal(out, again), (split, max_keys)
    st = _native._stream(q.device)
    ws = _native.workspace(q.device, st, _native.ATTENTION_WORKSPACE_BYTES)
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(ws[:4096])) == 0


@pytest.mark.parametrize("hq,hkv,L,positions", [(12, 2, 300, [63, 64, 65]), (16, 2, 600, list(range(100, 148))),
                                                (28, 4, 2048, list(range(5, 40))), (16, 2, 4096, list(range(700, 716)))])
@pytest.mark.parametrize("poison", [float("nan"), float("inf")])
def test_attention_ignores_unwritten_cache_rows(cuda, hq, hkv, L, positions, poison):
    """Cache rows past the step's last position are never attended: filled with NaN or Inf (an uninitialized cache),
    they leave every output finite and equal to the fp32 softmax over the written rows -- on the decode kernel (few
    query rows per KV head) and on the MFMA kernel (32 or more), with and without key partitions."""
    g = torch.Generator(device="cuda").manual_seed(L + len(positions))
    m = len(positions)
    q = torch.randn(m, hq, 128, generator=g, device="cuda").half()
    k_cache = torch.randn(hkv, L, 128, generator=g, device="cuda").half()
    v_cache = torch.randn(hkv, L, 128, generator=g, device="cuda").half()
    last = max(positions)
    k_cache[:, last + 1:] = poison
    v_cache[:, last + 1:] = poison
    pos = torch.tensor(positions, device="cuda")
    scale = 1 / math.sqrt(128)
    grp = hq // hkv
    ref = torch.empty(m, hq, 128, dtype=torch.float32, device="cuda")
    for i, p in enumerate(positions):
        for h in range(hq):
            kk, vv = k_cache[h // grp, :p + 1].float(), v_cache[h // grp, :p + 1].float()
            ref[i, h] = torch.softmax(kk @ q[i, h].float() * scale, 0) @ vv
    for split in (False, True):
        out = torch.empty(m, hq * 128, dtype=torch.half, device="cuda")
        ops.ext().attention(q, k_cache, v_cache, pos, out, hq, hkv, L, scale, split=split)
        assert bool(torch.isfinite(out).all()), split
        assert rel(out.view(m, hq, 128), ref.double()) < 3e-3, split


@pytest.fixture(scope="module")
def tiny_models():
    torch.cuda.set_device(0)
    return decode.random_model("tiny", seed=21)


def test_fused_greedy_feeds_its_argmax_back_in_the_graph(cuda, tiny_models):
    """FusedDecoder.greedy (replays back to back, the graph writing its argmax into the next input and advancing the
    position) gives the tokens of stepping the same graph with the argmax fed by hand, for fp16 and int4
    projections; step() afterwards still feeds the given token."""
    m = tiny_models
    prompt = torch.randint(0, 1024, (1, 30), generator=torch.Generator(device="cuda").manual_seed(9), device="cuda")
    for quant in ("fp16", "int4"):
        f = fused.FusedQwen2(m, 30 + 40, quant=quant)
        dec = fused.FusedDecoder(f, chunk=1)
        first = dec.prefill(prompt).argmax(-1)
        dec.capture()
        toks = dec.greedy(first, 24)
        ref = fused.FusedDecoder(f, chunk=1)
        nxt = ref.prefill(prompt).argmax(-1)
        ref.capture()
        by_hand = [int(nxt)]
        for _ in range(23):
            by_hand.append(int(ref.step(torch.tensor([by_hand[-1]], device="cuda"))[-1].argmax(-1)))
        assert toks.tolist() == by_hand, quant
        assert dec.pos == ref.pos
        logits = dec.step(torch.tensor([by_hand[-1]], device="cuda")).clone()
        assert torch.equal(logits, ref.step(torch.tensor([by_hand[-1]], device="cuda"))), quant


def test_fused_qwen2_matches_transformers(cuda, tiny_models):
    m = tiny_models
    gen = torch.Generator(device="cuda").manual_seed(5)
    prompt = torch.randint(0, 1024, (1, 70), generator=gen, device="cuda")
    feed = torch.randint(0, 1024, (16,), generator=gen, device="cuda")
    with torch.inference_mode():
        ref = m(torch.cat([prompt[0], feed]).view(1, -1)).logits[0, 70:].float()
    f16 = fused.FusedQwen2(m, 128, quant="fp16")
    dec = fused.FusedDecoder(f16, chunk=1)
    dec.prefill(prompt)
    dec.capture()
    rows = [dec.step(feed[i:i + 1]).float().clone() for i in range(16)]
    got = torch.cat(rows)
    # step i feeds feed[i] at position 70 + i: its logits are the full-sequence forward's at that position
    err = float((got - ref).abs().max() / ref.pow(2).mean().sqrt())
    assert err < 2e-2, err
    assert float((got.argmax(-1) == ref.argmax(-1)).float().mean()) >= 0.9
    # int4: same quantized weights as lowbit.model's W4Linear path (fake-quant reference in torch); 16 tokens per step
    # (MFMA projections, separate RMSNorm) and one (GEMV with the RMSNorm in its prologue)
    q4 = fused.FusedQwen2(m, 128, quant="int4")
    d4 = fused.FusedDecoder(q4, chunk=16)
    d4.prefill(prompt)
    d4.capture()
    got4 = d4.step(feed).float()
    d1 = fused.FusedDecoder(q4, chunk=1)
    d1.prefill(prompt)
    d1.capture()
    got1 = torch.cat([d1.step(feed[i:i + 1]).float().clone() for i in range(16)])
    layers = lbmodel.quantize_layers(m, 128)
    lbmodel.apply_fake_quant(layers)
    with torch.inference_mode():
        ref4 = m(torch.cat([prompt[0], feed]).view(1, -1)).logits[0, 70:].float()
    for got in (got4, got1):
        err4 = float((got - ref4).abs().max() / ref4.pow(2).mean().sqrt())
        assert err4 < 2e-2, err4


@pytest.mark.parametrize("k,n", [(1024, 2560), (16384, 512)])
def test_linear_with_bias_equals_linear_then_add(cuda, k, n):
    """ops.linear's bias (the GEMV, MFMA and prefill kernels add it in their store) gives the bits of linear() then
    `+ bias`, the reference W4Linear's two ops, on every route: v6, v5, dequantize + BLAS, and the long-K prefill."""
    wq, _, *_, gen = make_weight(k, n, k + n, layouts=("mma",), sd=0.05)
    bias = (torch.randn(n, generator=gen) * 0.5).half().cuda()
    for m in (1, 3, 16, 64, 96):
        x = torch.randn(m, k, generator=gen).half().cuda()
        assert torch.equal(ops.linear(x, wq, bias=bias), ops.linear(x, wq) + bias), (k, n, m)


def test_bias_is_normalised_once_for_every_route(cuda):
    """linear() casts a bias of another dtype to fp16 on x's device before routing, so every route (fused GEMV, MFMA,
    dequantize + BLAS) adds the same fp16 values; a bias of the wrong size is refused before any kernel runs."""
    k, n = 1024, 2560
    wq, _, *_, gen = make_weight(k, n, 77, layouts=("mma",), sd=0.05)
    bias32 = torch.randn(n, generator=gen) * 0.5                     # float32, on the CPU
    for m in (1, 16, 300):
        x = torch.randn(m, k, generator=gen).half().cuda()
        assert torch.equal(ops.linear(x, wq, bias=bias32), ops.linear(x, wq, bias=bias32.half().cuda())), m
    with pytest.raises(ValueError, match="bias must hold"):
        ops.linear(torch.zeros(1, k, dtype=torch.half, device="cuda"), wq, bias=torch.zeros(n - 1))


def test_fused_wrappers_refuse_addends_of_the_wrong_size(cuda):
    """The C ABI cannot see the size of aux or of the norm weight; the binding checks them against N, [M, N] and K."""
    k, n = 1024, 512
    wq, *_ = make_weight(k, n, 78, layouts=("mma",))
    e = ops.ext()
    x1 = torch.randn(1, k).half().cuda()
    x4 = torch.randn(4, k).half().cuda()
    call = lambda x, epi, aux=None, norm=None: e.w4_linear_fused(x, wq.packed_mma, wq.scales, 128, epi, aux,  # noqa
                                                                  norm=norm)
    with pytest.raises(RuntimeError, match="bias must hold"):
        call(x1, fused.EPI_BIAS, torch.zeros(n // 2, dtype=torch.half, device="cuda"))
    with pytest.raises(RuntimeError, match="residual must be"):
        call(x4, fused.EPI_RESIDUAL, torch.zeros(1, n, dtype=torch.half, device="cuda"))
    with pytest.raises(RuntimeError, match="need aux"):
        call(x4, fused.EPI_BIAS)
    with pytest.raises(RuntimeError, match="norm weight"):
        call(x1, fused.EPI_STORE, norm=(torch.ones(k // 2, dtype=torch.half, device="cuda"), 1e-6))
    with pytest.raises(RuntimeError, match="norm weight"):
        call(x1, fused.EPI_STORE, norm=(torch.ones(k, dtype=torch.float32, device="cuda"), 1e-6))
    with pytest.raises(RuntimeError, match="bias must hold"):
        e.w4_gemm_prefill(torch.randn(96, k).half().cuda(), wq.packed_mma, wq.scales, 128, fused.EPI_BIAS,
                          torch.zeros(n + 16, dtype=torch.half, device="cuda"))
    with pytest.raises(RuntimeError, match="norm weight"):
        e.rmsnorm(x4, torch.ones(k + 8, dtype=torch.half, device="cuda"), 1e-6)


def test_w4_torch_fallback_rounds_like_the_kernels(cuda):
    """Beyond the kernels' rows a fused W4 projection falls back to dequantize + BLAS with the epilogue in torch: the
    product is rounded to fp16 before the bias or residual is added, as the kernels and linear() + bias do."""
    k, n, m = 2048, 8192, 600                       # wide, short K, many rows: neither the MFMA nor the prefill GEMM
    packed, scales = ops.quantize_w4_gpu(torch.randn(n, k, device="cuda") * 0.02, 128)
    proj = fused._W4(packed, scales, 128)
    assert m > 64 and not ops.prefill_path(m, proj.wq)
    x = torch.randn(m, k, device="cuda").half()
    bias = (torch.randn(n, device="cuda") * 0.5).half()
    plain = torch.nn.functional.linear(x, ops.dequant(proj.wq))
    assert torch.equal(proj(x, fused.EPI_BIAS, bias), plain + bias)
    resid = torch.randn(m, n, device="cuda").half()
    want = resid + plain
    assert torch.equal(proj(x, fused.EPI_RESIDUAL, resid.clone()), want)
    inplace = resid.clone()
    proj(x, fused.EPI_RESIDUAL, inplace, out=inplace)
    assert torch.equal(inplace, want)


def test_capture_allocates_no_workspace(cuda, tiny_models, monkeypatch):
    """The decoders warm up on the stream they capture on, so every library workspace exists before capture (no
    allocation or fill kernel inside a graph), and a second decoder's capture creates none."""
    created = []
    real = _native.workspace

    def watching(device, stream, nbytes=_native.WORKSPACE_BYTES, tag=""):
        key = (device.index if device.index is not None else torch.cuda.current_device(), stream.value, nbytes, tag)
        if key not in _native._WORKSPACES:
            created.append((key, torch.cuda.is_current_stream_capturing()))
        return real(device, stream, nbytes, tag)

    monkeypatch.setattr(_native, "workspace", watching)
    prompt = torch.randint(0, 1024, (1, 20), generator=torch.Generator(device="cuda").manual_seed(3), device="cuda")
    f = fused.FusedQwen2(tiny_models, 64, quant="int4")
    for i, chunk in enumerate((1, 16, 1)):
        dec = fused.FusedDecoder(f, chunk=chunk)
        dec.prefill(prompt)
        before = len(_native._WORKSPACES)
        dec.capture()
        assert not any(during for _, during in created), created
        if i == 2:                                  # a second one-token decoder: its capture creates nothing at all
            assert len(_native._WORKSPACES) == before
        assert bool(torch.isfinite(dec.step(torch.arange(chunk, device="cuda")).float()).all())
