"""One decoded token's attention followed by its output projection in two launches, the key partitions merged in the
projection's prologue (lowbit_w4_attention_linear, lowbit_f16_attention_linear), through the C ABI. The merge uses the
attention's own arithmetic, so the result must be the bits of lowbit_attention -- given a workspace that holds the
same 8 partitions -- followed by the M = 1 fused projection (lowbit_w4_linear_fused / lowbit_f16_linear_fused), for
every epilogue the projection takes (residual in place included), short caches (one partition: the attention writes
its output to the workspace) and long ones, and the head counts of Qwen2.5 1.5B / 3B / 7B; and within the fp32
softmax reference's tolerance."""
import ctypes
import math

import pytest
import torch

from lowbit import _native, fused, ops

from test_gpu_kernels import make_weight

pytestmark = pytest.mark.gpu


def attention_8(q, kc, vc, pos, hq, hkv, max_keys, scale):
    """lowbit_attention with a workspace sized for at most 8 key partitions (the fused call's cap)."""
    out = torch.empty(1, hq * 128, dtype=torch.half, device="cuda")
    ws = torch.empty(4096 + 8 * hq * 132 * 4, dtype=torch.uint8, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _native.check(_native.lib().lowbit_attention(_native.ptr(q), _native.ptr(kc), _native.ptr(vc), _native.ptr(pos),
                                                 _native.ptr(out), 1, hq, hkv, kc.shape[1], max_keys, scale,
                                                 _native.ptr(ws), ws.numel(), st))
    return out


CASES = [(16, 2, 832, 640, 832), (16, 2, 832, 100, 832), (12, 2, 600, 500, 600), (28, 4, 1024, 900, 1024),
         (2, 1, 64, 10, 64), (16, 2, 4096, 4095, 4096), (16, 2, 300, 299, 300)]


@pytest.mark.parametrize("hq,hkv,L,p,max_keys", CASES)
def test_w4_equals_attention_then_projection(cuda, hq, hkv, L, p, max_keys):
    g = torch.Generator(device="cuda").manual_seed(hq * 1000 + p)
    q = torch.randn(1, hq, 128, generator=g, device="cuda").half()
    kc = torch.randn(hkv, L, 128, generator=g, device="cuda").half()
    vc = torch.randn(hkv, L, 128, generator=g, device="cuda").half()
    pos = torch.tensor([p], device="cuda")
    scale = 1 / math.sqrt(128)
    k = hq * 128
    ext = ops.ext()
    attn = attention_8(q, kc, vc, pos, hq, hkv, max_keys, scale)
    # the attention itself against the fp32 softmax
    ref = torch.empty(hq, 128, dtype=torch.float64, device="cuda")
    grp = hq // hkv
    for h in range(hq):
        kk, vv = kc[h // grp, :p + 1].float(), vc[h // grp, :p + 1].float()
        ref[h] = (torch.softmax(kk @ q[0, h].float() * scale, 0) @ vv).double()
    assert float((attn.view(hq, 128).double() - ref).abs().max() / ref.pow(2).mean().sqrt()) < 3e-3
    for n in (2048, 208, 1536):
        wq, *_, wg = make_weight(k, n, k + n + p, layouts=("mma",), sd=0.02)
        bias = (torch.randn(n, generator=wg) * 0.5).half().cuda()
        res = torch.randn(1, n, generator=wg).half().cuda()
        for epi, aux in ((fused.EPI_STORE, None), (fused.EPI_BIAS, bias), (fused.EPI_RESIDUAL, res),
                         (fused.EPI_SILU_MUL, None)):
            if epi == fused.EPI_SILU_MUL and n % 16:
                continue
            want = ext.w4_linear_fused(attn, wq.packed_mma, wq.scales, wq.group, epi, aux)
            got = ext.w4_attention_linear(q, kc, vc, pos, hq, hkv, max_keys, scale, wq.packed_mma, wq.scales, wq.group,
                                          epi, aux)
            assert torch.equal(got, want), (n, epi)
        inplace = res.clone()                                  # the decoder's residual update in place
        ext.w4_attention_linear(q, kc, vc, pos, hq, hkv, max_keys, scale, wq.packed_mma, wq.scales, wq.group,
                                fused.EPI_RESIDUAL, inplace, out=inplace)
        assert torch.equal(inplace, ext.w4_linear_fused(attn, wq.packed_mma, wq.scales, wq.group, fused.EPI_RESIDUAL,
                                                        res))


@pytest.mark.parametrize("hq,hkv,L,p,max_keys", CASES[:4] + CASES[5:6])
def test_f16_equals_attention_then_projection(cuda, hq, hkv, L, p, max_keys):
    g = torch.Generator(device="cuda").manual_seed(hq * 7 + p)
    q = torch.randn(1, hq, 128, generator=g, device="cuda").half()
    kc = torch.randn(hkv, L, 128, generator=g, device="cuda").half()
    vc = torch.randn(hkv, L, 128, generator=g, device="cuda").half()
    pos = torch.tensor([p], device="cuda")
    scale = 1 / math.sqrt(128)
    ext = ops.ext()
    attn = attention_8(q, kc, vc, pos, hq, hkv, max_keys, scale)
    n = 2048
    w = (torch.randn(n, hq * 128, generator=g, device="cuda") * 0.05).half()
    res = torch.randn(1, n, generator=g, device="cuda").half()
    for epi, aux in ((fused.EPI_STORE, None), (fused.EPI_RESIDUAL, res), (fused.EPI_SILU_MUL, None)):
        want = ext.f16_linear_fused(attn, w, epi, aux)
        got = ext.f16_attention_linear(q, kc, vc, pos, hq, hkv, max_keys, scale, w, epi, aux)
        assert torch.equal(got, want), epi


def test_refusals(cuda):
    lib = _native.lib()
    q = torch.zeros(1, 64, 128, dtype=torch.half, device="cuda")
    kc = torch.zeros(8, 64, 128, dtype=torch.half, device="cuda")
    pos = torch.zeros(1, dtype=torch.long, device="cuda")
    w = torch.zeros(256, 64 * 64, dtype=torch.uint8, device="cuda")
    s = torch.zeros(256, 64, dtype=torch.half, device="cuda")
    y = torch.zeros(1, 256, dtype=torch.half, device="cuda")
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    P = _native.ptr
    args = lambda hq, hkv, wsp, nbytes, epi: (P(q), P(kc), P(kc), P(pos), hq, hkv, 64, 64, 0.1, P(w), P(s), P(y), 256,
                                              128, epi, None, wsp, nbytes, st)
    assert lib.lowbit_w4_attention_linear(*args(64, 8, P(ws), ws.numel(), 0)) != 0      # more than 32 query heads
    assert "32 query heads" in lib.lowbit_last_error().decode()
    assert lib.lowbit_w4_attention_linear(*args(16, 2, None, 0, 0)) != 0                # a workspace is required
    assert lib.lowbit_w4_attention_linear(*args(16, 2, P(ws), 4096, 0)) != 0           # too small for one partition
    assert lib.lowbit_w4_attention_linear(*args(16, 2, P(ws), ws.numel(), 4)) != 0     # the RoPE epilogue: no
