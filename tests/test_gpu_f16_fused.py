"""The fp16-weight mode of the one-row GEMV (lowbit_f16_linear_fused, lowbit_f16_qkv_rope): the W4A16 decode's fp16
comparator, through the C ABI.
* the plain store against an fp32 torch product of the same fp16 operands (fp32 accumulation in another order:
  within one fp16 ulp of the fp64 value plus 2^-16 of the output RMS), on ragged N, every tile split the planner
  can pick and forced wave counts;
* bias and residual give the bits of the same kernel's store plus the torch add, silu-mul is within one ulp of
  torch's silu(gate) * up on the stored rows, the fused input norm within the unfused norm's tolerance;
* the q|k|v projection with RoPE and the cache write gives the bits of the bias-epilogue projection followed by
  lowbit_rope_kv on the permuted layout;
* FusedQwen2(quant="fp16_gemv") against the hipBLASLt fp16 variant on the same tokens (same weights, another
  summation order), and its graph decode against eager stepping."""
import pytest
import torch
import torch.nn.functional as F

from lowbit import _native, decode, fused, ops

from test_gpu_gemv_splits import same_up_to_order

pytestmark = pytest.mark.gpu


def rel(y, ref):
    return float((y.double() - ref).abs().max() / ref.pow(2).mean().sqrt())


@pytest.fixture
def reset_override():
    yield
    _native.check(_native.lib().lowbit_set_launch_override(0, 0, 0))


@pytest.mark.parametrize("k,n", [(1536, 256), (2048, 2560), (2048, 200), (11008, 2048), (128, 40), (8960, 1536)])
def test_store_against_fp32_product(cuda, reset_override, k, n):
    g = torch.Generator(device="cuda").manual_seed(k + n)
    w = (torch.randn(n, k, generator=g, device="cuda") * 0.05).half()
    x = torch.randn(1, k, generator=g, device="cuda").half()
    ref = x.double() @ w.double().T
    ext = ops.ext()
    base = ext.f16_linear_fused(x, w, fused.EPI_STORE)
    assert same_up_to_order(base.double(), ref, ref), (k, n)
    for waves, splits in ((1, 1), (4, 1), (16, 1), (0, 2), (0, 4), (2, 4)):
        if (k // 32) % splits:
            continue
        _native.check(_native.lib().lowbit_set_launch_override(waves, 0, splits))
        y = ext.f16_linear_fused(x, w, fused.EPI_STORE)
        assert same_up_to_order(y.double(), ref, ref), (k, n, waves, splits)
        assert torch.equal(ext.f16_linear_fused(x, w, fused.EPI_STORE), y)


@pytest.mark.parametrize("k,n", [(2048, 2048), (1536, 208), (2048, 22016)])
def test_epilogues_and_norm(cuda, k, n):
    g = torch.Generator(device="cuda").manual_seed(3 * k + n)
    w = (torch.randn(n, k, generator=g, device="cuda") * 0.05).half()
    x = torch.randn(1, k, generator=g, device="cuda").half()
    bias = (torch.randn(n, generator=g, device="cuda") * 0.5).half()
    res = torch.randn(1, n, generator=g, device="cuda").half()
    nw = (torch.rand(k, generator=g, device="cuda") + 0.5).half()
    ext = ops.ext()
    plain = ext.f16_linear_fused(x, w, fused.EPI_STORE)
    assert torch.equal(ext.f16_linear_fused(x, w, fused.EPI_BIAS, bias), plain + bias)
    assert torch.equal(ext.f16_linear_fused(x, w, fused.EPI_RESIDUAL, res), res + plain)
    inplace = res.clone()
    ext.f16_linear_fused(x, w, fused.EPI_RESIDUAL, inplace, out=inplace)
    assert torch.equal(inplace, res + plain)
    gu = plain.view(1, -1, 2, 8)
    want = (F.silu(gu[:, :, 0].float()).half().float() * gu[:, :, 1].float()).half().reshape(1, -1)
    got = ext.f16_linear_fused(x, w, fused.EPI_SILU_MUL)
    assert int((got.view(torch.int16).int() - want.view(torch.int16).int()).abs().max()) <= 1
    normed = ext.rmsnorm(x, nw, 1e-6)
    want_n = ext.f16_linear_fused(normed, w, fused.EPI_STORE)
    got_n = ext.f16_linear_fused(x, w, fused.EPI_STORE, norm=(nw, 1e-6))
    assert rel(got_n, want_n.double()) < 2e-3


@pytest.mark.parametrize("hq,hkv,k", [(2, 1, 256), (16, 2, 2048), (12, 2, 1536)])
def test_qkv_rope_equals_projection_then_rope(cuda, reset_override, hq, hkv, k):
    n, L = (hq + 2 * hkv) * 128, 64
    g = torch.Generator(device="cuda").manual_seed(k + n)
    w = (torch.randn(n, k, generator=g, device="cuda") * 0.05).half()
    bias = (torch.randn(n, generator=g, device="cuda") * 0.5).half()
    nw = (1 + 0.1 * torch.randn(k, generator=g, device="cuda")).half()
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).cuda()
    ext = ops.ext()
    for p in (0, 37, 64):
        x = (torch.randn(1, k, generator=g, device="cuda") * 3).half()
        pos = torch.tensor([p], device="cuda")
        outs = []
        for fused_call in (False, True):
            q = torch.zeros(1, hq, 128, dtype=torch.half, device="cuda")
            kc = torch.zeros(hkv, L, 128, dtype=torch.half, device="cuda")
            vc = torch.zeros_like(kc)
            if fused_call:
                ext.f16_qkv_rope(x, w, bias, pos, inv_freq, q, kc, vc, hq, hkv, norm=(nw, 1e-6))
            else:                                           # RoPE pairs rows r, r + 8: the unsplit plan on both sides
                _native.check(_native.lib().lowbit_set_launch_override(0, 0, 1))
                qkv = ext.f16_linear_fused(x, w, fused.EPI_BIAS, bias, norm=(nw, 1e-6))
                _native.check(_native.lib().lowbit_set_launch_override(0, 0, 0))
                ext.rope_kv(qkv, pos, inv_freq, q, kc, vc, hq, hkv, permuted=True)
            outs.append((q, kc, vc))
        for a, b in zip(*outs):
            assert torch.equal(a, b), p


def test_refusals(cuda):
    ext = ops.ext()
    x = torch.randn(1, 200, device="cuda").half()
    w = torch.randn(64, 200, device="cuda").half()
    with pytest.raises(RuntimeError, match="multiple of 128"):
        ext.f16_linear_fused(x, w, fused.EPI_STORE)
    x2 = torch.randn(2, 256, device="cuda").half()
    with pytest.raises(RuntimeError, match=r"x \[1, K\]"):
        ext.f16_linear_fused(x2, torch.randn(64, 256, device="cuda").half(), fused.EPI_STORE)


def test_fused_qwen2_fp16_gemv_matches_the_blas_variant(cuda):
    m = decode.random_model("tiny", seed=22)
    gen = torch.Generator(device="cuda").manual_seed(6)
    prompt = torch.randint(0, 1024, (1, 40), generator=gen, device="cuda")
    feed = torch.randint(0, 1024, (12,), generator=gen, device="cuda")
    outs = {}
    for quant in ("fp16", "fp16_gemv"):
        f = fused.FusedQwen2(m, 64, quant=quant)
        dec = fused.FusedDecoder(f, chunk=1)
        dec.prefill(prompt)
        dec.capture()
        outs[quant] = torch.cat([dec.step(feed[i:i + 1]).float().clone() for i in range(12)])
        if quant == "fp16_gemv":                              # graph replay == eager forward, bit for bit
            eager = fused.FusedDecoder(f, chunk=1)
            eager.prefill(prompt)
            rows = []
            for i in range(12):
                pos = torch.tensor([40 + i], device="cuda")
                rows.append(f(feed[i:i + 1], pos).float())
            assert torch.equal(torch.cat(rows), outs[quant])
    a, b = outs["fp16_gemv"], outs["fp16"]
    assert rel(a, b.double()) < 1e-2
    assert float((a.argmax(-1) == b.argmax(-1)).float().mean()) >= 0.9
