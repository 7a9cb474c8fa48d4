"""The BASELINE configurations at full size on the GPU: config 1 (M=1, K=896, N=4864), the M=1 sweep over the
Qwen2.5-1.5B / 3B projections, and the skinny sweep M in {1..64} on the 3B and 7B-shaped MLP layers, each against
fp64 on the same quantized weights (bound 3e-3, reference bench/gpu_run.py:179,245), with N(0, 0.02) weights and
N(0, 1) activations as BASELINE states. Also size-independent properties: linearity in x and the dequant+BLAS path
agreeing with the kernels."""
import numpy as np
import pytest
import torch

from lowbit import ops
from oracle import quant_ref as R

pytestmark = pytest.mark.gpu

SWEEP = [(1536, 1536), (1536, 256), (1536, 8960), (8960, 1536), (2048, 2048), (2048, 256), (2048, 11008), (11008, 2048)]
SKINNY = [(2048, 11008), (11008, 2048), (3584, 18944), (18944, 3584)]


def setup(k, n, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, scales = R.quantize_w4(w, 128)
    wq = ops.W4Weight(packed, scales, 128, ("mma",))
    ref_w = torch.from_numpy(R.dequantize_w4(packed, scales, 128)).cuda().double()
    return wq, ref_w


def rel(y, ref):
    return ((y.double() - ref).abs().max() / ref.pow(2).mean().sqrt()).item()


def test_config1_and_m1_sweep(cuda):
    gen = torch.Generator(device="cuda").manual_seed(0)
    for k, n in [(896, 4864)] + SWEEP:
        wq, ref_w = setup(k, n, k * 7 + n)
        x = torch.randn(1, k, generator=gen, device="cuda").half()
        ref = x.double() @ ref_w.T
        assert rel(ops.linear(x, wq), ref) <= R.REL_BOUND, (k, n)
        assert ops.auto_version(1, wq) == 6


def test_skinny_sweep_and_boundaries(cuda):
    gen = torch.Generator(device="cuda").manual_seed(1)
    for k, n in SKINNY:
        wq, ref_w = setup(k, n, k + n)
        for m in (1, 2, 4, 8, 16, 24, 32, 48, 64, 65):
            x = torch.randn(m, k, generator=gen, device="cuda").half()
            ref = x.double() @ ref_w.T
            e = rel(ops.linear(x, wq), ref)
            assert e <= R.REL_BOUND, (k, n, m, e)
            if m <= 64:
                assert rel(ops.gemv(x, wq, 5), ref) <= R.REL_BOUND, (k, n, m)
        del wq, ref_w
        torch.cuda.empty_cache()


def test_linearity_in_x_at_full_size(cuda):
    """gemv(a x1 + x2) vs a gemv(x1) + gemv(x2): equal up to fp16 rounding of the inputs and outputs."""
    wq, ref_w = setup(11008, 2048, 5)
    gen = torch.Generator(device="cuda").manual_seed(2)
    x1 = torch.randn(1, 11008, generator=gen, device="cuda").half()
    x2 = torch.randn(1, 11008, generator=gen, device="cuda").half()
    xs = (x1.float() * 0.5 + x2.float()).half()
    lhs = ops.gemv(xs, wq, 6).double()
    rhs = 0.5 * ops.gemv(x1, wq, 6).double() + ops.gemv(x2, wq, 6).double()
    ref = xs.double() @ ref_w.T
    assert rel(lhs, ref) <= R.REL_BOUND and rel(rhs, ref) <= 2 * R.REL_BOUND


def test_dequant_blas_and_kernels_agree(cuda):
    wq, ref_w = setup(2048, 11008, 6)
    gen = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(16, 2048, generator=gen, device="cuda").half()
    y_blas = torch.nn.functional.linear(x, ops.dequant(wq, "mma"))
    y_mfma = ops.gemv(x, wq, 5)
    ref = x.double() @ ref_w.T
    assert rel(y_blas, ref) <= R.REL_BOUND and rel(y_mfma, ref) <= R.REL_BOUND
