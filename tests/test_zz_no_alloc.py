"""lowbit_w4_gemm_mfma_noalloc (the MFMA GEMM with the library's own device scratch instead of a caller workspace)
against lowbit_w4_gemm_mfma with a workspace of the same size, through the C ABI: the same bits on two calls in a
row, the second with a smaller input, on shapes that split K over workgroups (the scratch's arrival counters and
partial sums in use) and on one that does not; both within the fp64 bound of the oracle's dequantized weights. The
same call captured in a hipGraph and replayed between eager calls gives the eager bits on every replay."""
import ctypes

import pytest
import torch

from lowbit import _native
from oracle import quant_ref as R

from test_gpu_kernels import bound, make_weight, rel

pytestmark = pytest.mark.gpu


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def with_workspace(x, wq, ws):
    n = wq.packed_mma.shape[0]
    y = torch.empty(x.shape[0], n, dtype=torch.half, device=x.device)
    _native.check(_native.lib().lowbit_w4_gemm_mfma(
        _native.ptr(x), _native.ptr(wq.packed_mma), _native.ptr(wq.scales), _native.ptr(y), x.shape[0], n,
        x.shape[1], wq.group, 0, _native.ptr(ws), ws.numel(), _stream()))
    return y


def without_allocation(x, wq, y=None):
    n = wq.packed_mma.shape[0]
    y = torch.empty(x.shape[0], n, dtype=torch.half, device=x.device) if y is None else y
    _native.check(_native.lib().lowbit_w4_gemm_mfma_noalloc(
        _native.ptr(x), _native.ptr(wq.packed_mma), _native.ptr(wq.scales), _native.ptr(y), x.shape[0], n,
        x.shape[1], wq.group, 0, _stream()))
    return y


# (M, K, N) in call order: 3B down at 48 rows (row groups, K split 8 ways), then a smaller 1.5B-down-shaped call
# (K split), then a q/o-shaped call the one-tile-per-workgroup kernel takes (no scratch use), then the first again
CALLS = [(48, 11008, 2048), (5, 8960, 1536), (16, 2048, 2048), (48, 11008, 2048)]


def test_noalloc_equals_the_workspace_entry_point(cuda):
    print(f"noalloc: calls {CALLS}", flush=True)
    ws = torch.zeros(_native.WORKSPACE_BYTES, dtype=torch.uint8, device=cuda)
    weights = {}
    for i, (m, k, n) in enumerate(CALLS):
        if (k, n) not in weights:
            weights[(k, n)] = make_weight(k, n, 7 * k + n, layouts=("mma",))
        wq, ref_w, *_, gen = weights[(k, n)]
        x = torch.randn(m, k, generator=torch.Generator().manual_seed(i)).half().cuda()
        y_free = without_allocation(x, wq)
        y_ws = with_workspace(x, wq, ws)
        torch.cuda.synchronize()
        assert torch.equal(y_free, y_ws), f"call {i} (M={m}, K={k}, N={n}) differs from the workspace entry point"
        ref = x.double() @ ref_w.T
        assert rel(y_free, ref) <= bound(x, ref_w, ref), f"call {i}: outside the fp64 bound"
        assert torch.equal(without_allocation(x, wq), y_free), f"call {i}: not repeatable"
    # the workspace entry point left its counters at zero; the scratch's are checked by the repeats above
    assert int(ws[:_native.WORKSPACE_COUNTER_BYTES].count_nonzero()) == 0


def test_noalloc_replays_in_a_graph(cuda):
    m, k, n = CALLS[1]
    wq, ref_w, *_ = make_weight(k, n, 7 * k + n, layouts=("mma",))
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(99)).half().cuda()
    eager = without_allocation(x, wq)
    y = torch.empty_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        without_allocation(x, wq, y)                      # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        without_allocation(x, wq, y)
    for replay in range(4):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {replay}"
        other = without_allocation(x[:2].contiguous(), wq)      # eager work on the same scratch between replays
        torch.cuda.synchronize()
        assert torch.equal(other, without_allocation(x[:2].contiguous(), wq))
    ref = x.double() @ ref_w.T
    assert rel(y, ref) <= bound(x, ref_w, ref)


def test_noalloc_refuses_what_the_workspace_entry_point_refuses(cuda):
    lib = _native.lib()
    fake = ctypes.c_void_p(4096)
    assert lib.lowbit_w4_gemm_mfma_noalloc(fake, fake, fake, fake, 65, 16, 128, 128, 0, None) == 5
    assert lib.lowbit_w4_gemm_mfma_noalloc(fake, fake, fake, fake, 4, 16, 128, 128, 3, None) == 8
    assert R.REL_BOUND == 3e-3
