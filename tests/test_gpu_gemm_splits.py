"""The MFMA GEMM's launch shapes (row tiles per wave, ring slots, K split across workgroups with the workspace
fixup) against the fp64 oracle, through the C ABI. Every shape must meet the same bound as the automatic one
(max(4 x BLAS, 4 x fp16-output floor, 3e-3), bench/gpu_run.py:229-245), be the fp16 rounding of the exact product
up to fp32 accumulation noise (every (u - 8) x product is exact), repeat bit for bit, and leave the workspace's arrival
counters at zero; zero weights stay exactly zero under every split."""
import ctypes

import numpy as np
import pytest
import torch

from lowbit import _native, ops
from oracle import quant_ref as R

from test_gpu_kernels import bound, make_weight, rel
from test_gpu_prefill import assert_rounds

pytestmark = pytest.mark.gpu

# (column tiles, row tiles per wave, ring slots, K-groups) the library builds: kernels.hpp gemm_fits
def fits(mt, rw, d, ks, tw=4):
    if tw == 3:
        return rw == 1 and d == 2 and (ks <= 2 or mt <= 2)
    if tw != 4:
        return rw == 1 and (d == 2 or (d == 3 and tw in (5, 6))) and ks <= 2 and (tw * ks <= 12 or mt <= 3)
    if ks == 4:
        return (mt <= 3 if rw == 1 else mt <= 2) if d == 2 else (rw == 1 and mt == 1)
    if ks == 2:
        return not ((rw == 2 and (d >= 3 if mt >= 3 else (mt == 2 and d == 4))) or (mt == 4 and rw == 1 and d == 4))
    return True


def gemm(x, wq, rw, d, splits, ws, ks=0, tw=0):
    lib = _native.lib()
    n = wq.packed_mma.shape[0]
    y = torch.empty(x.shape[0], n, dtype=torch.half, device="cuda")
    _native.check(lib.lowbit_set_launch_override(4 * ks, d, splits))
    _native.check(lib.lowbit_set_gemm_tile_waves(tw))
    try:
        _native.check(lib.lowbit_w4_gemm_mfma(_native.ptr(x), _native.ptr(wq.packed_mma), _native.ptr(wq.scales),
                                              _native.ptr(y), x.shape[0], n, x.shape[1], wq.group, rw,
                                              _native.ptr(ws) if ws is not None else None,
                                              ws.numel() if ws is not None else 0,
                                              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    finally:
        _native.check(lib.lowbit_set_launch_override(0, 0, 0))
        _native.check(lib.lowbit_set_gemm_tile_waves(0))
    return y


@pytest.mark.parametrize("k,n", [(1024, 1001), (2048, 4096), (11008, 640), (384, 37), (3584, 200)])
def test_every_launch_shape_against_fp64(cuda, k, n):
    wq, ref_w, *_, gen = make_weight(k, n, k + 3 * n, layouts=("mma",))
    ws = _native.workspace(torch.device("cuda", 0), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    for m in (1, 3, 16, 17, 33, 64):
        x = torch.randn(m, k, generator=gen).half().cuda()
        ref = x.double() @ ref_w.T
        lim = bound(x, ref_w, ref)
        mt = (m + 15) // 16
        for rw in (1, 2):
            for d in (2, 3, 4):
                for ks in (1, 2, 4):
                    if not fits(mt, rw, d, ks):
                        continue
                    for splits in (1, 3, 32):
                        y = gemm(x, wq, rw, d, splits, ws, ks)
                        e = rel(y, ref)
                        assert e <= lim, (k, n, m, rw, d, ks, splits, e, lim)
                        assert_rounds(y, ref)
                        assert torch.equal(y, gemm(x, wq, rw, d, splits, ws, ks)), (k, n, m, rw, d, ks, splits)
        y0 = gemm(x, wq, 0, 0, 0, None)                  # no workspace: no split
        assert rel(y0, ref) <= lim
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(ws[:_native.WORKSPACE_COUNTER_BYTES])) == 0


@pytest.mark.parametrize("k,n", [(1024, 16 * 37 + 5), (3584, 4096), (2048, 16 * 101)])
def test_k_group_widths_give_the_bits_of_four_tile_waves(cuda, k, n):
    """K-groups of 3, 5, 6 or 8 tile-waves (one tile per wave; 5 and 6 also with a 3-slot ring) compute every tile as
    K-groups of 4 do: the same chunks per K-group in the same order, so the bits are the same, with and without a K
    split. The tile counts leave a partial last workgroup, and 16 M rows over 3, 5 or 6 waves a partial last round of
    x staging."""
    wq, ref_w, *_, gen = make_weight(k, n, k + n, layouts=("mma",))
    ws = _native.workspace(torch.device("cuda", 0), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    for m in (1, 16, 17, 40, 64):
        x = torch.randn(m, k, generator=gen).half().cuda()
        ref = x.double() @ ref_w.T
        lim = bound(x, ref_w, ref)
        mt = (m + 15) // 16
        for ks in (1, 2, 4):
            if not fits(mt, 1, 2, ks):
                continue
            for splits in (1, 3):
                base = gemm(x, wq, 1, 2, splits, ws, ks, tw=4)
                assert rel(base, ref) <= lim, (k, n, m, ks, splits)
                for tw in (3, 5, 6, 8):
                    for d in (2, 3):
                        if not fits(mt, 1, d, ks, tw):
                            continue
                        y = gemm(x, wq, 1, d, splits, ws, ks, tw)
                        assert torch.equal(y, base), (k, n, m, ks, splits, tw, d)
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(ws[:_native.WORKSPACE_COUNTER_BYTES])) == 0


def test_automatic_tile_waves_balance_the_rounds(cuda):
    """Past 1024 tiles the planner takes the fewest tile-waves that fit one round of workgroups (3584 x 18944: 1184
    tiles -> 237 workgroups of 5, with 2 K-groups; a 3-slot ring at 24 rows, 2 at 64); the result equals that launch
    forced with 2 slots, bit for bit (the ring depth does not change the order of the chunks)."""
    wq, ref_w, *_, gen = make_weight(3584, 18944, 7, layouts=("mma",))
    ws = _native.workspace(torch.device("cuda", 0), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    for m in (24, 64):
        x = torch.randn(m, 3584, generator=gen).half().cuda()
        auto = ops.ext().w4_gemm_tc(x, wq.packed_mma, wq.scales, wq.group)
        ref = x.double() @ ref_w.T
        assert rel(auto, ref) <= bound(x, ref_w, ref)
        assert torch.equal(auto, gemm(x, wq, 1, 2, 1, ws, 2, tw=5)), m


@pytest.mark.parametrize("n,cases", [(16 * 700, ((8, 3, 4), (40, 4, 2))), (16 * 1000, ((16, 4, 4),))])
def test_automatic_k_groups_fill_the_cus(cuda, n, cases):
    """Up to 16 rows, layers of 385-768 tiles take 4 K-groups of 3 tile-waves (700 tiles -> 234 workgroups) and a
    layer of 256 row groups of 4 still takes 4 K-groups; beyond 16 rows the 700 tiles keep 4 tile-waves, 2 K-groups.
    Each result equals that launch forced, bit for bit."""
    wq, ref_w, *_, gen = make_weight(1024, n, 11, layouts=("mma",))
    ws = _native.workspace(torch.device("cuda", 0), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    for m, tw, ks in cases:
        x = torch.randn(m, 1024, generator=gen).half().cuda()
        auto = ops.ext().w4_gemm_tc(x, wq.packed_mma, wq.scales, wq.group)
        ref = x.double() @ ref_w.T
        assert rel(auto, ref) <= bound(x, ref_w, ref)
        assert torch.equal(auto, gemm(x, wq, 1, 2, 1, ws, ks, tw=tw)), (n, m)


def test_zero_weights_stay_zero_under_every_split(cuda):
    rng = np.random.default_rng(5)
    n, k = 96, 4096
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[::2] = 0.0
    packed, scales = R.quantize_w4(w, 128)
    wq = ops.W4Weight(packed, scales, 128, ("mma",))
    ws = _native.workspace(torch.device("cuda", 0), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    for m in (2, 16, 40):
        x = torch.from_numpy((rng.standard_normal((m, k)) * 30).astype(np.float16)).cuda()
        ref = torch.from_numpy(R.gemv_reference(x.double().cpu().numpy(), packed, scales, 128)).cuda()
        for splits, ks in ((1, 1), (2, 2), (7, 4), (16, 2)):
            y = gemm(x, wq, 2, 2, splits, ws, ks)
            assert torch.count_nonzero(y[:, ::2]) == 0, (m, splits)
            assert rel(y, ref) <= R.REL_BOUND, (m, splits)


def test_tiny_activations_keep_their_precision(cuda):
    """Rows of tiny activations (down to fp16 subnormals) keep the same relative accuracy as rows of ordinary and of
    large ones: every product is formed exactly, whatever the magnitude of x."""
    wq, ref_w, *_, gen = make_weight(1024, 256, 99, layouts=("mma",))
    ws = _native.workspace(torch.device("cuda", 0), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    x = torch.randn(4, 1024, generator=gen)
    x[0] *= 1e-5
    x[1] *= 3e-3
    x[2, ::7] = 300.0
    x = x.half().cuda()
    ref = x.double() @ ref_w.T
    for m in range(4):
        ym = gemm(x, wq, 2, 4, 4, ws)[m:m + 1]
        assert rel(ym, ref[m:m + 1]) <= R.REL_BOUND, m


@pytest.mark.parametrize("k,n", [(11008, 2048), (3584, 200), (18944, 3584), (2048, 1001)])
def test_split_order_gives_the_same_bits(cuda, k, n):
    """The workgroup order of a K-split launch (row groups fastest, or splits fastest so that one split's workgroups
    share an XCD) only changes where the workgroups run: the same bits at every split count and row count, the
    counters left at zero."""
    wq, ref_w, *_, gen = make_weight(k, n, 7 * k + n, layouts=("mma",))
    ws = _native.workspace(torch.device("cuda", 0), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    lib = _native.lib()
    try:
        for m in (2, 16, 48, 64):
            x = torch.randn(m, k, generator=gen).half().cuda()
            for splits in (0, 2, 3, 8, 16):
                outs = []
                for order in (1, 2):
                    _native.check(lib.lowbit_set_gemm_order(order))
                    outs.append(gemm(x, wq, 1, 0, splits, ws))
                assert torch.equal(outs[0], outs[1]), (k, n, m, splits)
            assert rel(outs[1], x.double() @ ref_w.T) <= bound(x, ref_w, x.double() @ ref_w.T)
    finally:
        _native.check(lib.lowbit_set_gemm_order(0))
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(ws[:_native.WORKSPACE_COUNTER_BYTES])) == 0
