"""Routing decisions of lowbit.ops.linear and the argument checks of W4Weight / gemv / dequant, on the CPU.

The kernel-calling functions of lowbit.ops (gemv, dequant, prefill) are replaced by a recorder, so only the Python
decisions run. The routing tables are data: the reference's own table (reference tests/test_dispatch.py:24-42, a T4
rule) is reproduced by giving the rule the reference's constants, and the MI355X table is derived from the AUTO_*
constants this library uses; the error messages are the reference's (lowbit/ops.py:33-41,67-78)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
from lowbit import ops  # noqa: E402


class FakeWeight:
    """What linear() / gemv() read from a W4Weight: sizes, group and which packed copies exist (a marker object
    stands for a kept copy, None for one that is not kept)."""

    def __init__(self, n=1024, k=256, keep=("mma",)):
        self.n, self.k, self.group = n, k, 128
        for attr, layout in (("packed", "canonical"), ("packed_v3", "v3"), ("packed_mma", "mma")):
            setattr(self, attr, object() if layout in keep else None)


class Router:
    """Records which path each ops.linear call takes: the GEMV/MFMA version number, "prefill" or "dequant"."""

    def __init__(self, monkeypatch):
        self.taken = []

        def fake_gemv(x, wq, version, rows_per_warp=0):
            self.taken.append(version)
            return torch.zeros(x.shape[0], wq.n)

        def fake_dequant(wq, layout=None):
            self.taken.append("dequant")
            return torch.zeros(wq.n, wq.k)

        def fake_prefill(x, wq):
            self.taken.append("prefill")
            return torch.zeros(x.shape[0], wq.n)

        monkeypatch.setattr(ops, "gemv", fake_gemv)
        monkeypatch.setattr(ops, "dequant", fake_dequant)
        monkeypatch.setattr(ops, "prefill", fake_prefill)

    def route(self, rows, weight, **kwargs):
        self.taken.clear()
        y = ops.linear(torch.zeros(rows, weight.k), weight, **kwargs)
        assert tuple(y.shape) == (rows, weight.n)
        return self.taken[0] if len(self.taken) == 1 else tuple(self.taken)


@pytest.fixture
def router(monkeypatch):
    return Router(monkeypatch)


def mi355x_table():
    """(rows, N, K, expected route) at the edges of every threshold of the MI355X rule (mma layout kept)."""
    one, narrow_rows, narrow_n, max_k = (ops.AUTO_GEMV_ROWS, ops.AUTO_GEMV_NARROW_ROWS, ops.AUTO_GEMV_NARROW_N,
                                         ops.AUTO_GEMV_MAX_K)
    v5, v5_wide, wide = ops.AUTO_V5_ROWS, ops.AUTO_V5_WIDE_ROWS, ops.AUTO_WIDE_N
    past_v5 = "prefill" if ops.AUTO_PREFILL_ROWS > v5 else "dequant"   # what a short-K layer gets beyond v5
    small_n = max(256, wide // 2)
    return [
        (1, small_n, 256, 6), (one, small_n, 256, 6),
        (narrow_rows, small_n, 256, 6), (narrow_rows + 1, small_n, 256, 5),         # narrow layers: GEMV to 3 rows
        (narrow_rows, narrow_n - 16, 256, 6), (one + 1, narrow_n, 256, 5),          # ... only below AUTO_GEMV_NARROW_N
        (narrow_rows, small_n, max_k, 6), (one + 1, small_n, max_k + 128, 5),       # ... and up to AUTO_GEMV_MAX_K
        (1, narrow_n, max_k + 128, 6),                                              # one row is always the GEMV
        (v5, small_n, 256, 5), (v5 + 1, small_n, 256, past_v5),
        (v5_wide, wide, 256, 5), (v5_wide + 1, wide, 256, past_v5),
    ]


@pytest.mark.parametrize("rows,n,k,want", mi355x_table())
def test_mi355x_rule(router, rows, n, k, want):
    assert router.route(rows, FakeWeight(n, k)) == want


# the reference's T4 constants and its routing table (reference lowbit/ops.py:57-59,137-160; tests/test_dispatch.py)
T4_CONSTANTS = {"AUTO_GEMV_ROWS": 1, "AUTO_V5_ROWS": 32, "AUTO_V5_WIDE_ROWS": 64, "AUTO_WIDE_N": 3072,
                "AUTO_GEMV_NARROW_ROWS": 1, "AUTO_PREFILL_ROWS": 0, "AUTO_PREFILL_NARROW_ROWS": 0,
                "AUTO_PREFILL_MIN_K": 1 << 30}
T4_TABLE = [(1, 1024, 6), (2, 1024, 5), (32, 1024, 5), (33, 1024, "dequant"), (33, 4096, 5), (64, 4096, 5),
            (65, 4096, "dequant")]


def test_the_rule_reduces_to_the_reference_table(router, monkeypatch):
    for name, value in T4_CONSTANTS.items():
        monkeypatch.setattr(ops, name, value)
    assert [router.route(rows, FakeWeight(n)) for rows, n, _ in T4_TABLE] == [want for _, _, want in T4_TABLE]


# weights that cannot keep the mma layout: the v3 GEMV (v4) when that copy is kept, else the canonical one (v2), up
# to 8 rows; dequantize + BLAS beyond
NO_MMA_TABLE = [(("canonical", "v3"), 1, 4), (("canonical", "v3"), 8, 4), (("canonical", "v3"), 9, "dequant"),
                (("canonical",), 1, 2), (("canonical",), 8, 2), (("canonical",), 9, "dequant")]


@pytest.mark.parametrize("keep,rows,want", NO_MMA_TABLE)
def test_rule_without_the_device_layout(router, keep, rows, want):
    assert router.route(rows, FakeWeight(keep=keep)) == want


def test_prefill_routing(router):
    """Beyond the MFMA kernel's rows an mma-layout weight takes the int4 prefill GEMM when K is long, when the rows
    are few, or when the layer is small enough; other weights, other layouts and fixed versions dequantize."""
    min_k, few, small, small_rows = (ops.AUTO_PREFILL_MIN_K, ops.AUTO_PREFILL_ROWS, ops.AUTO_PREFILL_NARROW,
                                     ops.AUTO_PREFILL_NARROW_ROWS)
    first = ops.AUTO_V5_ROWS + 1
    wide = max(2 * small, 8192)
    assert small < min_k and few < small_rows
    cases = [
        (first, FakeWeight(1024, min_k), {}, "prefill"), (4096, FakeWeight(1024, 2 * min_k), {}, "prefill"),
        (few, FakeWeight(wide, min_k - 128), {}, "prefill"), (few + 1, FakeWeight(wide, min_k - 128), {}, "dequant"),
        (small_rows, FakeWeight(small, small), {}, "prefill"), (small_rows + 1, FakeWeight(small, small), {}, "dequant"),
        (small_rows, FakeWeight(small + 16, small), {}, "dequant"),
        (small_rows, FakeWeight(small, small + 128), {}, "dequant"),
        (first, FakeWeight(1024, min_k, keep=("canonical",)), {}, "dequant"),
        (first, FakeWeight(1024, min_k), {"version": 5}, "dequant"),
        (1, FakeWeight(1024, min_k), {}, 6), (first - 1, FakeWeight(1024, min_k), {}, 5),
    ]
    for rows, weight, kwargs, want in cases:
        assert router.route(rows, weight, **kwargs) == want, (rows, weight.n, weight.k, kwargs)
        if not kwargs:                                  # prefill_path describes the automatic routing only
            assert ops.prefill_path(rows, weight) == (want == "prefill")


# a fixed version runs up to min(max_gemv_rows, its own limit) rows (v5: 64 whatever max_gemv_rows says), then
# dequantize + BLAS: (rows, version, max_gemv_rows, expected)
FIXED_VERSION_TABLE = [(8, 6, 8, 6), (9, 6, 16, "dequant"), (4, 6, 3, "dequant"), (8, 4, 8, 4), (9, 4, 16, "dequant"),
                       (2, 1, 2, 1), (64, 5, 8, 5), (65, 5, 8, "dequant"), (1, 5, 8, 5)]


@pytest.mark.parametrize("rows,version,limit,want", FIXED_VERSION_TABLE)
def test_fixed_versions_stop_at_their_row_limit(router, rows, version, limit, want):
    every = FakeWeight(keep=("canonical", "v3", "mma"))
    assert router.route(rows, every, version=version, max_gemv_rows=limit) == want


def test_unknown_version_is_refused_and_no_rows_run_nothing(router):
    for bad in (-1, 7, 99):
        with pytest.raises(ValueError, match="version must be"):
            router.route(4, FakeWeight(), version=bad)
    empty = ops.linear(torch.zeros(0, 256), FakeWeight())
    assert tuple(empty.shape) == (0, 1024) and router.taken == []


# (call, expected message) for misuse the Python layer refuses before any GPU work
REFUSALS = [
    (lambda: ops.gemv(torch.zeros(1, 256), FakeWeight(keep=("mma",)), 4), "packed_v3"),
    (lambda: ops.gemv(torch.zeros(1, 256), FakeWeight(keep=("mma",)), 2), "packed"),
    (lambda: ops.gemv(torch.zeros(1, 256), FakeWeight(keep=("canonical",)), 6), "packed_mma"),
    (lambda: ops.gemv(torch.zeros(1, 256), FakeWeight(), 0), "version must be one of"),
    (lambda: ops.dequant(FakeWeight(keep=("mma",)), "canonical"), "not kept"),
    (lambda: ops.prefill(torch.zeros(80, 256), FakeWeight(keep=("canonical",))), "packed_mma"),
]


@pytest.mark.parametrize("call,message", REFUSALS)
def test_python_layer_refusals(call, message):
    with pytest.raises(ValueError, match=message):
        call()


# W4Weight validates the requested layouts against K and the group size before any copy reaches the GPU:
# (K, group, layouts, expected message); packed [4, K / 2] and scales [4, K / group]
CONSTRUCTION_REFUSALS = [(96, 32, ("mma",), "multiples of 128"), (256, 64, ("mma",), "multiples of 128"),
                         (96, 32, ("v3",), "canonical or the mma"), (256, 128, ("v3",), "canonical or the mma"),
                         (256, 128, ("canonical", "int8"), "unknown layout")]


@pytest.mark.parametrize("k,group,layouts,message", CONSTRUCTION_REFUSALS)
def test_weight_construction_refusals(k, group, layouts, message):
    packed, scales = np.zeros((4, k // 2), np.uint8), np.ones((4, k // group), np.float16)
    with pytest.raises(ValueError, match=message):
        ops.W4Weight(packed, scales, group, layouts)


def test_row_major_rows_per_wave_choice():
    """pick_rows mirrors the native rule of the row-major GEMVs: 4 rows per wave from N = 512, else 2 from M = 4."""
    assert [ops.pick_rows(n, m) for n, m in [(512, 1), (4096, 8), (511, 1), (511, 3), (511, 4), (100, 8)]] == \
        [4, 4, 1, 1, 2, 2]
