"""linear() routing and W4Weight validation, on the CPU (no kernel runs: gemv / dequant are stubbed).
A port of the reference's tests/test_dispatch.py:1-64; the routing table follows the AUTO_* constants."""
import types

import numpy as np
import pytest

torch = pytest.importorskip("torch")
from lowbit import ops  # noqa: E402


def weight(n=1024, k=256, layouts=("mma",)):
    have = lambda name: object() if name in layouts else None  # noqa: E731
    return types.SimpleNamespace(n=n, k=k, group=128, packed=have("canonical"), packed_v3=have("v3"), packed_mma=have("mma"))


@pytest.fixture
def calls(monkeypatch):
    seen = []
    monkeypatch.setattr(ops, "gemv", lambda x, wq, v, rpw=0: seen.append(v) or torch.zeros(x.shape[0], wq.n))
    monkeypatch.setattr(ops, "dequant", lambda wq, layout=None: seen.append("dequant") or torch.zeros(wq.n, wq.k))
    monkeypatch.setattr(ops, "prefill", lambda x, wq: seen.append("prefill") or torch.zeros(x.shape[0], wq.n))
    return seen


def _rule_cases():
    g, v5, v5w, wide = ops.AUTO_GEMV_ROWS, ops.AUTO_V5_ROWS, ops.AUTO_V5_WIDE_ROWS, ops.AUTO_WIDE_N
    gn, gwide, kmax = ops.AUTO_GEMV_NARROW_ROWS, ops.AUTO_GEMV_NARROW_N, ops.AUTO_GEMV_MAX_K
    narrow, wide_n = max(256, wide // 2), wide
    past = "prefill" if v5w + 1 <= ops.AUTO_PREFILL_ROWS else "dequant"   # beyond the MFMA kernel's rows
    return [(1, narrow, 256, 6), (g, narrow, 256, 6), (gn, narrow, 256, 6), (gn + 1, narrow, 256, 5),
            (g + 1, gwide, 256, 5), (gn, gwide - 16, 256, 6), (g + 1, narrow, kmax + 128, 5), (gn, narrow, kmax, 6),
            (1, gwide, kmax + 128, 6), (v5, narrow, 256, 5), (v5 + 1, narrow, 256, past),
            (v5 + 1, wide_n, 256, 5 if v5w > v5 else past), (v5w, wide_n, 256, 5),
            (v5w + 1, wide_n, 256, past)]


@pytest.mark.parametrize("m,n,k,want", _rule_cases())
def test_auto_rule_on_the_mma_layout(calls, m, n, k, want):
    ops.linear(torch.zeros(m, k), weight(n, k))
    assert calls == [want]


def test_reference_table_with_the_t4_constants(calls, monkeypatch):
    """The rule's structure reproduces the reference's own table when given the reference's (T4) constants (and no
    int4 prefill GEMM, which the reference does not have)."""
    for name, value in (("AUTO_GEMV_ROWS", 1), ("AUTO_V5_ROWS", 32), ("AUTO_V5_WIDE_ROWS", 64), ("AUTO_WIDE_N", 3072),
                        ("AUTO_GEMV_NARROW_ROWS", 1), ("AUTO_PREFILL_ROWS", 0), ("AUTO_PREFILL_NARROW_ROWS", 0),
                        ("AUTO_PREFILL_MIN_K", 1 << 30)):
        monkeypatch.setattr(ops, name, value)
    for m, n, want in [(1, 1024, 6), (2, 1024, 5), (32, 1024, 5), (33, 1024, "dequant"), (33, 4096, 5), (64, 4096, 5),
                       (65, 4096, "dequant")]:
        calls.clear()
        ops.linear(torch.zeros(m, 256), weight(n))
        assert calls == [want]


def test_prefill_rule(calls):
    """Beyond the MFMA kernel's rows, the int4 prefill GEMM takes long-K weights at any M, every weight up to
    AUTO_PREFILL_ROWS rows and small layers up to AUTO_PREFILL_NARROW_ROWS; the rest, other layouts and fixed
    versions keep dequantize + BLAS; decode rows never reach it."""
    kmin, few, small, small_rows = ops.AUTO_PREFILL_MIN_K, ops.AUTO_PREFILL_ROWS, ops.AUTO_PREFILL_NARROW, \
        ops.AUTO_PREFILL_NARROW_ROWS
    rows = ops.AUTO_V5_ROWS + 1
    big = max(2 * small, 8192)
    assert small < kmin and few < small_rows
    for m, n, k, layouts, version, want in [
            (rows, 1024, kmin, ("mma",), 0, "prefill"), (4096, 1024, 2 * kmin, ("mma",), 0, "prefill"),
            (few, big, kmin - 128, ("mma",), 0, "prefill"), (few + 1, big, kmin - 128, ("mma",), 0, "dequant"),
            (small_rows, small, small, ("mma",), 0, "prefill"), (small_rows + 1, small, small, ("mma",), 0, "dequant"),
            (small_rows, small + 16, small, ("mma",), 0, "dequant"), (small_rows, small, small + 128, ("mma",), 0, "dequant"),
            (rows, 1024, kmin, ("canonical",), 0, "dequant"), (rows, 1024, kmin, ("mma",), 5, "dequant"),
            (1, 1024, kmin, ("mma",), 0, 6), (rows - 1, 1024, kmin, ("mma",), 0, 5)]:
        calls.clear()
        ops.linear(torch.zeros(m, k), weight(n, k, layouts), version=version)
        assert calls == [want], (m, n, k, layouts, version)


@pytest.mark.parametrize("layouts,m,want", [(("canonical", "v3"), 1, 4), (("canonical", "v3"), 8, 4),
                                            (("canonical",), 3, 2), (("canonical", "v3"), 9, "dequant")])
def test_auto_rule_without_the_mma_layout(calls, layouts, m, want):
    ops.linear(torch.zeros(m, 256), weight(layouts=layouts))
    assert calls == [want]


def test_a_fixed_version_never_passes_its_row_limit(calls):
    ops.linear(torch.zeros(9, 256), weight(), max_gemv_rows=16, version=6)      # v6 takes at most 8 rows
    ops.linear(torch.zeros(64, 256), weight(), version=5)
    ops.linear(torch.zeros(65, 256), weight(), version=5)
    assert calls == ["dequant", 5, "dequant"]


def test_bad_versions_and_empty_input(calls):
    with pytest.raises(ValueError):
        ops.linear(torch.zeros(4, 256), weight(), version=7)
    assert ops.linear(torch.zeros(0, 256), weight()).shape == (0, 1024)
    assert calls == []


def test_gemv_refuses_a_layout_the_weight_does_not_keep():
    with pytest.raises(ValueError, match="packed_v3"):
        ops.gemv(torch.zeros(1, 256), weight(layouts=("mma",)), 4)
    with pytest.raises(ValueError, match="version must be one of"):
        ops.gemv(torch.zeros(1, 256), weight(), 7)


def test_construction_checks_layouts_before_touching_the_gpu():
    packed, scales = np.zeros((4, 48), np.uint8), np.ones((4, 3), np.float16)       # K = 96, G = 32
    with pytest.raises(ValueError, match="multiples of 128"):
        ops.W4Weight(packed, scales, 32, ("mma",))
    with pytest.raises(ValueError, match="canonical or the mma"):
        ops.W4Weight(packed, scales, 32, ("v3",))
    with pytest.raises(ValueError, match="unknown layout"):
        ops.W4Weight(packed, scales, 32, ("nope",))


def test_dequant_refuses_a_layout_not_kept():
    with pytest.raises(ValueError, match="not kept"):
        ops.dequant(weight(layouts=("mma",)), "canonical")


def test_pick_rows_mirrors_the_native_choice():
    assert [ops.pick_rows(n, m) for n, m in [(512, 1), (511, 1), (511, 4), (100, 8)]] == [4, 1, 2, 2]
