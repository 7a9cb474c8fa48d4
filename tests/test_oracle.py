"""Pins the CPU oracle (oracle/quant_ref.py) before anything is checked against it.

Each function is tied to something other than its own formula: the reference's known-answer tests
(tests/test_quant.py:24-30,49-76,96-118), an independent restatement by exact rational arithmetic or by index
arithmetic, brute force on tiny inputs, invariants, and the committed fixtures (tests/golden/w4_golden.npz).
Each check is chosen so that a plausible slip (wrong nibble order, dropped offset, transposed operand, a rounding
rule other than half-to-even, a scale rounded twice) fails it.
"""
import fractions
import pathlib

import numpy as np
import pytest

from oracle import quant_ref as R

GOLDEN = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "w4_golden.npz")
CASES = sorted({k[:-5] for k in GOLDEN.files if k.endswith("_meta")})


def words_of(packed):
    return np.ascontiguousarray(packed).view("<u4")


# ---- known answers from the reference's tests ----

def test_kat_two_nibbles_per_byte_low_first():
    packed, scales = R.quantize_w4(GOLDEN["kat_layout_w"], 128)
    assert scales[0, 0] == GOLDEN["kat_layout_scale"][0]
    assert np.array_equal(packed[0, :2], GOLDEN["kat_layout_bytes"])


def test_kat_magic_number():
    u = GOLDEN["kat_magic_u"]
    h = (u | 0x6400).view(np.float16)
    assert np.array_equal(h.astype(np.float32) - 1032.0, GOLDEN["kat_magic_value"])
    assert np.array_equal(h - np.float16(1032), GOLDEN["kat_magic_value"].astype(np.float16))


def test_kat_overflow_case_closed_form():
    c = R.OVERFLOW_CASE
    packed = np.full((c["n"], c["k"] // 2), c["byte"], np.uint8)
    scales = np.full((c["n"], 1), c["scale"], np.float16)
    for xv, want in GOLDEN["kat_overflow"]:
        y = R.gemv_reference(np.full((1, c["k"]), xv), packed, scales, c["k"])
        assert np.all(y == want)                                   # 7 * 2^-10 * x * 128, exact in fp64


# ---- quantize: independent exact-arithmetic restatement and invariants ----

def _f16_of_exact(fr):
    """Round an exact rational to float32 (nearest, ties even), then to float16 -- the reference's two roundings."""
    f32 = np.float32(float(fr))                     # float(fr) is correctly rounded to fp64
    # fp64 -> fp32 is a second rounding; redo it exactly: pick the fp32 neighbour nearest to fr
    lo = np.nextafter(f32, np.float32(-np.inf))
    hi = np.nextafter(f32, np.float32(np.inf))
    best = min((lo, f32, hi), key=lambda v: (abs(fractions.Fraction(float(v)) - fr),
                                             int(np.array(v, np.float32).view(np.uint32)) & 1))
    return np.float16(best)


def test_quantize_scale_matches_exact_arithmetic():
    rng = np.random.default_rng(101)
    w = (rng.standard_normal((6, 512)) * rng.choice([1e-4, 0.02, 3.0, 2000.0], (6, 1))).astype(np.float32)
    _, scales = R.quantize_w4(w, 128)
    for n in range(6):
        for g in range(4):
            amax = fractions.Fraction(float(np.abs(w[n, 128 * g:128 * (g + 1)]).max()))
            want = _f16_of_exact(amax / 7)
            assert scales[n, g].view(np.uint16) == np.float16(want).view(np.uint16)


def test_quantize_brute_force_nearest_level():
    """Every q is the nearest level of -8..7 to w / scale (ties to even), by exhaustive search."""
    rng = np.random.default_rng(102)
    w = rng.standard_normal((4, 256)).astype(np.float32)
    packed, scales = R.quantize_w4(w, 128)
    q = R.unpack_w4(packed)
    for n in range(4):
        for k in range(256):
            s = np.float32(scales[n, k // 128])
            t = np.float32(w[n, k] / s)                            # the fp32 quotient the format rounds
            levels = np.arange(-8, 8)
            d = np.abs(levels - np.float64(t))
            best = levels[d == d.min()]
            want = best[0] if len(best) == 1 else best[best % 2 == 0][0]
            assert q[n, k] == want


def test_error_is_at_most_half_a_step():
    rng = np.random.default_rng(103)
    w = rng.standard_normal((64, 512)).astype(np.float32)
    packed, scales = R.quantize_w4(w, 128)
    err = np.abs(R.dequantize_w4(packed, scales, 128) - w).reshape(64, 4, 128)
    assert np.all(err <= scales.astype(np.float32)[..., None] / 2 + 1e-6)


def test_range_and_zero_group():
    rng = np.random.default_rng(104)
    w = rng.standard_normal((8, 256)).astype(np.float32) * 50
    w[3] = 0
    packed, scales = R.quantize_w4(w, 128)
    q = R.unpack_w4(packed)
    assert q.min() >= -8 and q.max() <= 7
    assert np.all(scales[3] == 1.0) and np.all(R.dequantize_w4(packed, scales, 128)[3] == 0)


def test_rejects_bad_shapes():
    with pytest.raises(ValueError):
        R.quantize_w4(np.zeros((4, 100), np.float32), 128)
    with pytest.raises(ValueError):
        R.quantize_w4(np.zeros((4, 96), np.float32), 48)
    with pytest.raises(ValueError):
        R.interleave_for_mma(np.zeros((1, 32), np.uint8))
    with pytest.raises(ValueError):
        R.interleave_for_mfma(np.zeros((1, 32), np.uint8))


# ---- layouts: bit logic simulated lane by lane ----

def test_canonical_words_v2_bit_logic():
    rng = np.random.default_rng(105)
    packed, _ = R.quantize_w4(rng.standard_normal((5, 256)).astype(np.float32))
    u = R.unpack_w4(packed) + 8
    words = words_of(packed)
    for b in range(8):
        assert np.array_equal((words >> (4 * b)) & 0xF, u[:, b::8])


def test_v3_words_bit_logic():
    rng = np.random.default_rng(106)
    packed, _ = R.quantize_w4(rng.standard_normal((5, 256)).astype(np.float32))
    u = R.unpack_w4(packed) + 8
    words = words_of(R.interleave_for_gpu(packed)).astype(np.uint64)
    for j in range(4):
        t = (words >> (4 * j)) & 0x000F000F
        assert np.array_equal(t & 0xFFFF, u[:, 2 * j::8])
        assert np.array_equal(t >> 16, u[:, 2 * j + 1::8])


def test_nv_mma_layout_feeds_each_lane_its_fragment():
    rng = np.random.default_rng(5)
    packed, _ = R.quantize_w4(rng.standard_normal((3, 384)).astype(np.float32))
    u = R.unpack_w4(packed) + 8
    words = R.interleave_for_mma(packed).reshape(3, -1, 4, 4, 4).view("<u4")[..., 0]
    for c in range(3):
        for t in range(4):
            for s in range(16):
                w, j = int(words[1, c, t, s >> 2]), s & 3
                k = 128 * c + 8 * s + 2 * t
                assert (w >> (4 * j)) & 0xF == u[1, k] and (w >> (4 * j + 16)) & 0xF == u[1, k + 1]


@pytest.mark.parametrize("n", [1, 5, 16, 21, 37])
def test_mfma_layout_lane_simulation(n):
    """Lane l of the wave that reads 1 KB block (tile t, chunk c) takes bytes [16 l, 16 l + 16): row 16 t + l // 4,
    k = 128 c + 32 (l % 4) + 8 j + {2e, 2e + 1} from word j, nibble pair e (v3 order)."""
    k_dim = 384
    rng = np.random.default_rng(n)
    packed, _ = R.quantize_w4(rng.standard_normal((n, k_dim)).astype(np.float32))
    u = R.unpack_w4(packed) + 8
    flat = R.interleave_for_mfma(packed).reshape(-1)
    for t in range((n + 15) // 16):
        rows = min(16, n - 16 * t)
        for c in range(k_dim // 128):
            block = flat[16 * t * k_dim // 2 + c * rows * 64:][:rows * 64]
            for lane in range(4 * rows):
                r, qq = lane // 4, lane % 4
                words = block[16 * lane:16 * lane + 16].view("<u4")
                for j in range(4):
                    for e in range(4):
                        pair = (int(words[j]) >> (4 * e)) & 0x000F000F
                        k = 128 * c + 32 * qq + 8 * j + 2 * e
                        assert pair & 0xF == u[16 * t + r, k] and pair >> 16 == u[16 * t + r, k + 1]


def test_layouts_are_permutations():
    rng = np.random.default_rng(107)
    packed, _ = R.quantize_w4(rng.standard_normal((19, 256)).astype(np.float32))
    for fn in (R.interleave_for_gpu, R.interleave_for_mma, R.interleave_for_mfma):
        out = fn(packed)
        assert out.shape == packed.shape
        assert sorted(R.unpack_w4(out).ravel().tolist()) == sorted(R.unpack_w4(packed).ravel().tolist())


# ---- dequant and the fp64 GEMV ----

def test_dequant_f16_is_fp64_product_rounded_once():
    rng = np.random.default_rng(108)
    packed = rng.integers(0, 256, (4, 64), dtype=np.uint8)
    # scales from deep subnormal to large, so the one rounding is exercised where it matters
    scales = np.array([[2.0 ** -24], [3.1e-5], [0.0123], [1900.0]], np.float16)
    got = R.dequantize_w4_f16(packed, scales, 128)
    q = R.unpack_w4(packed)
    for n in range(4):
        for k in range(128):
            want = np.float16(float(q[n, k]) * float(scales[n, 0]))
            assert got[n, k].view(np.uint16) == want.view(np.uint16)


def test_torch_dequant_is_fp64_product_rounded_once():
    """The reference's torch dequantize, restated for the CPU baseline (dequantize_w4_torch), gives the bits of
    fp16(fp64 product) element by element: a swapped nibble order, a missing offset or a second rounding fails here."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(109)
    packed = rng.integers(0, 256, (5, 128), dtype=np.uint8)
    scales = np.array([[2.0 ** -24, 1.0], [3.1e-5, 6.1e-5], [0.0123, 0.5], [1900.0, 60000.0], [7.0, 0.1]], np.float16)
    got = R.dequantize_w4_torch(packed, scales, 128)
    assert got.dtype == torch.float16 and tuple(got.shape) == (5, 256)
    got = got.numpy()
    for n in range(5):
        for k in range(256):
            u = (int(packed[n, k // 2]) >> (4 * (k % 2))) & 0xF
            want = np.float16((u - 8) * float(scales[n, k // 128]))
            assert got[n, k].view(np.uint16) == want.view(np.uint16), (n, k)
    assert np.array_equal(got.view(np.uint16), R.dequantize_w4_f16(packed, scales, 128).view(np.uint16))
    w = rng.standard_normal((16, 512)).astype(np.float32)
    p2, s2 = R.quantize_w4(w, 64)
    assert np.array_equal(R.dequantize_w4_torch(p2, s2, 64).numpy().view(np.uint16),
                          R.dequantize_w4_f16(p2, s2, 64).view(np.uint16))
    x = torch.from_numpy(rng.standard_normal((2, 512)).astype(np.float16))
    y = R.cpu_torch_linear(x, p2, s2, 64)
    assert R.rel_err(y.numpy(), R.gemv_reference(x.double().numpy(), p2, s2, 64)) < R.REL_BOUND


def test_gemv_reference_brute_force():
    rng = np.random.default_rng(109)
    packed, scales = R.quantize_w4(rng.standard_normal((5, 256)).astype(np.float32), 128)
    x = rng.standard_normal((2, 256))
    y = R.gemv_reference(x, packed, scales, 128)
    q = R.unpack_w4(packed)
    for m in range(2):
        for n in range(5):
            want = sum(x[m, k] * float(q[n, k]) * float(scales[n, k // 128]) for k in range(256))
            assert abs(y[m, n] - want) <= 1e-12 * max(1.0, abs(want))


def test_rel_err_closed_form():
    ref = np.array([3.0, -4.0])                                    # RMS = sqrt(12.5)
    assert R.rel_err(ref + np.array([0.5, 0.0]), ref) == pytest.approx(0.5 / np.sqrt(12.5))


# ---- clip search: invariants (no reference vector exists) ----

def test_clip_search_invariants():
    rng = np.random.default_rng(110)
    w = (rng.standard_normal((12, 512)) * 0.02).astype(np.float32)
    w[2, :128] = 0
    grid = R.CLIP_GRID
    packed, scales, idx, errs = R.quantize_w4_clip(w, 128, grid)
    g = w.reshape(12, 4, 128).astype(np.float64)
    amax = np.abs(w.reshape(12, 4, 128)).max(-1)
    for n in range(12):
        for gi in range(4):
            i = idx[n, gi]
            # the chosen scale is the candidate of grid entry i
            a = grid[i]
            num = np.float32(amax[n, gi] * np.float32(a)) if a != 1.0 else amax[n, gi]
            cand = np.float16(np.float32(num) / np.float32(7))
            cand = np.float16(1.0) if cand == 0 else cand
            assert scales[n, gi].view(np.uint16) == cand.view(np.uint16)
            # its fp32 error is the minimum, and no earlier entry ties it
            assert errs[i, n, gi] == errs[:, n, gi].min()
            assert np.all(errs[:i, n, gi] > errs[i, n, gi])
            # the fp32 error agrees with an fp64 recomputation from the packed result
            q = R.unpack_w4(packed)[n, 128 * gi:128 * (gi + 1)].astype(np.float64)
            e64 = ((q * float(scales[n, gi]) - g[n, gi]) ** 2).sum()
            assert abs(e64 - errs[i, n, gi]) <= 1e-5 * max(e64, 1e-30)
    assert np.all(scales[2, 0] == 1.0)


def test_clip_search_without_grid_is_absmax():
    rng = np.random.default_rng(111)
    w = rng.standard_normal((7, 384)).astype(np.float32)
    p0, s0 = R.quantize_w4(w, 128)
    p1, s1, idx, _ = R.quantize_w4_clip(w, 128, None)
    assert np.array_equal(p0, p1) and np.array_equal(s0.view(np.uint16), s1.view(np.uint16)) and not idx.any()


# ---- the committed fixtures ----

@pytest.mark.parametrize("case", CASES)
def test_oracle_reproduces_golden_fixtures(case):
    n, k, g, m, seed = GOLDEN[f"{case}_meta"]
    packed, scales = R.quantize_w4(GOLDEN[f"{case}_w"], int(g))
    assert np.array_equal(packed, GOLDEN[f"{case}_packed"])
    assert np.array_equal(scales.view(np.uint16), GOLDEN[f"{case}_scales"].view(np.uint16))
    assert np.array_equal(R.interleave_for_gpu(packed), GOLDEN[f"{case}_v3"])
    if k % 128 == 0:
        assert np.array_equal(R.interleave_for_mma(packed), GOLDEN[f"{case}_nvmma"])
        assert np.array_equal(R.interleave_for_mfma(packed), GOLDEN[f"{case}_mfma"])
    assert np.array_equal(R.dequantize_w4_f16(packed, scales, int(g)).view(np.uint16),
                          GOLDEN[f"{case}_dequant16"].view(np.uint16))
    y = R.gemv_reference(GOLDEN[f"{case}_x"].astype(np.float64), packed, scales, int(g))
    assert np.allclose(y, GOLDEN[f"{case}_y64"], rtol=1e-12, atol=1e-12)


def test_golden_clip_case():
    p, s, idx, _ = R.quantize_w4_clip(GOLDEN["clip_w"], 128, R.CLIP_GRID)
    assert np.array_equal(p, GOLDEN["clip_packed"]) and np.array_equal(idx, GOLDEN["clip_index"])
    assert np.array_equal(s.view(np.uint16), GOLDEN["clip_scales"].view(np.uint16))
