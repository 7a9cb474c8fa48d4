"""Pins the CPU oracle (oracle/quant_ref.py) before anything is checked against it.

Each function is tied to something other than its own formula: the reference's known-answer tests
(tests/test_quant.py:24-30,49-76,96-118), an independent restatement by exact rational arithmetic or by index
arithmetic, brute force on tiny inputs, invariants, and the committed fixtures (tests/golden/w4_golden.npz).
Each check is chosen so that a plausible slip (wrong nibble order, dropped offset, transposed operand, a rounding
rule other than half-to-even, a scale rounded twice) fails it.
"""
import fractions
import pathlib
import struct

import numpy as np
import pytest

from oracle import quant_ref as R

GOLDEN = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "w4_golden.npz")
CASES = sorted({k[:-5] for k in GOLDEN.files if k.endswith("_meta")})


def assemble_le32(b):
    """uint8 [N, 4 W] -> uint32 [N, W]: byte 4 i + j of a row is bits 8 j .. 8 j + 7 of word i (little-endian),
    computed arithmetically rather than through a dtype view."""
    b = np.asarray(b, np.uint32).reshape(b.shape[0], -1, 4)
    return b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16) | (b[..., 3] << 24)


def place(words, row, word, slot, value):
    words[row, word] |= np.uint32(int(value) << (4 * slot))


# ---- known answers from the reference's tests ----

def test_kat_two_nibbles_per_byte_low_first():
    packed, scales = R.quantize_w4(GOLDEN["kat_layout_w"], 128)
    assert scales[0, 0] == GOLDEN["kat_layout_scale"][0]
    assert np.array_equal(packed[0, :2], GOLDEN["kat_layout_bytes"])


def test_kat_magic_number():
    """binary16 0x6400 is 2^10, where the mantissa step is exactly 1: a nibble u in mantissa bits 0..3 reads as
    1024 + u, in bits 4..7 as 1024 + 16 u; subtracting 1032 from the first leaves u - 8 with no rounding (every
    operand and result is an integer below 2^11). Decoded with the standard library's binary16 codec."""
    def half(bits):
        return struct.unpack("<e", struct.pack("<H", bits))[0]
    for u, want in zip(GOLDEN["kat_magic_u"].tolist(), GOLDEN["kat_magic_value"].tolist()):
        assert half(0x6400 | u) == 1024 + u
        assert half(0x6400 | (u << 4)) == 1024 + 16 * u
        assert half(0x6400 | u) - 1032 == want
        assert float(np.float16(half(0x6400 | u)) - np.float16(1032)) == want


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


def test_reconstruction_within_half_a_step_under_heavy_tails():
    """Absmax scaling never clips: with a heavy-tailed weight (a few outliers set each group's scale) every weight is
    within half a step of code * scale, checked in fp64 per element."""
    rng = np.random.default_rng(203)
    w = (rng.standard_t(3, (40, 768)) * 0.3).astype(np.float32)
    packed, scales = R.quantize_w4(w, 128)
    step = np.repeat(scales.astype(np.float64), 128, axis=1)
    codes = R.unpack_w4(packed).astype(np.float64)
    assert float(np.max(np.abs(w.astype(np.float64) - codes * step) / step)) <= 0.5 + 1e-6


def test_group_peak_takes_the_end_code_and_zero_groups_are_exact():
    """The largest-magnitude weight of a group maps to +7 or -7 with its sign (amax / fp16(amax / 7) is 7 to within
    fp16 rounding); a group of zeros gets scale 1.0 and code 0 throughout, so it dequantizes to exact zeros; no code
    leaves -8..7."""
    rng = np.random.default_rng(204)
    w = (rng.standard_normal((10, 512)) * 40).astype(np.float32)
    w[4, 256:384] = 0.0
    packed, scales = R.quantize_w4(w, 128)
    q = R.unpack_w4(packed).reshape(10, 4, 128)
    g = w.reshape(10, 4, 128)
    for n in range(10):
        for gi in range(4):
            if (n, gi) == (4, 2):
                continue
            i = int(np.abs(g[n, gi]).argmax())
            assert int(q[n, gi, i]) == (7 if g[n, gi, i] > 0 else -7), (n, gi)
    assert scales[4, 2] == 1.0 and not q[4, 2].any()
    assert not R.dequantize_w4(packed, scales, 128)[4, 256:384].any()
    assert int(q.min()) >= R.QMIN and int(q.max()) <= R.QMAX


@pytest.mark.parametrize("call", [
    lambda: R.quantize_w4(np.zeros((2, 200), np.float32), 64),      # K not a multiple of G
    lambda: R.quantize_w4(np.zeros((2, 160), np.float32), 80),      # G not a multiple of 32
    lambda: R.quantize_w4(np.zeros((2, 96), np.float32), 128),      # K smaller than one group
    lambda: R.interleave_for_mma(np.zeros((2, 96), np.uint8)),      # K = 192: not whole 128-k chunks
    lambda: R.interleave_for_mfma(np.zeros((3, 32), np.uint8)),     # K = 64
])
def test_shapes_outside_the_format_raise(call):
    with pytest.raises(ValueError):
        call()


# ---- layouts: each value placed where the specification puts it (packing direction) ----

def _random_codes(seed, n, k):
    """Nibbles u in 0..15 and the canonical bytes holding them, packed by definition (byte j: u[2 j] low nibble,
    u[2 j + 1] high nibble)."""
    u = np.random.default_rng(seed).integers(0, 16, (n, k))
    canon = np.zeros((n, k // 2), np.uint8)
    for row in range(n):
        for kk in range(k):
            canon[row, kk // 2] |= np.uint8(int(u[row, kk]) << (4 * (kk % 2)))
    return u, canon


def test_canonical_words_place_value_k_at_nibble_k_mod_8():
    """In the canonical layout read as little-endian words, value k sits in word k // 8 at nibble k % 8, and the
    oracle's unpack recovers every value."""
    u, canon = _random_codes(205, 5, 256)
    words = np.zeros((5, 32), np.uint32)
    for row in range(5):
        for k in range(256):
            place(words, row, k // 8, k % 8, u[row, k])
    assert np.array_equal(assemble_le32(canon), words)
    assert np.array_equal(R.unpack_w4(canon).astype(np.int64) + 8, u)


def test_v3_words_place_even_values_low_and_odd_values_high():
    """v3 order: value k0 + p of a word goes to nibble slot p / 2 when p is even (low half) and 4 + (p - 1) / 2
    when odd (high half), so a (k0 + 2 j, k0 + 2 j + 1) pair lands in the two 16-bit halves at the same shift."""
    u, canon = _random_codes(206, 5, 256)
    words = np.zeros((5, 32), np.uint32)
    for row in range(5):
        for k in range(256):
            p = k % 8
            place(words, row, k // 8, p // 2 + 4 * (p % 2), u[row, k])
    assert np.array_equal(assemble_le32(R.interleave_for_gpu(canon)), words)


def test_nv_mma_words_hold_the_fragment_pairs():
    """NVIDIA m16n8k8 order: word i of 16-byte group t of 128-k chunk c holds, in nibble pair j, the values
    k = 128 c + 32 i + 8 j + 2 t (low half) and k + 1 (high half)."""
    n, k_dim = 4, 512
    u, canon = _random_codes(207, n, k_dim)
    words = np.zeros((n, k_dim // 8), np.uint32)
    for row in range(n):
        for c in range(k_dim // 128):
            for t in range(4):
                for i in range(4):
                    for j in range(4):
                        k = 128 * c + 32 * i + 8 * j + 2 * t
                        place(words, row, 16 * c + 4 * t + i, j, u[row, k])
                        place(words, row, 16 * c + 4 * t + i, 4 + j, u[row, k + 1])
    assert np.array_equal(assemble_le32(R.interleave_for_mma(canon)), words)


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
