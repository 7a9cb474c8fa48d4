"""lowbit.quant, the product's host-side format functions (native host code), checked against the format
specification of reference lowbit/quant.py:1-84 and against the oracle.

Each check is derived from the specification rather than from an existing test: known answers worked out by hand,
layouts rebuilt in the packing direction (value -> word) instead of decoded, fp16 bit patterns read with the standard
library's binary16 codec, and the fp64 GEMV against a plain Python triple loop."""
import pathlib
import struct

import numpy as np
import pytest

from lowbit import quant
from oracle import quant_ref as R

GOLDEN = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "w4_golden.npz")

# ---- known answers (hand-derived from the specification) ----
# (leading values of a row whose other entries are 0, group size, expected scale, expected leading bytes)
#   * [7, -7, 1, 0]: absmax 7 -> scale 1, nibbles 15, 1, 9, 8 -> 0x1F, 0x89 (the reference's own known answer,
#     tests/test_quant.py:24-30);
#   * halving every value halves the scale and keeps the codes;
#   * [7, 0.5, 1.5, 2.5]: round half to even gives 0, 2, 2 -> nibbles 15, 8, 10, 10 -> 0x8F, 0xAA;
#   * G = 32, [-7, 7, -3.5, 3.5]: -3.5 rounds to -4 and 3.5 to 4 -> nibbles 1, 15, 4, 12 -> 0xF1, 0xC4; the second
#     group is all zeros, so its scale is 1.0.
KNOWN_ANSWERS = [
    ([7.0, -7.0, 1.0, 0.0], 128, [1.0], [0x1F, 0x89, 0x88]),
    ([3.5, -3.5, 0.5, 0.0], 128, [0.5], [0x1F, 0x89, 0x88]),
    ([7.0, 0.5, 1.5, 2.5], 128, [1.0], [0x8F, 0xAA, 0x88]),
    ([-7.0, 7.0, -3.5, 3.5], 32, [1.0, 1.0], [0xF1, 0xC4, 0x88]),
]


@pytest.mark.parametrize("lead,group,want_scales,want_bytes", KNOWN_ANSWERS)
def test_known_answers(lead, group, want_scales, want_bytes):
    row = np.zeros((1, max(128, len(want_scales) * group)), np.float32)
    row[0, :len(lead)] = lead
    packed, scales = quant.quantize_w4(row, group)
    assert scales.dtype == np.float16 and scales.shape == (1, row.shape[1] // group)
    assert scales[0, :len(want_scales)].tolist() == want_scales
    assert packed[0, :len(want_bytes)].tolist() == want_bytes
    assert packed.shape == (1, row.shape[1] // 2)


def _random_weight(seed, n, k, sd):
    return (np.random.default_rng(seed).standard_normal((n, k)) * sd).astype(np.float32)


@pytest.mark.parametrize("group", [32, 64, 128, 256])
def test_each_code_is_the_nearest_level_and_scales_follow_absmax(group):
    """Spec: scale = fp16(amax / 7) per group (1.0 for a zero group); q = the nearest integer to w / scale, ties to
    even, clipped to -8..7. Checked per element against an fp64 evaluation of the same definition."""
    w = _random_weight(group, 24, 512, 0.05)
    w[5, :group] = 0.0
    packed, scales = quant.quantize_w4(w, group)
    groups = w.reshape(24, -1, group)
    amax = np.abs(groups).max(-1)
    want = (amax / np.float32(7)).astype(np.float16)
    want[want == 0] = 1.0
    assert np.array_equal(scales.view(np.uint16), want.view(np.uint16))
    ratio = groups.astype(np.float64) / scales.astype(np.float64)[..., None]
    q = quant.unpack_w4(packed).reshape(24, -1, group).astype(np.float64)
    assert np.all(np.abs(q - np.clip(ratio, -8, 7)) <= 0.5 + 1e-9)
    ties = np.abs(np.abs(ratio - np.trunc(ratio)) - 0.5) < 1e-12
    assert np.all(q[ties] % 2 == 0)
    assert np.all(q[5, 0] == 0) and scales[5, 0] == 1.0


def test_reconstruction_error_and_range():
    w = _random_weight(11, 16, 1024, 3.0)
    packed, scales = quant.quantize_w4(w, 128)
    codes = quant.unpack_w4(packed)
    assert codes.dtype == np.int8 and codes.min() >= quant.QMIN and codes.max() <= quant.QMAX
    back = quant.dequantize_w4(packed, scales, 128)
    half_step = np.repeat(scales.astype(np.float32), 128, axis=1) / 2
    assert np.all(np.abs(back - w) <= half_step * (1 + 1e-6))
    # dequantize is exactly code * scale in float32 (at most 15 significant bits: no rounding)
    assert np.array_equal(back, codes.astype(np.float32) * np.repeat(scales.astype(np.float32), 128, axis=1))


@pytest.mark.parametrize("k,group", [(100, 128), (96, 48), (200, 40), (64, 128)])
def test_shapes_the_format_cannot_hold_are_refused(k, group):
    with pytest.raises(ValueError):
        quant.quantize_w4(np.ones((3, k), np.float32), group)


def test_three_dimensional_input_is_refused():
    with pytest.raises(ValueError):
        quant.quantize_w4(np.ones((2, 2, 128), np.float32), 128)


# ---- byte and word layouts, rebuilt from the specification in the packing direction ----

def _codes(seed, n, k, low=0):
    """Random nibbles u in low..15 and their canonical packing, built by hand: byte j = u[2j] | u[2j+1] << 4."""
    u = np.random.default_rng(seed).integers(low, 16, size=(n, k)).astype(np.uint8)
    return u, _pack(u)


def _pack(u):
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def _words(u, slot_to_k):
    """Little-endian 32-bit words of 8 values each: nibble slot s of word i holds u[8 i + slot_to_k[s]]."""
    n, k = u.shape
    blocks = u.reshape(n, k // 8, 8).astype(np.uint32)
    out = np.zeros((n, k // 8), np.uint32)
    for s, kk in enumerate(slot_to_k):
        out |= blocks[:, :, kk] << np.uint32(4 * s)
    return out


def test_canonical_packing_and_unpacking():
    u, _ = _codes(1, 6, 256, low=1)
    u[:, ::128] = 15                                # amax 7 * 0.25 in every group pins the scale to 0.25
    canonical = _pack(u)
    w = (u.astype(np.float32) - 8) * 0.25          # exact multiples of the scale: the codes come back unchanged
    packed, scales = quant.quantize_w4(w, 128)
    assert np.all(scales == 0.25)
    assert np.array_equal(packed, canonical)
    assert np.array_equal(quant.unpack_w4(packed), u.astype(np.int8) - 8)
    # a GPU reading 32-bit words sees value k0 + s in nibble slot s (the v1 / v2 kernels' order)
    assert np.array_equal(packed.view("<u4"), _words(u, range(8)))


def test_v3_word_order():
    u, canonical = _codes(2, 5, 384)
    assert np.array_equal(quant.interleave_for_gpu(canonical).view("<u4"), _words(u, [0, 2, 4, 6, 1, 3, 5, 7]))
    assert quant.SLOT_TO_K.tolist() == [0, 2, 4, 6, 1, 3, 5, 7]


def test_reference_mma_layout():
    """The reference's m16n8k8 order (lowbit/quant.py:67-78): inside each 64-byte chunk, byte 16 t + s is canonical
    byte 4 s + t; then every word takes the v3 order."""
    u, canonical = _codes(3, 4, 512)
    regrouped = np.empty_like(canonical)
    for c in range(512 // 128):
        for t in range(4):
            for s in range(16):
                regrouped[:, 64 * c + 16 * t + s] = canonical[:, 64 * c + 4 * s + t]
    u_regrouped = np.empty_like(u)
    u_regrouped[:, 0::2], u_regrouped[:, 1::2] = regrouped & 0xF, regrouped >> 4
    want = _words(u_regrouped, [0, 2, 4, 6, 1, 3, 5, 7])
    assert np.array_equal(quant.interleave_for_mma(canonical).view("<u4"), want)


@pytest.mark.parametrize("n", [16, 21, 40])
def test_mfma_device_layout(n):
    """This library's device layout: 16-row tiles (the last holds n % 16 rows); tile t starts at byte 8 t K; in a
    tile with `rows` rows, the 128-k chunk c is rows x 64 bytes at 64 rows c, row r at 64 r inside it; words in v3
    order."""
    k = 384
    u, canonical = _codes(n, n, k)
    v3 = quant.interleave_for_gpu(canonical)
    want = np.empty(n * k // 2, np.uint8)
    for row in range(n):
        t, r = divmod(row, 16)
        rows = min(16, n - 16 * t)
        for c in range(k // 128):
            at = 8 * t * k + 64 * rows * c + 64 * r
            want[at:at + 64] = v3[row, 64 * c:64 * c + 64]
    assert np.array_equal(quant.interleave_for_mfma(canonical).reshape(-1), want)


def test_layouts_refuse_k_that_is_not_whole_chunks():
    for fn in (quant.interleave_for_mma, quant.interleave_for_mfma):
        with pytest.raises(ValueError):
            fn(np.zeros((2, 48), np.uint8))


def test_fp16_magic_number_decodes():
    """0x6400 | u reads as 1024 + u (mantissa step 1 on [1024, 2048)); with the nibble in bits 4..7 it reads
    1024 + 16 u. Read with the standard library's IEEE binary16 codec."""
    half = lambda bits: struct.unpack("<e", struct.pack("<H", bits))[0]   # noqa: E731
    for u in range(16):
        assert half(0x6400 | u) - 1032 == u - 8
        assert half(0x6400 | (u << 4)) / 16 - 72 == u - 8
        assert half(u) == u * 2.0 ** -24                 # the subnormal decode the GEMV and MFMA kernels use
        assert half(u << 4) == u * 2.0 ** -20


def test_fp64_gemv_reference_against_a_triple_loop():
    w = _random_weight(9, 5, 256, 1.0)
    x = np.random.default_rng(10).standard_normal((3, 256))
    packed, scales = quant.quantize_w4(w, 64)
    y = quant.gemv_reference(x, packed, scales, 64)
    codes = quant.unpack_w4(packed)
    for m in range(3):
        for n in range(5):
            want = sum(float(x[m, kk]) * float(codes[n, kk]) * float(scales[n, kk // 64]) for kk in range(256))
            assert abs(y[m, n] - want) <= 1e-12 * max(1.0, abs(want))
    with pytest.raises(ValueError):
        quant.gemv_reference(x[:, :128], packed, scales, 64)


# ---- bit-for-bit agreement with the oracle and the committed fixtures ----

@pytest.mark.parametrize("n,k,g,sd", [(5, 256, 128, 0.02), (33, 384, 128, 1.0), (7, 96, 32, 1e-3), (17, 320, 64, 50.0),
                                      (16, 1024, 256, 0.02), (1, 128, 128, 1e4), (3, 2048, 128, 3e-6)])
def test_host_functions_match_the_oracle(n, k, g, sd):
    rng = np.random.default_rng(n * 1000 + k)
    w = (rng.standard_normal((n, k)) * sd).astype(np.float32)
    w[0, :g] = 0
    p1, s1 = quant.quantize_w4(w, g)
    p2, s2 = R.quantize_w4(w, g)
    assert np.array_equal(p1, p2) and np.array_equal(s1.view(np.uint16), s2.view(np.uint16))
    assert np.array_equal(quant.unpack_w4(p1), R.unpack_w4(p1))
    assert np.array_equal(quant.dequantize_w4(p1, s1, g), R.dequantize_w4(p1, s1, g))
    assert np.array_equal(quant.interleave_for_gpu(p1), R.interleave_for_gpu(p1))
    if k % 128 == 0:
        assert np.array_equal(quant.interleave_for_mma(p1), R.interleave_for_mma(p1))
        assert np.array_equal(quant.interleave_for_mfma(p1), R.interleave_for_mfma(p1))
    x = rng.standard_normal((3, k))
    assert np.allclose(quant.gemv_reference(x, p1, s1, g), R.gemv_reference(x, p1, s1, g), rtol=1e-12, atol=1e-12)


def test_host_quantizer_is_threaded_and_still_exact():
    w = _random_weight(7, 1536, 1024, 0.02)        # above the threading threshold
    p1, s1 = quant.quantize_w4(w, 128)
    p2, s2 = R.quantize_w4(w, 128)
    assert np.array_equal(p1, p2) and np.array_equal(s1.view(np.uint16), s2.view(np.uint16))


def test_golden_fixtures_through_the_product():
    for case in sorted({k[:-5] for k in GOLDEN.files if k.endswith("_meta")}):
        n, k, g, m, seed = (int(v) for v in GOLDEN[f"{case}_meta"])
        packed, scales = quant.quantize_w4(GOLDEN[f"{case}_w"], g)
        assert np.array_equal(packed, GOLDEN[f"{case}_packed"])
        assert np.array_equal(scales.view(np.uint16), GOLDEN[f"{case}_scales"].view(np.uint16))
        if k % 128 == 0:
            assert np.array_equal(quant.interleave_for_mfma(packed), GOLDEN[f"{case}_mfma"])
