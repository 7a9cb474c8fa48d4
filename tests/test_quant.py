"""The product's host-side format module (lowbit.quant, native host code) -- the reference's golden-model tests
(reference tests/test_quant.py:1-118) run against it unchanged in substance, plus bit-for-bit agreement with the
oracle on random inputs and the committed fixtures."""
import pathlib

import numpy as np
import pytest

from lowbit import quant
from lowbit.quant import dequantize_w4, gemv_reference, interleave_for_gpu, quantize_w4, unpack_w4
from oracle import quant_ref as R

RNG = np.random.default_rng(0)
GOLDEN = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "w4_golden.npz")


def words_of(packed):
    """uint8 [N, K//2] -> little-endian uint32 words [N, K//8], as a GPU reads them."""
    return np.ascontiguousarray(packed).view("<u4")


def test_error_is_at_most_half_a_step():
    w = RNG.standard_normal((64, 512)).astype(np.float32)
    packed, scales = quantize_w4(w, 128)
    err = np.abs(dequantize_w4(packed, scales, 128) - w).reshape(64, 4, 128)
    step = scales.astype(np.float32)[..., None]
    assert np.all(err <= step / 2 + 1e-6)


def test_layout_two_nibbles_per_byte_low_first():
    w = np.zeros((1, 128), np.float32)
    w[0, :4] = [7, -7, 1, 0]
    packed, scales = quantize_w4(w, 128)
    assert scales[0, 0] == 1.0
    assert packed[0, 0] == (7 + 8) | ((-7 + 8) << 4)
    assert packed[0, 1] == (1 + 8) | ((0 + 8) << 4)


def test_values_stay_in_range_and_zero_group_is_exact():
    w = RNG.standard_normal((8, 256)).astype(np.float32) * 50
    w[3] = 0
    packed, scales = quantize_w4(w, 128)
    q = unpack_w4(packed)
    assert q.min() >= -8 and q.max() <= 7
    assert np.all(dequantize_w4(packed, scales, 128)[3] == 0)


def test_rejects_bad_shapes():
    with pytest.raises(ValueError):
        quantize_w4(np.zeros((4, 100), np.float32), 128)
    with pytest.raises(ValueError):
        quantize_w4(np.zeros((4, 96), np.float32), 48)


def test_canonical_decoder_matches_v2_bit_logic():
    w = RNG.standard_normal((5, 256)).astype(np.float32)
    packed, _ = quantize_w4(w, 128)
    u = unpack_w4(packed) + 8
    words = words_of(packed)
    for b in range(8):
        assert np.array_equal((words >> (4 * b)) & 0xF, u[:, b::8])


def test_interleaved_decoder_matches_v3_bit_logic():
    w = RNG.standard_normal((5, 256)).astype(np.float32)
    packed, _ = quantize_w4(w, 128)
    u = unpack_w4(packed) + 8
    words = words_of(interleave_for_gpu(packed)).astype(np.uint64)
    for j in range(4):
        t = (words >> (4 * j)) & 0x000F000F
        assert np.array_equal(t & 0xFFFF, u[:, 2 * j::8])
        assert np.array_equal(t >> 16, u[:, 2 * j + 1::8])


def test_magic_number_trick_is_exact_in_fp16():
    u = np.arange(16, dtype=np.uint16)
    h = (u | 0x6400).view(np.float16)
    assert np.array_equal(h.astype(np.float32) - 1032.0, u.astype(np.float32) - 8)
    assert np.array_equal(h - np.float16(1032), (u.astype(np.int16) - 8).astype(np.float16))
    # the high-nibble form the kernels also use: (1024 + 16 u) / 16 - 72 == u - 8, exactly
    h16 = ((u << 4) | 0x6400).view(np.float16)
    assert np.array_equal(h16.astype(np.float32) / 16 - 72, u.astype(np.float32) - 8)


def test_interleave_keeps_the_byte_count_and_is_a_permutation():
    w = RNG.standard_normal((3, 128)).astype(np.float32)
    packed, _ = quantize_w4(w, 128)
    inter = interleave_for_gpu(packed)
    assert inter.shape == packed.shape
    assert sorted(unpack_w4(inter)[1]) == sorted(unpack_w4(packed)[1])


def test_reference_gemv():
    w = RNG.standard_normal((16, 256)).astype(np.float32)
    x = RNG.standard_normal((3, 256)).astype(np.float32)
    packed, scales = quantize_w4(w, 128)
    y = gemv_reference(x, packed, scales, 128)
    assert y.shape == (3, 16)
    assert np.allclose(y, x @ dequantize_w4(packed, scales, 128).T, rtol=1e-5, atol=1e-4)


def test_mma_layout_feeds_each_lane_its_fragment():
    rng = np.random.default_rng(5)
    packed, _ = quant.quantize_w4(rng.standard_normal((3, 384)).astype(np.float32))
    u = quant.unpack_w4(packed) + quant.OFFSET
    mma = quant.interleave_for_mma(packed)
    words = mma.reshape(3, -1, 4, 4, 4).view("<u4")[..., 0]
    for c in range(384 // 128):
        for t in range(4):
            for s in range(16):
                w, j = int(words[1, c, t, s >> 2]), s & 3
                k = 128 * c + 8 * s + 2 * t
                assert (w >> (4 * j)) & 0xF == u[1, k] and (w >> (4 * j + 16)) & 0xF == u[1, k + 1]


def test_mma_layout_is_a_permutation_and_rejects_bad_k():
    rng = np.random.default_rng(6)
    packed, _ = quant.quantize_w4(rng.standard_normal((2, 256)).astype(np.float32))
    a = quant.unpack_w4(packed)
    b = quant.unpack_w4(quant.interleave_for_mma(packed))
    assert sorted(a[0].tolist()) == sorted(b[0].tolist())
    with pytest.raises(ValueError):
        quant.interleave_for_mma(np.zeros((1, 32), np.uint8))
    with pytest.raises(ValueError):
        quant.interleave_for_mfma(np.zeros((1, 32), np.uint8))


# ---- bit-for-bit agreement with the oracle ----

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
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((1536, 1024)) * 0.02).astype(np.float32)        # above the threading threshold
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
