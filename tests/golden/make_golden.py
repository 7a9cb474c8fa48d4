"""Write tests/golden/w4_golden.npz: the reference's known answers plus seeded vectors from the oracle.

    python tests/golden/make_golden.py

Known answers (data taken from the reference's own tests and harness, no code):
  * [7, -7, 1, 0] in a 128-group -> scale 1.0, bytes 0x1F, 0x89 (reference tests/test_quant.py:24-30);
  * the magic number: fp16(0x6400 | u) - 1032 == u - 8 for u = 0..15 (tests/test_quant.py:71-76);
  * overflow: q = 7 (byte 0xFF), scale 2^-10, K = 128 -> 3584 for x = 4096 and -7168 for x = -8192
    (bench/gpu_run.py:144-159).
Seeded vectors (oracle/quant_ref.py, seed recorded per case): W, packed (canonical, v3, the reference's m16n8k8 order,
the gfx950 MFMA layout), scales, fp16 dequant, x and the fp64 GEMV, over odd N, G = 32/64/128/256 and a clip-search case.
"""
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import quant_ref as R  # noqa: E402

CASES = [  # (name, N, K, G, M, seed, weight scale)
    ("g128_small", 16, 256, 128, 3, 11, 0.02),
    ("g128_oddn", 37, 384, 128, 2, 12, 1.0),
    ("g128_n1", 1, 128, 128, 1, 13, 0.02),
    ("g256", 24, 512, 256, 4, 14, 0.02),
    ("g64", 13, 320, 64, 5, 15, 50.0),
    ("g32", 9, 96, 32, 8, 16, 0.02),
    ("g128_n1001_slice", 33, 256, 128, 1, 17, 0.02),
]


def main():
    out = {}
    w = np.zeros((1, 128), np.float32)
    w[0, :4] = [7, -7, 1, 0]
    out["kat_layout_w"] = w
    out["kat_layout_bytes"] = np.array([(7 + 8) | ((-7 + 8) << 4), (1 + 8) | ((0 + 8) << 4)], np.uint8)
    out["kat_layout_scale"] = np.array([1.0], np.float16)
    out["kat_magic_u"] = np.arange(16, dtype=np.uint16)
    out["kat_magic_value"] = np.arange(16, dtype=np.float32) - 8
    out["kat_overflow"] = np.array([[4096.0, 3584.0], [-8192.0, -7168.0]], np.float32)
    for name, n, k, g, m, seed, sd in CASES:
        rng = np.random.default_rng(seed)
        wf = (rng.standard_normal((n, k)) * sd).astype(np.float32)
        wf[0, :g] = 0.0                                          # one all-zero group: scale 1, exact zeros
        packed, scales = R.quantize_w4(wf, g)
        x = rng.standard_normal((m, k)).astype(np.float16)
        out[f"{name}_meta"] = np.array([n, k, g, m, seed], np.int64)
        out[f"{name}_w"] = wf
        out[f"{name}_packed"] = packed
        out[f"{name}_scales"] = scales
        out[f"{name}_v3"] = R.interleave_for_gpu(packed)
        if k % 128 == 0:
            out[f"{name}_nvmma"] = R.interleave_for_mma(packed)
            out[f"{name}_mfma"] = R.interleave_for_mfma(packed)
        out[f"{name}_dequant16"] = R.dequantize_w4_f16(packed, scales, g)
        out[f"{name}_x"] = x
        out[f"{name}_y64"] = R.gemv_reference(x.astype(np.float64), packed, scales, g)
    rng = np.random.default_rng(21)
    wc = (rng.standard_normal((8, 512)) * 0.02).astype(np.float32)
    p, s, idx, _ = R.quantize_w4_clip(wc, 128, R.CLIP_GRID)
    out["clip_w"], out["clip_packed"], out["clip_scales"], out["clip_index"] = wc, p, s, idx
    path = pathlib.Path(__file__).resolve().parent / "w4_golden.npz"
    np.savez_compressed(path, **out)
    print(path, sum(v.nbytes for v in out.values()), "bytes raw")


if __name__ == "__main__":
    main()
