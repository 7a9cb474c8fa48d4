"""The C ABI on the CPU: the library loads, exports every function include/lowbit_w4.h declares, and refuses bad
arguments with the reference's messages before it touches any GPU (no kernel runs here)."""
import ctypes
import pathlib
import re

import pytest

from lowbit import _native

HEADER = pathlib.Path(__file__).resolve().parent.parent / "include" / "lowbit_w4.h"
FAKE = ctypes.c_void_p(4096)          # a 16-byte aligned, non-null address that validation never dereferences


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(lowbit_\w+)\s*\(", text)))


def test_header_declares_what_the_binding_binds():
    assert declared() == sorted(_native.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.lowbit_version().decode().endswith("gfx950")


def _msg(rc):
    assert rc != 0
    return _native.lib().lowbit_last_error().decode()


@pytest.mark.parametrize("call,code,text", [
    (lambda l: l.lowbit_w4_gemv(None, FAKE, FAKE, FAKE, 1, 16, 128, 128, 6, 0, None), 1, "null pointer"),
    (lambda l: l.lowbit_w4_gemv(FAKE, FAKE, FAKE, FAKE, 1, 16, 128, 0, 6, 0, None), 2, "group size must be positive"),
    (lambda l: l.lowbit_w4_gemv(FAKE, FAKE, FAKE, FAKE, 1, 16, 100, 32, 6, 0, None), 2, "multiple of the group size"),
    (lambda l: l.lowbit_w4_gemv(FAKE, FAKE, FAKE, FAKE, 9, 16, 128, 128, 6, 0, None), 5, "1..8 rows"),
    (lambda l: l.lowbit_w4_gemv(FAKE, FAKE, FAKE, FAKE, 1, 16, 128, 128, 5, 0, None), 6, "version is 1..4 or 6"),
    (lambda l: l.lowbit_w4_gemv(FAKE, FAKE, FAKE, FAKE, 1, 16, 96, 32, 6, 0, None), 7, "multiples of 128"),
    (lambda l: l.lowbit_w4_gemv(FAKE, FAKE, FAKE, FAKE, 1, 16, 128, 128, 6, 3, None), 8, "rows_per_warp"),
    (lambda l: l.lowbit_w4_gemv(ctypes.c_void_p(4098), FAKE, FAKE, FAKE, 1, 16, 128, 128, 6, 0, None), 4, "16-byte"),
    (lambda l: l.lowbit_w4_gemm_mfma(FAKE, FAKE, FAKE, FAKE, 65, 16, 128, 128, 0, None, 0, None), 5, "1..64 rows"),
    (lambda l: l.lowbit_w4_gemm_mfma(FAKE, FAKE, FAKE, FAKE, 4, 16, 128, 128, 3, None, 0, None), 8, "row_tiles"),
    (lambda l: l.lowbit_w4_gemm_mfma(FAKE, FAKE, FAKE, FAKE, 4, 16, 192, 64, 0, None, 0, None), 7, "multiples of 128"),
    (lambda l: l.lowbit_w4_gemm_mfma(FAKE, FAKE, FAKE, FAKE, 4, 16, 128, 128, 0, ctypes.c_void_p(4104), 1 << 20, None),
     1, "workspace"),
    (lambda l: l.lowbit_w4_gemm_mfma(FAKE, FAKE, FAKE, FAKE, 4, 16, 128, 128, 0, FAKE, 4096, None), 1, "workspace"),
    (lambda l: l.lowbit_w4_gemm_mfma(FAKE, FAKE, FAKE, FAKE, 4, 16, 1 << 23, 128, 0, None, 0, None), 3, "K is at most"),
    (lambda l: l.lowbit_w4_gemm_mfma_noalloc(FAKE, FAKE, FAKE, FAKE, 65, 16, 128, 128, 0, None), 5, "1..64 rows"),
    (lambda l: l.lowbit_w4_gemm_mfma_noalloc(FAKE, FAKE, FAKE, FAKE, 4, 16, 128, 128, 3, None), 8, "row_tiles"),
    (lambda l: l.lowbit_w4_gemm_mfma_noalloc(None, FAKE, FAKE, FAKE, 4, 16, 128, 128, 0, None), 1, "null pointer"),
    (lambda l: l.lowbit_w4_gemm_mfma_noalloc(FAKE, FAKE, FAKE, FAKE, 4, 16, 192, 64, 0, None), 7, "multiples of 128"),
    # the v6 GEMV stages 16 x K / G scales per tile in 64 KiB of LDS: 2 tiles per wave halve the K / G it takes
    (lambda l: l.lowbit_w4_gemv(FAKE, FAKE, FAKE, FAKE, 1, 16, 1536 * 128, 128, 6, 2, None), 2, "at most 1024"),
    (lambda l: l.lowbit_w4_gemv(FAKE, FAKE, FAKE, FAKE, 1, 16, 600 * 128, 128, 6, 4, None), 2, "at most 512"),
    (lambda l: l.lowbit_w4_gemv(FAKE, FAKE, FAKE, FAKE, 1, 16, 2049 * 128, 128, 6, 0, None), 2, "at most 2048"),
    (lambda l: l.lowbit_w4_dequant(FAKE, FAKE, FAKE, 16, 128, -1, 0, None), 2, "positive group size"),
    (lambda l: l.lowbit_w4_dequant(FAKE, FAKE, FAKE, 16, 96, 32, 1, None), 7, "group % 128"),
    (lambda l: l.lowbit_w4_quantize(FAKE, 0, FAKE, FAKE, 16, 128, 2048, None, 0, None), 2, "multiple of the group"),
    (lambda l: l.lowbit_w4_quantize(FAKE, 7, FAKE, FAKE, 16, 128, 128, None, 0, None), 1, "dtype"),
    (lambda l: l.lowbit_w4_relayout(FAKE, FAKE, 16, 128, 2, None), 1, "alias"),
    (lambda l: l.lowbit_w4_relayout(FAKE, ctypes.c_void_p(8192), 16, 96, 2, None), 7, "multiple of 128"),
    (lambda l: l.lowbit_set_launch_override(3, 0, 0), 8, "waves_per_group"),
    (lambda l: l.lowbit_set_launch_override(4, 5, 0), 8, "ring"),
    (lambda l: l.lowbit_set_launch_override(4, 4, 33), 8, "k_splits"),
    (lambda l: l.lowbit_set_gemm_kernel(3), 8, "kernel is 0"),
    (lambda l: l.lowbit_set_gemm_kernel(-1), 8, "kernel is 0"),
    (lambda l: l.lowbit_set_gemm_tile_waves(2), 8, "tile_waves is 0"),
    (lambda l: l.lowbit_set_gemm_tile_waves(7), 8, "tile_waves is 0"),
    (lambda l: l.lowbit_w4_qkv_rope_rows(FAKE, FAKE, FAKE, 0, 512, 128, 128, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 1,
                                         64, None, ctypes.c_float(0), None, 0, None), 5, "at least one row"),
    (lambda l: l.lowbit_w4_qkv_rope_rows(FAKE, FAKE, FAKE, 4, 640, 128, 128, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 1,
                                         64, None, ctypes.c_float(0), None, 0, None), 3, "(Hq + 2 Hkv) * 128"),
    (lambda l: l.lowbit_w4_qkv_rope_rows(FAKE, FAKE, FAKE, 4, 512, 128, 128, None, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 1,
                                         64, None, ctypes.c_float(0), None, 0, None), 1, "null pointer"),
    (lambda l: l.lowbit_w4_qkv_rope_rows(FAKE, FAKE, FAKE, 100, 512, 1 << 23, 128, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                         2, 1, 64, None, ctypes.c_float(0), None, 0, None), 3, "K is at most"),
    (lambda l: l.lowbit_w4_qkv_rope_rows(FAKE, FAKE, FAKE, 4, 512, 128, 128, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 1,
                                         64, None, ctypes.c_float(0), FAKE, 4096, None), 1, "workspace"),
    (lambda l: l.lowbit_w4_qkv_rope_rows(FAKE, FAKE, FAKE, 4, 512, 128, 128, FAKE, FAKE, ctypes.c_void_p(4104), FAKE,
                                         FAKE, FAKE, 2, 1, 64, None, ctypes.c_float(0), None, 0, None), 4, "16-byte aligned rope table"),
    (lambda l: l.lowbit_w4_qkv_rope_rows(FAKE, FAKE, FAKE, 4, 512, 128, 128, FAKE, FAKE, FAKE, FAKE,
                                         ctypes.c_void_p(4098), FAKE, 2, 1, 64, None, ctypes.c_float(0), None, 0, None), 4, "8-byte aligned"),
    (lambda l: l.lowbit_w4_qkv_rope_rows(FAKE, FAKE, FAKE, 100, 512, 128, 128, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 1,
                                         64, FAKE, ctypes.c_float(1e-6), None, 0, None), 1, "at most 64 rows"),
    (lambda l: l.lowbit_rope_table(FAKE, None, FAKE, 4, None), 1, "null pointer"),
    (lambda l: l.lowbit_rope_table(FAKE, FAKE, FAKE, 0, None), 3, "M must be positive"),
    (lambda l: l.lowbit_rope_table(FAKE, FAKE, ctypes.c_void_p(4098), 4, None), 4, "4-byte aligned"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 100, 64, None, 1 << 20,
                                      FAKE, None, None, 0, None, None, None, None), 1, "null pointer"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 100, 64, FAKE, 1 << 20,
                                      None, None, None, 0, None, None, None, None), 1, "null pointer"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 100, 60, FAKE, 1 << 20,
                                      FAKE, None, None, 0, None, None, None, None), 3, "K % 8"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 100, 65536, FAKE, 1 << 20,
                                      FAKE, None, None, 0, None, None, None, None), 3, "K % 8"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 0, 64, FAKE, 1 << 20,
                                      FAKE, None, None, 0, None, None, None, None), 3, "K % 8"),
    (lambda l: l.lowbit_f16_gemv_pick(ctypes.c_void_p(4104), FAKE, FAKE, 100, 64, FAKE, 1 << 20,
                                      FAKE, None, None, 0, None, None, None, None), 4,
     "16-byte aligned"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 100, 64, ctypes.c_void_p(4100), 1 << 20,
                                      FAKE, None, None, 0, None, None, None, None), 4,
     "8-byte aligned"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 100, 64, FAKE, 1 << 20,
                                      FAKE, ctypes.c_void_p(4100), None, 0, None, None, None, None), 4,
     "8-byte aligned"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 151936, 64, FAKE, 1000,
                                      FAKE, None, None, 0, None, None, None, None), 1, "workspace"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 100, 64, FAKE, 1 << 20, FAKE, None, FAKE, 4, None, None, None,
                                      None), 1, "out_tokens goes with out_count"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 100, 64, FAKE, 1 << 20, FAKE, None, None, 0, None, FAKE, None,
                                      None), 1, "embed with h_out"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 100, 64, FAKE, 1 << 20, FAKE, None, FAKE, -1, FAKE, None, None,
                                      None), 3, "out_capacity"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 100, 64, FAKE, 1 << 20, FAKE, None, None, 0, None,
                                      ctypes.c_void_p(4104), FAKE, None), 4, "embed and h_out must be 16-byte"),
    (lambda l: l.lowbit_f16_gemv_pick(FAKE, FAKE, FAKE, 100, 64, FAKE, 1 << 20, FAKE, None, FAKE, 4,
                                      ctypes.c_void_p(4098), None, None, None), 4, "naturally aligned"),
    (lambda l: l.lowbit_attention(FAKE, FAKE, FAKE, FAKE, FAKE, 1, 2, 1, 64, 64, ctypes.c_float(1.0), FAKE, 1024,
                                  None), 1, "at least 4096 bytes"),
    (lambda l: l.lowbit_f16_gemv(FAKE, FAKE, FAKE, 65, 16, 128, None), 5, "1..64 rows"),
    (lambda l: l.lowbit_f16_gemv(FAKE, FAKE, FAKE, 17, 16, 136, None), 3, "K % 128"),
    (lambda l: l.lowbit_f16_gemv(FAKE, FAKE, FAKE, 1, 16, 12, None), 3, "K % 8"),
    (lambda l: l.lowbit_f16_gemv(FAKE, FAKE, FAKE, 4, 16, 16392, None), 3, "K % 128"),
    (lambda l: l.lowbit_f16_gemv(ctypes.c_void_p(4100), FAKE, FAKE, 1, 16, 128, None), 4, "16-byte"),
    (lambda l: l.lowbit_hbm_read(None, 1024, FAKE, 256, None), 1, "null pointer"),
    (lambda l: l.lowbit_hbm_read(FAKE, 1000, FAKE, 256, None), 3, "multiple of 16"),
    (lambda l: l.lowbit_hbm_read(FAKE, 1024, FAKE, 0, None), 3, "blocks"),
    (lambda l: l.lowbit_hbm_read(ctypes.c_void_p(4100), 1024, FAKE, 256, None), 4, "16-byte"),
    (lambda l: l.lowbit_hbm_copy(FAKE, FAKE, 0, 256, None), 3, "multiple of 16"),
    (lambda l: l.lowbit_hbm_copy(FAKE, FAKE, 1024, 70000, None), 3, "blocks"),
])
def test_validation_refuses_before_any_gpu_call(call, code, text):
    rc = call(_native.lib())
    assert rc == code
    assert text in _msg(rc)


def test_strerror_names_every_code():
    lib = _native.lib()
    names = {lib.lowbit_strerror(c).decode() for c in range(11)}
    assert len(names) == 11 and "unknown status" not in names


def test_check_raises_runtime_error_with_the_message():
    lib = _native.lib()
    lib.lowbit_w4_gemv(FAKE, FAKE, FAKE, FAKE, 9, 16, 128, 128, 6, 0, None)
    with pytest.raises(RuntimeError, match="1..8 rows"):
        _native.check(5)


def test_format_library_needs_no_gpu_stack():
    """liblowbit_format.so (the host format functions, built with g++) exports them with the same error reporting and
    links no HIP library, so lowbit.quant packs weights on a machine without ROCm."""
    import shutil
    import subprocess
    host = _native.host_lib()
    for name in _native.HOST_FUNCTIONS:
        assert hasattr(host, name), name
    assert host.lowbit_host_unpack(None, None, 1, 32) == 1 and b"null" in host.lowbit_last_error()
    if shutil.which("readelf"):
        needed = subprocess.run(["readelf", "-d", str(_native.FORMAT_LIB_PATH)], capture_output=True, text=True).stdout
        assert "NEEDED" in needed and "amdhip" not in needed and "hsa" not in needed


def test_quant_runs_without_the_kernel_library(tmp_path):
    """With the kernel library unreachable (LOWBIT_LIB points nowhere), lowbit.quant still quantizes and relayouts."""
    import os
    import subprocess
    import sys
    code = ("import numpy as np; from lowbit import quant; "
            "p, s = quant.quantize_w4(np.ones((2, 128), np.float32)); "
            "assert p[0, 0] == 0xFF and float(s[0, 0]) == np.float16(1 / 7); "
            "assert quant.interleave_for_mfma(p).shape == (2, 64); print('ok')")
    root = pathlib.Path(__file__).resolve().parent.parent
    env = dict(os.environ, LOWBIT_LIB=str(tmp_path / "missing.so"),
               PYTHONPATH=os.pathsep.join([str(root / "lowbit-kernels_amd"), str(root)]))
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stderr[-2000:]


def test_build_info_names_the_commit_the_library_was_built_from(tmp_path):
    """build.py records the git commit (and whether the tree had uncommitted changes) beside the library, for the
    bench's provenance on machines where the tree travels without its history."""
    import json
    import subprocess
    import sys
    pkg = pathlib.Path(__file__).resolve().parent.parent / "lowbit-kernels_amd"
    sys.path.insert(0, str(pkg))
    try:
        import build as lowbit_build
    finally:
        sys.path.remove(str(pkg))
    out = tmp_path / "build_info.json"
    lowbit_build.write_build_info(out)
    info = json.loads(out.read_text())
    assert set(info) == {"git_commit", "uncommitted_changes"}
    head = subprocess.run(["git", "-C", str(pkg.parent), "rev-parse", "HEAD"], capture_output=True, text=True)
    if head.returncode == 0:
        assert info["git_commit"] == head.stdout.strip()
        assert isinstance(info["uncommitted_changes"], bool)
    else:                                                   # a copy of the tree without its git history
        assert info["git_commit"] is None
