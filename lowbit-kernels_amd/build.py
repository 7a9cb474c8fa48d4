"""Build liblowbit_w4.so (gfx950 only) in-tree: lowbit-kernels_amd/lowbit/liblowbit_w4.so.

    python lowbit-kernels_amd/build.py [--jobs N] [--asm]

Every source is compiled with hipcc for gfx950 (host code for the .cpp file), in parallel, then linked. --asm also
writes the device assembly of each kernel file into lowbit-kernels_amd/_build/ for inspection.
"""
import argparse
import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
OUT = PKG / "lowbit" / "liblowbit_w4.so"
SOURCES = ["capi.hip", "gemv.hip", "gemm_mfma.hip", "gemm_prefill.hip", "dequant.hip", "quantize.hip", "decode_ops.hip", "hbm_probe.hip",
           "host_format.cpp"]
ARCH = "gfx950"
# packed-fp32 ops stay off: only scalar fp32 and packed fp16 arithmetic is emitted
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", f"-I{ROOT / 'include'}", f"-I{CSRC}"]


def hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = pathlib.Path(rocm) / "bin" / "hipcc"
    return str(path) if path.exists() else (shutil.which("hipcc") or "hipcc")


def _run(cmd):
    p = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature name and says so; that warning is expected
    err = "\n".join(l for l in p.stderr.splitlines() if "packed-fp32-ops" not in l)
    return p.returncode, err


def compile_one(src, asm=False):
    obj = BUILD / (src + ".o")
    if src.endswith(".hip"):
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-x", "hip", *COMMON, *DEVICE_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    else:
        cmd = [hipcc(), *COMMON, "-c", str(CSRC / src), "-o", str(obj)]
    rc, err = _run(cmd)
    if rc:
        return src, rc, err
    if asm and src.endswith(".hip"):
        rc2, err2 = _run([hipcc(), f"--offload-arch={ARCH}", "-x", "hip", *COMMON, *DEVICE_FLAGS, "--cuda-device-only", "-S",
                          str(CSRC / src), "-o", str(BUILD / (src + ".s"))])
        if rc2:
            return src, rc2, err2
    return src, 0, err


def build(jobs=None, asm=False, verbose=False):
    BUILD.mkdir(exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(lambda s: compile_one(s, asm), SOURCES))
    failed = [(s, err) for s, rc, err in results if rc]
    for s, rc, err in results:
        if err.strip() and (verbose or rc):
            print(f"--- {s}\n{err}", file=sys.stderr)
    if failed:
        raise RuntimeError(f"hipcc failed on {[s for s, _ in failed]}")
    tmp = OUT.with_suffix(".so.tmp")
    rc, err = _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
                    *[str(BUILD / (s + ".o")) for s in SOURCES]])
    if rc:
        raise RuntimeError(f"link failed:\n{err}")
    os.replace(tmp, OUT)
    return OUT


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--asm", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.asm, a.verbose))


if __name__ == "__main__":
    main()
