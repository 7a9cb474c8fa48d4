"""Build the libraries in-tree (gfx950 only):

    lowbit-kernels_amd/lowbit/liblowbit_w4.so      every kernel and the C ABI (hipcc)
    lowbit-kernels_amd/lowbit/liblowbit_format.so  the host format functions alone (g++; no HIP dependency), which
                                                   lowbit.quant loads, so packing weights needs no GPU stack

    python lowbit-kernels_amd/build.py [--jobs N] [--asm]
    python lowbit-kernels_amd/build.py --sanitize   # CPU ASan + UBSan build of the host code into _build_asan/

Every source is compiled with hipcc for gfx950 (host code for the .cpp files), in parallel, then linked. --asm also
writes the device assembly of each kernel file into lowbit-kernels_amd/_build/ for inspection. --sanitize builds the
host code (the format functions, the C ABI's validation, the launch planners) with AddressSanitizer and
UndefinedBehaviorSanitizer -- the device code is built without them -- into _build_asan/liblowbit_w4.so and
_build_asan/liblowbit_format.so, then runs tests/test_quant.py and tests/test_capi.py against them (no GPU needed).
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
OUT_FORMAT = PKG / "lowbit" / "liblowbit_format.so"
ASAN = PKG / "_build_asan"
SOURCES = ["capi.hip", "gemv.hip", "gemm_mfma.hip", "gemm_prefill.hip", "dequant.hip", "quantize.hip", "decode_ops.hip", "hbm_probe.hip",
           "host_format.cpp", "status.cpp"]
FORMAT_SOURCES = ["host_format.cpp", "status.cpp"]
# host-only sanitizers: on a hipcc line each -fsanitize= goes after -Xarch_host, so the device code is built without
SANITIZE_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-Xarch_host",
                 "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]

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


def compile_one(src, asm=False, outdir=BUILD, extra=()):
    obj = outdir / (src + ".o")
    if src.endswith(".hip"):
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-x", "hip", *COMMON, *DEVICE_FLAGS, *extra, "-c", str(CSRC / src),
               "-o", str(obj)]
    else:
        cmd = [hipcc(), *COMMON, *extra, "-c", str(CSRC / src), "-o", str(obj)]
    rc, err = _run(cmd)
    if rc:
        return src, rc, err
    if asm and src.endswith(".hip"):
        rc2, err2 = _run([hipcc(), f"--offload-arch={ARCH}", "-x", "hip", *COMMON, *DEVICE_FLAGS, "--cuda-device-only", "-S",
                          str(CSRC / src), "-o", str(BUILD / (src + ".s"))])
        if rc2:
            return src, rc2, err2
    return src, 0, err


def build_format(out=OUT_FORMAT, extra=(), compiler="g++"):
    """The host format functions alone, with g++ (hipcc's host compiler for the sanitizer build, so that one ASan
    runtime serves both libraries): no HIP runtime dependency."""
    tmp = out.with_suffix(".so.tmp")
    rc, err = _run([compiler, "-O3", "-std=c++17", "-fPIC", "-shared", "-pthread", "-Wall", f"-I{ROOT / 'include'}",
                    f"-I{CSRC}", *extra, *[str(CSRC / src) for src in FORMAT_SOURCES], "-o", str(tmp)])
    if rc:
        raise RuntimeError(f"g++ failed on the format library:\n{err}")
    os.replace(tmp, out)
    return out


def build(jobs=None, asm=False, verbose=False, outdir=BUILD, out=OUT, extra=()):
    outdir.mkdir(exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(lambda s: compile_one(s, asm, outdir, extra), SOURCES))
    failed = [(s, err) for s, rc, err in results if rc]
    for s, rc, err in results:
        if err.strip() and (verbose or rc):
            print(f"--- {s}\n{err}", file=sys.stderr)
    if failed:
        raise RuntimeError(f"hipcc failed on {[s for s, _ in failed]}")
    tmp = out.with_suffix(".so.tmp")
    rc, err = _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *extra, "-o", str(tmp),
                    *[str(outdir / (s + ".o")) for s in SOURCES]])
    if rc:
        raise RuntimeError(f"link failed:\n{err}")
    os.replace(tmp, out)
    if out == OUT:
        build_format()
        write_build_info()
    return out


BUILD_INFO = PKG / "lowbit" / "build_info.json"


def write_build_info(path=BUILD_INFO):
    """The git commit the library was built from (and whether the tree had uncommitted changes), beside the library,
    for provenance records made where the tree travels without its git history."""
    import json
    def git(*args):
        try:
            p = subprocess.run(["git", "-C", str(ROOT), *args], capture_output=True, text=True, timeout=10)
            return p.stdout.strip() if p.returncode == 0 else None
        except (OSError, subprocess.SubprocessError):
            return None
    status = git("status", "--porcelain", "--untracked-files=no")
    path.write_text(json.dumps({"git_commit": git("rev-parse", "HEAD"),
                                "uncommitted_changes": None if status is None else bool(status)}) + "\n")


def sanitizer_check(jobs=None):
    """Build the host code with ASan + UBSan and run the CPU tests of the format functions and the C ABI on it."""
    ASAN.mkdir(exist_ok=True)
    lib = build(jobs, outdir=ASAN, out=ASAN / "liblowbit_w4.so", extra=SANITIZE_HOST)
    fmt = build_format(ASAN / "liblowbit_format.so", SANITIZE_HOST, compiler=hipcc())
    # python itself is not instrumented: clang's ASan runtime is preloaded
    clang_rt = subprocess.run([hipcc(), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                              text=True).stdout.strip()
    env = dict(os.environ, LOWBIT_LIB=str(lib), LOWBIT_FORMAT_LIB=str(fmt), LD_PRELOAD=clang_rt,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    tests = [str(ROOT / "tests" / "test_quant.py"), str(ROOT / "tests" / "test_capi.py")]
    p = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", *tests], env=env, text=True,
                       capture_output=True)
    print(p.stdout[-3000:], p.stderr[-3000:], sep="\n")
    return p.returncode


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--asm", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--sanitize", action="store_true", help="ASan + UBSan build of the host code, then its CPU tests")
    a = ap.parse_args()
    if a.sanitize:
        sys.exit(sanitizer_check(a.jobs))
    print(build(a.jobs, a.asm, a.verbose))


if __name__ == "__main__":
    main()
