"""W4A16 benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]        # the contract line
    python bench.py --sweep skinny [--out FILE]                # M = 1..64, three ways
    python bench.py --sweep prefill [--out FILE]               # M = 128..2048: dequant + BLAS vs the int4 GEMM
    python bench.py --no-cpu --steps 50                        # shorter run (profiling)

Workload (the M=1 GEMV sweep over the Qwen2.5-1.5B and 3B decoder projections): one step is an
M=1 ops.linear (the deployed path: the v6 GEMV on the device layout) over every projection of one 1.5B decoder layer
and one 3B decoder layer -- q, k, v, o, gate, up, down at (K, N) = (1536|2048, ...) -- i.e. 14 launches. Weights are
random N(0, 0.02), int4 g128 with the per-group clip search (GPU quantizer), x ~ N(0, 1) fp16. Step i reads layer copy
i mod C, with C distinct copies sized so the rotation covers >= 1 GiB, so no weight is served from the 256 MB
Infinity Cache. The K timed steps run as one hipGraph replay (torch.cuda.CUDAGraph) between two synchronizations.

value = algorithmic bytes moved per step (int4 weights + fp16 scales + x + y, reference bench/gpu_run.py:255,267)
x K / elapsed, in GB/s: whole-job throughput including the per-kernel launch gap of the graph.
roofline = the GEMV kernel: the timed graph holds only its launches, so its average launch duration is elapsed /
(14 K) and achieved = the same bytes / that time; peak = 8 TB/s (MI355X HBM3E). per_shape: each distinct (K, N) alone,
per call in a graph over >= 1 GiB of copies.
measured_peak = HBM read and copy bandwidth over a 2 GiB buffer, by the reference's torch method and by the library's
streaming probes; per_shape also gives each layer's share of the measured read peak.
cpu_baseline = the reference's CPU torch path (its torch dequantize, lowbit/ops.py:119-123, restated in the oracle,
then torch.nn.functional.linear; torch's CPU kernels on all their threads) on a bounded sample of the same steps, plus
the per-call breakdown at BASELINE configs[0] (quantize, dequantize + linear, linear alone; all threads and one).
skinny = the M = 2..64 half of the metric: us per call of the MFMA kernel (v5), dequantize + hipBLASLt and fp16
hipBLASLt at M = 2, 16, 32, 64 on the 3B gate/up and 7B down shapes, with bandwidth and MFMA utilisation.
provenance = GPU, software versions, source and library hashes and the dispatch constants of the run.
"""
import hashlib
import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for p in (ROOT / "lowbit-kernels_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GROUP = 128
CLIP_GRID = tuple(round(1.0 - 0.025 * i, 3) for i in range(11))       # reference bench/e2e.py:30
HBM_PEAK_GBPS = 8000.0
# HBM bytes per GEMV launch of this workload, measured: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE over
# `bench.py --pmc-workload` (20 eager steps), each scaled by what the counter reads for a 1 GiB elementwise copy in the
# same run (FETCH x2.0, WRITE x1.0); 1.034x the algorithmic bytes. Re-measure when the kernel changes.
TRAFFIC_PER_LAUNCH = 4730115
MODELS = {"1.5b": (1536, 8960), "3b": (2048, 11008)}                   # hidden, intermediate; 2 KV heads x 128


def step_projections():
    out = []
    for name, (h, inter) in MODELS.items():
        kv = 2 * 128
        out += [(f"{name}.q", h, h), (f"{name}.k", h, kv), (f"{name}.v", h, kv), (f"{name}.o", h, h),
                (f"{name}.gate", h, inter), (f"{name}.up", h, inter), (f"{name}.down", inter, h)]
    return out


def w4_bytes(k, n):
    return n * k // 2 + n * (k // GROUP) * 2


def alg_bytes(k, n, m=1):
    return w4_bytes(k, n) + 2 * (m * k + m * n)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-fp16", action="store_true", help="skip the fp16 BLAS step")
    ap.add_argument("--no-detail", action="store_true",
                    help="skip the measured peak, the per-shape timings and the skinny block (the timed graph only)")
    ap.add_argument("--pmc-skinny", action="store_true",
                    help="counter workload for the skinny path: a 1 GiB copy (calibration), then eager v5 calls at "
                         "M = 16, 32, 64 on the 3B and 7B MLP shapes over cold copies")
    ap.add_argument("--per-shape-only", action="store_true",
                    help="profiler workload: only the per-shape graphs (the 8 BASELINE decode shapes and 7B gate/up "
                         "and down), nothing else")
    ap.add_argument("--replays", type=int, default=5,
                    help="timed replays of the K-step graph: the first is the contract's timed region, all of them "
                         "give the spread")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="counter workload: a 1 GiB elementwise copy (calibration), then eager steps, nothing else")
    ap.add_argument("--sweep", choices=["skinny", "prefill", "gemv", "ldsring", "order", "tiles", "tilewaves", "splits"],
                    default=None,
                    help="skinny: M=1..64 per path; prefill: M>64; gemv: the M=1 GEMV's tile split x waves; "
                         "ldsring: the M=1 GEMV's weight ring in registers vs in LDS; "
                         "tiles: the MFMA GEMM's row groups vs one tile per workgroup, M=2..32; "
                         "tilewaves: the row groups' tile-waves and K-groups on layers of 560 to 2368 tiles; "
                         "splits: the row groups' K split x K-groups on the decode projections, M=16..64")
    ap.add_argument("--e2e", choices=["tiny", "1.5b", "3b"], default=None,
                    help="hipGraph batch-1 decode of a random-init Qwen2.5 model: fp16 vs fake-quant vs W4Linear")
    ap.add_argument("--decode-trace", choices=["hf_fp16", "hf_int4", "fused_fp16", "fused_int4"], default=None,
                    help="with --e2e MODEL: build only that variant, prefill, capture one step and replay --steps greedy "
                         "tokens (a profiler workload; prints nothing else)")
    ap.add_argument("--chunk", type=int, default=1,
                    help="with --decode-trace: tokens fed per captured step (1 = greedy decoding)")
    ap.add_argument("--no-decode", action="store_true", help="skip the configs[4] decode block")
    ap.add_argument("--host-cost", action="store_true",
                    help="per-call host cost of the M=1 entry points and eager vs graph decode (3B)")
    ap.add_argument("--no-trace", action="store_true",
                    help="skip the traced run of the timed workload (roofline from graph time per launch instead)")
    ap.add_argument("--trace-child", action="store_true",
                    help="(internal) the timed workload alone, run by the parent under rocprofv3 --kernel-trace")
    ap.add_argument("--out", default=None)
    return ap.parse_args()


def build_pool(torch, ops, projs, gib=1.0, fp16=False, seed=0):
    """C layer copies (list of dicts name -> W4Weight, and optionally name -> fp16 weight), C covering >= gib GiB."""
    per_copy = sum(w4_bytes(k, n) for _, k, n in projs)
    copies = int(-(-gib * 2 ** 30 // per_copy)) + 1
    gen = torch.Generator(device="cuda").manual_seed(seed)
    pool, pool16, host = [], [], []
    for c in range(copies):
        layer, layer16, layer_host = {}, {}, {}
        for name, k, n in projs:
            w = torch.randn(n, k, generator=gen, device="cuda") * 0.02
            packed, scales = ops.quantize_w4_gpu(w, GROUP, CLIP_GRID)
            layer[name] = ops.W4Weight(packed, scales, GROUP, ("mma",), device=packed.device)
            if fp16:
                layer16[name] = ops.dequantize_w4_gpu(packed, scales, GROUP)
            if c < 2:                       # canonical host copies for the CPU baseline
                layer_host[name] = (packed.cpu().numpy(), scales.cpu().numpy())
            del w, packed
        pool.append(layer)
        pool16.append(layer16)
        if layer_host:
            host.append(layer_host)
    torch.cuda.synchronize()
    return pool, pool16, host, copies


def cpu_baseline(projs, host, xs, budget_s=15.0):
    """The reference's CPU torch path on the host: its torch dequantize ((u - 8) * scale in fp32, rounded once to fp16,
    reference lowbit/ops.py:119-123, restated as oracle.dequantize_w4_torch) then torch.nn.functional.linear, on all of
    torch's threads -- timed over whole steps of the contract workload until budget_s."""
    import torch
    from oracle import quant_ref as R
    xh = {name: x.cpu() for name, x in xs.items()}
    threads = torch.get_num_threads()
    steps, t0 = 0, time.perf_counter()
    while True:
        layer = host[steps % len(host)]
        for name, k, n in projs:
            packed, scales = layer[name]
            R.cpu_torch_linear(xh[name], packed, scales, GROUP)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    step_bytes = sum(alg_bytes(k, n) for _, k, n in projs)
    return {"value": round(step_bytes * steps / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{steps} steps of the same 14-projection M=1 sweep ({step_bytes / 1e6:.1f} MB each): the "
                      f"reference's torch dequantize to fp16 + torch.nn.functional.linear on {threads} host threads "
                      f"(torch CPU kernels), {el:.1f} s",
            "ms_per_step": round(1000 * el / steps, 3), "config1": cpu_breakdown()}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_breakdown(k=896, n=4864, rounds=25):
    """BASELINE configs[0] on the host: M=1, K=896, N=4864, weights N(0, 0.02), x N(0, 1) fp16, absmax g128. Per call
    (milliseconds, min and median of `rounds` after 3 warm-up calls each) of (i) the reference's torch dequantize to
    fp16 + torch linear, (ii) the dequantize alone, (iii) torch linear on the pre-dequantized fp16 weight, (iv)
    quantize (one-off; the reference's numpy quantizer, single-threaded either way), with torch on all its threads
    and on one. The thread count is set before the warm-up, and the cells are timed round-robin (one call of each
    per round), so a slow stretch of the host hits every cell alike. (i) does (ii)'s work and more, so its min must
    not be below (ii)'s: a run where it is is timed again (once), and `ordering_ok` reports the check. The fp64
    error of the result is reported beside."""
    import numpy as np
    import torch
    from oracle import quant_ref as R
    rng = np.random.default_rng(k * 7 + n)                  # the reference's seed rule, bench/gpu_run.py:206
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal((1, k)).astype(np.float16))
    packed, scales = R.quantize_w4(w, GROUP)
    w16 = torch.from_numpy(R.dequantize_w4_f16(packed, scales, GROUP))
    cells = {"dequant_linear_ms": lambda: R.cpu_torch_linear(x, packed, scales, GROUP),
             "dequant_only_ms": lambda: R.dequantize_w4_torch(packed, scales, GROUP),
             "linear_only_ms": lambda: torch.nn.functional.linear(x, w16),
             "quantize_ms": lambda: R.quantize_w4(w, GROUP)}

    def timed():
        for fn in cells.values():
            for _ in range(3):
                fn()
        ts = {name: [] for name in cells}
        for _ in range(rounds):
            for name, fn in cells.items():
                t0 = time.perf_counter()
                fn()
                ts[name].append(time.perf_counter() - t0)
        return {name: {"min": round(min(v) * 1e3, 4), "median": round(sorted(v)[len(v) // 2] * 1e3, 4)}
                for name, v in ts.items()}

    full = torch.get_num_threads()
    out = {"shape": {"M": 1, "K": k, "N": n, "group": GROUP}, "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(),
           "torch_threads": full, "unit": f"ms per call, min and median of {rounds} round-robin rounds"}
    ok = True
    for threads in (full, 1):
        torch.set_num_threads(threads)
        cell = timed()
        if cell["dequant_linear_ms"]["min"] < cell["dequant_only_ms"]["min"]:
            cell = timed()
        ok &= cell["dequant_linear_ms"]["min"] >= cell["dequant_only_ms"]["min"]
        out[f"threads_{threads}"] = cell
    torch.set_num_threads(full)
    out["ordering_ok"] = bool(ok)
    y = torch.nn.functional.linear(x, w16).numpy()
    out["rel_err_vs_fp64"] = R.rel_err(y, R.gemv_reference(x.double().numpy(), packed, scales, GROUP))
    return out


def measured_peak(torch, ops, gib=2):
    """HBM bandwidth over a `gib` GiB buffer, two ways. The reference's method (bench/gpu_run.py:133-141, there over
    256 MiB): torch's device copy (read + write every byte) and torch's sum (read). And this library's streaming
    probes (lowbit_hbm_read / lowbit_hbm_copy), swept over grid sizes. Each figure is the best of 3 timed rounds of
    5 calls after one warm-up; read_gbps = the best read figure of either method is the roofline's measured peak."""
    e = ops.ext()
    n = gib * 2 ** 30 // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    nbytes = n * 4

    def best_gbps(fn, moved):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        best = 1e30
        for _ in range(3):
            e0.record()
            for _ in range(5):
                fn()
            e1.record()
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1) / 5)
        return round(moved / (best * 1e-3) / 1e9, 1)

    out = {"bytes": nbytes,
           "torch_copy_gbps": best_gbps(lambda: dst.copy_(src), 2 * nbytes),
           "torch_sum_gbps": best_gbps(lambda: src.sum(), nbytes)}
    reads, copies = {}, {}
    for blocks in (512, 1024, 2048, 4096, 8192):
        reads[blocks] = best_gbps(lambda: e.hbm_read(src, sink, blocks), nbytes)
        copies[blocks] = best_gbps(lambda: e.hbm_copy(src, dst, blocks), 2 * nbytes)
    out["probe_read_gbps"], out["probe_copy_gbps"] = reads, copies
    out["read_gbps"] = max(max(reads.values()), out["torch_sum_gbps"])
    out["copy_gbps"] = max(max(copies.values()), out["torch_copy_gbps"])
    del src, dst
    torch.cuda.empty_cache()
    return out


def graph_time_us(torch, fn, iters, reps=3):
    """Per-call time of fn(i) for i < iters captured as one hipGraph (best of reps replays after one untimed)."""
    fn(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = 1e30
    for _ in range(reps):
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1000 / iters)
    del g
    return best


def shape_detail(torch, ops, projs, pool, xs, peak=None):
    """Per distinct (K, N): M=1 ops.linear per call in a hipGraph over >= 1 GiB of copies of that layer; its share of
    8 TB/s and of the measured read peak `peak` (GB/s)."""
    out = {}
    seen = set()
    for name, k, n in projs:
        if (k, n) in seen:
            continue
        seen.add((k, n))
        wq0 = pool[0][name]
        copies = int(-(-2 ** 30 // w4_bytes(k, n)))
        cl = []
        for _ in range(copies):
            c = ops.W4Weight.__new__(ops.W4Weight)
            c.__dict__.update(wq0.__dict__)
            c.packed_mma = wq0.packed_mma.clone()
            c.scales = wq0.scales.clone()
            cl.append(c)
        x = xs[name]
        us = graph_time_us(torch, lambda i: ops.linear(x, cl[i % copies]), max(400, copies))
        out[f"{k}x{n}"] = {"us_per_call": round(us, 2), "GBps": round(alg_bytes(k, n) / (us * 1e-6) / 1e9, 1),
                           "pct_of_8TBps": round(100 * alg_bytes(k, n) / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 1),
                           "copies": copies}
        if peak:
            out[f"{k}x{n}"]["pct_of_measured_peak"] = round(100 * alg_bytes(k, n) / (us * 1e-6) / 1e9 / peak, 1)
        del cl
        torch.cuda.empty_cache()
    return out


# the shapes the per-shape table adds to the step's 1.5B / 3B shapes: BASELINE configs[0]'s Qwen2.5-0.5B gate/up
# and the 7B-shaped MLP projections of configs[2]
SHAPES_EXTRA = [("0.5b.gate_up", 896, 4864), ("7b.gate", 3584, 18944), ("7b.down", 18944, 3584)]
# the skinny block of the default line: every (shape, M) of BASELINE configs[2] above M = 1 (the M = 2..64 half of
# the metric; M = 1 is per_shape)
SKINNY_BLOCK = [("3b.gate_up", 2048, 11008), ("3b.down", 11008, 2048), ("7b.gate_up", 3584, 18944),
                ("7b.down", 18944, 3584)]
SKINNY_BLOCK_M = (2, 4, 8, 16, 24, 32, 48, 64)
MFMA_F16_PEAK_TFLOPS = 2500.0               # MI355X dense fp16 MFMA


def _sha256_files(paths):
    h = hashlib.sha256()
    for path in sorted(paths):
        h.update(str(path.relative_to(ROOT)).encode())
        h.update(path.read_bytes())
    return h.hexdigest()[:16]


def provenance(torch, ops):
    """What the numbers were measured on and with (reference bench/gpu_run.py:41-66): GPU, driver-visible versions,
    the source and library hashes, the git commit when the tree has one, and the dispatch constants."""
    import subprocess
    props = torch.cuda.get_device_properties(0)
    pkg = ROOT / "lowbit-kernels_amd"
    sources = [*(pkg / "csrc").glob("*"), *(pkg / "lowbit").glob("*.py"), *(ROOT / "include").glob("*.h"),
               ROOT / "bench.py"]
    lib = pkg / "lowbit" / "liblowbit_w4.so"
    try:
        commit = subprocess.run(["git", "-C", str(ROOT), "rev-parse", "HEAD"], capture_output=True, text=True,
                                timeout=10).stdout.strip() or None
    except (OSError, subprocess.SubprocessError):
        commit = None
    built_from = None                                       # the commit the library was built from (build.py)
    info = pkg / "lowbit" / "build_info.json"
    if info.exists():
        try:
            built_from = json.loads(info.read_text())
        except ValueError:
            built_from = None
    return {"gpu": props.name, "gcn_arch": getattr(props, "gcnArchName", None), "cus": props.multi_processor_count,
            "hbm_gib": round(props.total_memory / 2 ** 30, 1), "torch": torch.__version__,
            "hip": getattr(torch.version, "hip", None), "git_commit": commit, "library_built_from": built_from,
            "sources_sha256": _sha256_files([q for q in sources if q.is_file()]),
            "library_sha256": _sha256_files([lib]) if lib.exists() else None,
            "library": ops._native.lib().lowbit_version().decode(),
            "dispatch": {name: getattr(ops, name) for name in dir(ops) if name.startswith("AUTO_")},
            "host": {"cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads()}}


def skinny_block(torch, ops):
    """The M = 2..64 half of the metric (the 3B and 7B-shaped MLP projections at M = 2, 4, 8,
    16, 24, 32, 48, 64): us per call of the MFMA kernel (v5), dequantize + hipBLASLt and fp16 hipBLASLt, each a graph
    over >= 1 GiB of cold copies (int4 for the first two, fp16 for the last); the v5 kernel's algorithmic bandwidth
    and its MFMA utilisation (2 M N K / t against the 2.5 PFLOP/s dense fp16 peak)."""
    rows = []
    for name, k, n in SKINNY_BLOCK:
        pool, pool16, _, copies = build_pool(torch, ops, [(name, k, n)], fp16=True, seed=k + n)
        iters = max(200, copies)
        for m in SKINNY_BLOCK_M:
            x = torch.randn(m, k, device="cuda").half()
            v5 = graph_time_us(torch, lambda i: ops.gemv(x, pool[i % copies][name], 5), iters)
            dq = graph_time_us(torch, lambda i: torch.nn.functional.linear(x, ops.dequant(pool[i % copies][name],
                                                                                            "mma")), iters)
            f16 = graph_time_us(torch, lambda i: torch.nn.functional.linear(x, pool16[i % copies][name]), iters)
            rows.append({"shape": name, "K": k, "N": n, "M": m, "mfma_v5_us": round(v5, 2),
                         "dequant_hipblaslt_us": round(dq, 2), "fp16_hipblaslt_us": round(f16, 2),
                         "v5_vs_dequant": round(dq / v5, 2), "v5_vs_fp16": round(f16 / v5, 2),
                         "v5_GBps": round(alg_bytes(k, n, m) / (v5 * 1e-6) / 1e9, 1),
                         "v5_mfma_util": round(2.0 * m * n * k / (v5 * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)})
        del pool, pool16
        torch.cuda.empty_cache()
    return rows


# BASELINE configs[4] in the default line: a 512-token prompt, greedy tokens and tokens fed 16 / 48 per step
DECODE_BLOCK = dict(model="3b", prompt=512, new=128, feed=192, chunks=(16, 48))


def decode_block(torch, ops):
    """Batch-1 decode of a random-init Qwen2.5-3B architecture, every step one hipGraph replay:
    * fused layers (lowbit.fused, 5 launches per layer for one token) with W4A16 projections (int4 g128, clip search),
      with fp16 projections through the library's fp16-weight GEMV (the same kernel structure, epilogues and fusions:
      only the weight bytes differ; multi-token steps use hipBLASLt), and with fp16 projections through hipBLASLt;
    * transformers' own modules with fp16 nn.Linear and with the W4Linear drop-in (the reference's comparison,
      bench/e2e.py:84-147), greedy only.
    Per variant: TTFT (median of 3 eager prefills of the prompt), greedy ms/token (one warm-up run, then the timed
    run), tokens/s fed `chunks` tokens per step; bytes per greedy token (projection weights + tied head + the KV rows
    read at the mean position) and that over the step time. Speed-ups W4A16 / fp16 both ways."""
    from lowbit import decode, fused, model as lbmodel
    cfg = DECODE_BLOCK
    m = decode.random_model(cfg["model"], seed=0)
    mc = m.config
    vocab, hidden, layers = mc.vocab_size, mc.hidden_size, mc.num_hidden_layers
    gen = torch.Generator(device="cuda").manual_seed(2024)
    prompt = torch.randint(0, vocab, (1, cfg["prompt"]), generator=gen, device="cuda")
    feed = torch.randint(0, vocab, (cfg["feed"],), generator=gen, device="cuda")
    max_len = cfg["prompt"] + max(cfg["new"], cfg["feed"]) + 64
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    mean_pos = cfg["prompt"] + cfg["new"] / 2
    kv_bytes = layers * 2 * mc.num_key_value_heads * 128 * 2 * mean_pos
    head_bytes = vocab * hidden * 2

    def timed(fn):
        e0, e1 = ev(), ev()
        e0.record()
        r = fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1), r

    def run(make, chunks, weight_bytes):
        dec = make(1)
        ttft = sorted(timed(lambda: dec.prefill(prompt).argmax(-1))[0] for _ in range(3))[1]
        dec.capture()
        for _ in range(2):                                   # a warm-up run, then the timed one
            first = dec.prefill(prompt).argmax(-1)
            ms, _ = timed(lambda: dec.greedy(first, cfg["new"]))
        del dec
        per_tok = ms / (cfg["new"] - 1)
        step_bytes = weight_bytes + head_bytes + kv_bytes
        r = {"ttft_ms": round(ttft, 3), "greedy_ms_per_token": round(per_tok, 4),
             "greedy_tokens_per_s": round(1000 / per_tok, 1), "bytes_per_token": int(step_bytes),
             "bytes_per_token_TBps": round(step_bytes / (per_tok * 1e-3) / 1e12, 3)}
        for c in chunks:
            dc = make(c)
            dc.prefill(prompt)
            dc.capture()
            best = 1e30
            for _ in range(2):
                dc.prefill(prompt)
                t, _ = timed(lambda: [dc.step(feed[i:i + c]) for i in range(0, cfg["feed"], c)])
                best = min(best, t)
            r[f"feed_{c}_tokens_per_s"] = round(cfg["feed"] / (best / 1000), 1)
            del dc
        torch.cuda.empty_cache()
        return r

    def fused_bytes(fq):
        b = 0
        for lay in fq.layers:
            for name in ("qkv", "o", "gu", "down"):
                pj = lay[name]
                b += pj.wq.nbytes() if hasattr(pj, "wq") else pj.w.numel() * 2
        return b

    out = {}
    fq = fused.FusedQwen2(m, max_len, quant="int4", clip_grid=CLIP_GRID)
    out["fused_int4"] = run(lambda c: fused.FusedDecoder(fq, c), cfg["chunks"], fused_bytes(fq))
    del fq
    fq = fused.FusedQwen2(m, max_len, quant="fp16_gemv")
    out["fused_fp16_gemv"] = run(lambda c: fused.FusedDecoder(fq, c), cfg["chunks"], fused_bytes(fq))
    del fq
    fq = fused.FusedQwen2(m, max_len, quant="fp16")
    out["fused_fp16_hipblaslt"] = run(lambda c: fused.FusedDecoder(fq, c), cfg["chunks"], fused_bytes(fq))
    del fq
    torch.cuda.empty_cache()
    linear_bytes = sum(mod.weight.numel() * 2 for name, mod in m.model.layers.named_modules()
                       if name.split(".")[-1] in lbmodel.TARGETS)
    out["hf_fp16"] = run(lambda c: decode.GraphDecoder(m, max_len, c), (), linear_bytes)
    layers_q = lbmodel.quantize_layers(m, GROUP, CLIP_GRID)
    _, int4_bytes = lbmodel.apply_int4(layers_q)
    out["hf_w4linear"] = run(lambda c: decode.GraphDecoder(m, max_len, c), (), int4_bytes)
    del m, layers_q
    torch.cuda.empty_cache()

    def sp(a, b, key):
        return round(out[b][key] / out[a][key], 3) if key.startswith("greedy_ms") else round(out[a][key] / out[b][key], 3)
    keys = ["greedy_ms_per_token"] + [f"feed_{c}_tokens_per_s" for c in cfg["chunks"]]
    return {"workload": f"BASELINE configs[4]: random-init Qwen2.5-{cfg['model']} architecture (no checkpoint), "
                        f"{cfg['prompt']}-token uniform-random prompt, {cfg['new']} greedy tokens, {cfg['feed']} "
                        f"tokens fed {'/'.join(map(str, cfg['chunks']))} per step; int4 g128 with the clip search",
            "variants": out,
            "speedup_w4a16": {
                "fused_int4_over_fused_fp16_gemv": {k: sp("fused_int4", "fused_fp16_gemv", k) for k in keys},
                "fused_int4_over_fused_fp16_hipblaslt": {k: sp("fused_int4", "fused_fp16_hipblaslt", k) for k in keys},
                "hf_w4linear_over_hf_fp16": {"greedy_ms_per_token": sp("hf_w4linear", "hf_fp16",
                                                                       "greedy_ms_per_token")},
                "fused_int4_over_hf_fp16": {"greedy_ms_per_token": sp("fused_int4", "hf_fp16",
                                                                      "greedy_ms_per_token")}},
            "ttft_ms": {k: v["ttft_ms"] for k, v in out.items()}}


def host_cost(a):
    """Host cost of one M = 1 call and eager decode (reference bench/gpu_run.py:304-322, bench/e2e.py:54-69).
    * Per call, interleaved over rounds (min of 7 rounds of 2000 back-to-back calls, wall time / calls after a
      synchronization): the C entry point through ctypes with a preallocated output (the floor), ext().w4_gemv
      (validation, torch.empty, launch), ops.gemv and ops.linear (routing on top), on a small and a mid-size decode
      layer, next to the GPU time per call of the same launch in a graph: where wall > graph time the host is the
      bound in eager mode.
    * Eager greedy decode (every step launched op by op) of the random-init Qwen2.5-3B architecture against the
      graph replay, for the fused layers (W4A16 and fp16 through the same GEMV) and transformers' modules (fp16 and
      the W4Linear drop-in)."""
    import ctypes
    import torch
    from lowbit import _native, decode, fused, ops, model as lbmodel
    torch.cuda.set_device(0)
    lib, ext = _native.lib(), ops.ext()
    out = {"per_call_us": {}}
    for k, n in ((1536, 256), (2048, 2048)):
        wq = ops.W4Weight.from_float(torch.randn(n, k, device="cuda") * 0.02, GROUP, ("mma",))
        x = torch.randn(1, k, device="cuda").half()
        y = torch.empty(1, n, dtype=torch.half, device="cuda")
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        args = (_native.ptr(x), _native.ptr(wq.packed_mma), _native.ptr(wq.scales), _native.ptr(y), 1, n, k, GROUP, 6,
                0, st)
        calls = {"c_abi_ctypes": lambda: lib.lowbit_w4_gemv(*args),
                 "ext_w4_gemv": lambda: ext.w4_gemv(x, wq.packed_mma, wq.scales, GROUP, 6),
                 "ops_gemv": lambda: ops.gemv(x, wq, 6),
                 "ops_linear": lambda: ops.linear(x, wq)}
        best = {name: 1e30 for name in calls}
        for _ in range(7):
            for name, fn in calls.items():
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for _ in range(2000):
                    fn()
                torch.cuda.synchronize()
                best[name] = min(best[name], (time.perf_counter() - t0) / 2000 * 1e6)
        r = {name: round(v, 2) for name, v in best.items()}
        r["gpu_graph_us"] = round(graph_time_us(torch, lambda i: ops.linear(x, wq), 2000), 2)
        out["per_call_us"][f"{k}x{n}"] = r
        progress(f"host cost {k}x{n}: {r}")
    cfg = DECODE_BLOCK
    m = decode.random_model(cfg["model"], seed=0)
    gen = torch.Generator(device="cuda").manual_seed(2024)
    prompt = torch.randint(0, m.config.vocab_size, (1, cfg["prompt"]), generator=gen, device="cuda")
    n_tok = 32
    max_len = cfg["prompt"] + 2 * n_tok + 16

    def run(dec):
        res = {}
        for mode in ("graph", "eager"):
            first = dec.prefill(prompt).argmax(-1)
            if mode == "graph":
                dec.capture()
                first = dec.prefill(prompt).argmax(-1)
                fn = lambda: dec.greedy(first, n_tok)  # noqa: E731
            else:
                fn = lambda: dec.eager_greedy(first, n_tok)  # noqa: E731
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            res[f"{mode}_ms_per_token"] = round((time.perf_counter() - t0) * 1000 / (n_tok - 1), 4)
        res["eager_over_graph"] = round(res["eager_ms_per_token"] / res["graph_ms_per_token"], 3)
        return res
    dec_out = {}
    for quant in ("int4", "fp16_gemv"):
        fq = fused.FusedQwen2(m, max_len, quant=quant, clip_grid=CLIP_GRID if quant == "int4" else None)
        run(fused.FusedDecoder(fq, 1))                       # warm-up of both modes
        dec_out[f"fused_{quant}"] = run(fused.FusedDecoder(fq, 1))
        del fq
        torch.cuda.empty_cache()
    run(decode.GraphDecoder(m, max_len, 1))
    dec_out["hf_fp16"] = run(decode.GraphDecoder(m, max_len, 1))
    lbmodel.apply_int4(lbmodel.quantize_layers(m, GROUP, CLIP_GRID))
    run(decode.GraphDecoder(m, max_len, 1))
    dec_out["hf_w4linear"] = run(decode.GraphDecoder(m, max_len, 1))
    out["decode_3b"] = {"tokens": n_tok, "prompt": cfg["prompt"], **dec_out,
                        "eager_w4_over_fp16": {
                            "fused": round(dec_out["fused_fp16_gemv"]["eager_ms_per_token"] /
                                           dec_out["fused_int4"]["eager_ms_per_token"], 3),
                            "transformers": round(dec_out["hf_fp16"]["eager_ms_per_token"] /
                                                  dec_out["hf_w4linear"]["eager_ms_per_token"], 3)}}
    out["host"] = {"cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads()}
    print(json.dumps(out), flush=True)
    if a.out:
        pathlib.Path(a.out).write_text(json.dumps(out, indent=1))


def per_shape_extra(torch, ops, peak=None):
    """The configs[0] and 7B-shaped projections, per call like shape_detail, on one clip-searched weight cloned into
    >= 1 GiB."""
    out = {}
    gen = torch.Generator(device="cuda").manual_seed(7)
    for name, k, n in SHAPES_EXTRA:
        w = torch.randn(n, k, generator=gen, device="cuda") * 0.02
        packed, scales = ops.quantize_w4_gpu(w, GROUP, CLIP_GRID)
        base = ops.W4Weight(packed, scales, GROUP, ("mma",), device=packed.device)
        del w
        x = torch.randn(1, k, generator=gen, device="cuda").half()
        out.update(shape_detail(torch, ops, [(name, k, n)], [{name: base}], {name: x}, peak))
        del base, packed, scales
        torch.cuda.empty_cache()
    return out


def per_shape_workload(a):
    """Profiler workload: only the per-shape graphs (the 8 decode shapes of the step and the two 7B shapes), so a
    kernel trace gives each shape's own GEMV duration (one grid size per shape)."""
    import torch
    from lowbit import ops
    torch.cuda.set_device(0)
    projs = step_projections()
    pool, _, _, _ = build_pool(torch, ops, projs, gib=0.01)
    gen = torch.Generator(device="cuda").manual_seed(1)
    xs = {name: torch.randn(1, k, generator=gen, device="cuda").half() for name, k, n in projs}
    detail = shape_detail(torch, ops, projs, pool, xs)
    detail.update(per_shape_extra(torch, ops))
    print(json.dumps({"per_shape_workload": True, "per_shape": detail}), flush=True)


GEMV_KERNEL = "gemv_mfma_layout"


def progress(msg):
    """A stage finished (stderr: stdout carries only the JSON line)."""
    print(f"[bench] {msg} ({time.strftime('%H:%M:%S')})", file=sys.stderr, flush=True)


def traced_gemv(a):
    """The timed workload (this script with --trace-child: pool, warm-up, capture, one untimed and `replays` timed
    replays of the K-step graph) run under `rocprofv3 --kernel-trace --stats`, the command whose summary is kept with
    the profiles (with the same --steps, --warmup and --replays: the same trace taken standalone on one box averaged
    3.89 us per GEMV dispatch against 3.80 here, while 20-step graphs average 4.62), before this process touches the
    GPU. Returns
    the durations of the GEMV dispatches of the timed replays (the last replays x steps x 14 of them) from the trace's
    own start / end stamps, the traced replays' wall time per launch (first start to last end: the tracer's gaps
    between dispatches), and per-instance averages; None when rocprofv3 is missing or the run fails."""
    import csv
    import glob
    import shutil
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3") or ("/opt/rocm/bin/rocprofv3" if os.path.exists("/opt/rocm/bin/rocprofv3") else None)
    if prof is None:
        return None
    tmp = tempfile.mkdtemp(prefix="lowbit_trace_")
    cmd = [prof, "--kernel-trace", "--stats", "--output-format", "csv", "-d", tmp, "-o", "head", "--", sys.executable, "-u",
           str(ROOT / "bench.py"), "--trace-child", "--steps", str(a.steps), "--warmup", str(a.warmup), "--replays",
           str(a.replays)]
    try:
        subprocess.run(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, timeout=600, cwd="/tmp",
                       env={**os.environ, "TMPDIR": "/tmp"})
    except (OSError, subprocess.SubprocessError):
        pass                        # the profiler may end abnormally after a complete trace: the files decide
    rows = []
    for path in glob.glob(os.path.join(tmp, "**", "*kernel_trace.csv"), recursive=True):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                if GEMV_KERNEL in r.get("Kernel_Name", ""):
                    rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    shutil.rmtree(tmp, ignore_errors=True)
    n = a.replays * a.steps * len(step_projections())
    if len(rows) < n:
        return None
    rows = sorted(rows)[-n:]
    dur = [(e - b) / 1000 for b, e, _ in rows]
    # a dispatch whose start stamp precedes the previous one's end had been queued behind it (the graph's launches are
    # ordered): how often, and the durations counted from the later of the two stamps
    overlaps = sum(1 for p, c in zip(rows, rows[1:]) if c[0] < p[1])
    busy = [dur[0]] + [(c[1] - max(c[0], p[1])) / 1000 for p, c in zip(rows, rows[1:])]
    last = rows[-a.steps * len(step_projections()):]        # the final replay alone
    per = {}
    for (b, e, name), d in zip(rows, dur):
        key = name[name.find(GEMV_KERNEL):].split("(")[0]   # the instance: template arguments
        per.setdefault(key, []).append(d)
    return {"avg_us": sum(dur) / len(dur), "dispatches": len(dur),
            "traced_wall_us_per_launch": (last[-1][1] - last[0][0]) / 1000 / len(last),
            "overlapping_dispatches": overlaps, "busy_avg_us": sum(busy) / len(busy),
            "instances": {k: {"calls": len(v), "avg_us": round(sum(v) / len(v), 3)} for k, v in sorted(per.items())}}


def roofline(trace, bytes_per_launch, graph_us, launches):
    """The GEMV kernel's roofline entry. With a trace, its average launch duration is the traced kernel duration
    (each dispatch timed alone by the profiler: the conservative figure, reproducible from a rocprofv3 summary of the
    same command); the untimed-graph figure, elapsed / launches (back-to-back launches overlap their dispatch), is
    kept beside it. Without one, the graph figure."""
    avg = trace["avg_us"] if trace else graph_us
    r = {"bound": "hbm", "achieved": round(bytes_per_launch / (avg * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBPS,
         "unit": "GB/s", "frac": round(bytes_per_launch / (avg * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
         "traffic": TRAFFIC_PER_LAUNCH,
         # one kernel template, three instances by layer: whole 16-row tiles (CS = 1: the 1.5B q/k/v/o and both
         # models' gate/up), tiles split over 2 workgroups (3B q/o, both downs) or 4 (3B k/v)
         "kernel": "lowbit::gemv_mfma_layout<1,1,4,true,false,CS>, CS = 1 / 2 / 4",
         "kernel_avg_us": round(avg, 3), "bytes_per_launch_avg": bytes_per_launch, "launches": launches,
         "kernel_avg_source": ("rocprofv3 --kernel-trace of the same timed workload (bench.py --trace-child), "
                               "mean duration of the timed replays' GEMV dispatches" if trace else
                               "graph elapsed / launches (no trace)"),
         "graph_us_per_launch": round(graph_us, 3),
         "graph_achieved": round(bytes_per_launch / (graph_us * 1e-6) / 1e9, 1),
         "frac_graph": round(bytes_per_launch / (graph_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}
    if trace:
        r["trace"] = {"dispatches": trace["dispatches"], "instances": trace["instances"],
                      "traced_wall_us_per_launch": round(trace["traced_wall_us_per_launch"], 3),
                      "overlapping_dispatches": trace["overlapping_dispatches"],
                      "busy_avg_us": round(trace["busy_avg_us"], 3)}
    return r


def contract(a):
    import torch
    from lowbit import ops
    from oracle import quant_ref as R

    torch.cuda.set_device(0)
    projs = step_projections()
    step_bytes = sum(alg_bytes(k, n) for _, k, n in projs)
    pool, pool16, host, copies = build_pool(torch, ops, projs, fp16=not a.no_fp16)
    gen = torch.Generator(device="cuda").manual_seed(1)
    xs = {name: torch.randn(1, k, generator=gen, device="cuda").half() for name, k, n in projs}

    # parity check before timing: every projection of copy 0 against the oracle's fp64 GEMV on the host copy
    for name, k, n in projs:
        packed, scales = host[0][name]
        ref = R.gemv_reference(xs[name].double().cpu().numpy(), packed, scales, GROUP)
        err = R.rel_err(ops.linear(xs[name], pool[0][name]).cpu().numpy(), ref)
        if err > R.REL_BOUND:
            raise SystemExit(f"parity check failed on {name}: {err:.2e}")

    def step(i):
        layer = pool[i % copies]
        for name, k, n in projs:
            ops.linear(xs[name], layer[name])

    for i in range(a.warmup):
        step(i)
    torch.cuda.synchronize()

    # the K timed steps: one graph replay between two synchronizations
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(0)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(a.steps):
            step(i)
    graph.replay()                                   # one untimed replay: instantiation and first-touch costs
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    replay_ms = []
    for _ in range(max(1, a.replays)):             # the first is the contract's timed region; the rest give the spread
        torch.cuda.synchronize()
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        replay_ms.append(e0.elapsed_time(e1))
    elapsed_ms = replay_ms[0]
    del graph
    launches = len(projs) * a.steps
    value = step_bytes * a.steps / (elapsed_ms / 1e3) / 1e9

    # fp16 BLAS on the same cold rotation (dequantized weights), one graph of K steps
    fp16 = None
    if pool16 and pool16[0]:
        def step16(i):
            layer = pool16[i % copies]
            for name, k, n in projs:
                torch.nn.functional.linear(xs[name], layer[name])
        fp16 = graph_time_us(torch, step16, a.steps, reps=1) / 1000
    progress(f"timed region done: {value:.1f} GB/s")
    peak = None if a.no_detail else measured_peak(torch, ops)
    detail = None if a.no_detail else shape_detail(torch, ops, projs, pool, xs, peak["read_gbps"])
    if detail is not None:
        detail.update(per_shape_extra(torch, ops, peak["read_gbps"]))
    progress("per-shape table done")
    skinny = None if a.no_detail else skinny_block(torch, ops)
    progress("skinny table done")
    decode_line = None if (a.no_detail or a.no_decode) else decode_block(torch, ops)
    progress("decode block done")
    by_step = sorted(step_bytes / (t / a.steps / 1e3) / 1e9 for t in replay_ms)

    line = {
        "metric": "W4A16 GEMV HBM GB/s (% of peak) at M=1; us/call M=1..64 vs hipBLASLt fp16",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(elapsed_ms / a.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x fp16 activations, fp32 accumulate",
        "data": "synthetic: random N(0,0.02) weights (int4 g128, clip search), N(0,1) fp16 x, "
                f"{copies} distinct layer copies ({copies * sum(w4_bytes(k, n) for _, k, n in projs) / 2**30:.2f} GiB) cycled",
        "config": {"workload": "BASELINE configs[1]: M=1 GEMV over the 7 projections of one Qwen2.5-1.5B and one "
                               "Qwen2.5-3B decoder layer per step (14 launches), hipGraph replay",
                   "step_bytes": step_bytes, "M": 1, "group": GROUP, "parallelism": "single GPU"},
        "roofline": roofline(a.trace, step_bytes // len(projs), 1000 * elapsed_ms / launches, launches),
        "replays": {"n": len(replay_ms), "ms_per_step": [round(t / a.steps, 4) for t in replay_ms],
                    "GBps_median": round(by_step[len(by_step) // 2], 1), "GBps_min": round(by_step[0], 1),
                    "GBps_max": round(by_step[-1], 1)},
        "fp16_blas_ms_per_step": round(fp16, 4) if fp16 else None,
        "speedup_vs_fp16_blas": round(fp16 / (elapsed_ms / a.steps), 3) if fp16 else None,
        "blas_backend": str(torch.backends.cuda.preferred_blas_library()),
        "measured_peak": peak,
        "per_shape": detail,
        "skinny": skinny,
        "decode": decode_line,
        "provenance": provenance(torch, ops),
    }
    if peak:
        line["roofline"]["measured_peak_gbps"] = peak["read_gbps"]
        line["roofline"]["frac_of_measured_peak"] = round(line["roofline"]["achieved"] / peak["read_gbps"], 4)
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline(projs, host, xs)
    print(json.dumps(line), flush=True)
    if a.out:
        pathlib.Path(a.out).write_text(json.dumps(line, indent=1))


def sweep_skinny(a):
    """M in {1,2,4,8,16,24,32,48,64} on 3B and 7B-shaped MLP layers; us/call for the v6 GEMV
    (M <= 8), the MFMA kernel (v5), dequant + BLAS, and fp16 BLAS, each a graph cycling >= 1 GiB of copies."""
    import torch
    from lowbit import ops
    torch.cuda.set_device(0)
    shapes = [("3b.gate_up", 2048, 11008), ("3b.down", 11008, 2048), ("7b.gate_up", 3584, 18944), ("7b.down", 18944, 3584)]
    ms = [1, 2, 4, 8, 16, 24, 32, 48, 64]
    rows = []
    for name, k, n in shapes:
        projs = [(name, k, n)]
        pool, pool16, _, copies = build_pool(torch, ops, projs, fp16=True, seed=k + n)
        for m in ms:
            x = torch.randn(m, k, device="cuda").half()
            r = {"shape": name, "K": k, "N": n, "M": m, "copies": copies}

            def timed(fn, iters=max(200, copies)):
                fn(0)
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for i in range(iters):
                        fn(i)
                g.replay()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                best = 1e30
                for _ in range(3):
                    e0.record()
                    g.replay()
                    e1.record()
                    torch.cuda.synchronize()
                    best = min(best, e0.elapsed_time(e1) * 1000 / iters)
                return round(best, 2)

            if m <= 8:
                r["gemv_v6_us"] = timed(lambda i: ops.gemv(x, pool[i % copies][name], 6))
            r["mfma_v5_us"] = timed(lambda i: ops.gemv(x, pool[i % copies][name], 5))
            r["dequant_blas_us"] = timed(lambda i: torch.nn.functional.linear(x, ops.dequant(pool[i % copies][name], "mma")))
            r["fp16_blas_us"] = timed(lambda i: torch.nn.functional.linear(x, pool16[i % copies][name]))
            r["linear_us"] = timed(lambda i: ops.linear(x, pool[i % copies][name]))
            r["linear_path"] = ops.auto_version(m, pool[0][name]) or "dequant+blas"
            r["int4_roofline_us"] = round(alg_bytes(k, n, m) / (HBM_PEAK_GBPS * 1e9) * 1e6, 2)
            rows.append(r)
            print(json.dumps(r), flush=True)
        del pool, pool16
        torch.cuda.empty_cache()
    if a.out:
        pathlib.Path(a.out).write_text(json.dumps(rows, indent=1))


# decode projections of the Qwen2.5-1.5B / 3B / 7B layers (K, N): q, k|v, o, gate / up, down and the merged q|k|v,
# gate|up
SWEEP_SHAPES = [(1536, 256), (1536, 1536), (1536, 2048), (1536, 8960), (1536, 17920), (8960, 1536), (2048, 256),
                (2048, 2048), (2048, 2560), (2048, 11008), (2048, 22016), (11008, 2048), (3584, 512), (3584, 3584),
                (3584, 4608), (3584, 18944), (18944, 3584)]


def cloned_copies(torch, ops, k, n, gib=1.0):
    """One absmax-quantized weight, cloned into >= gib GiB of copies (each call reads a cold copy)."""
    w = torch.randn(n, k, device="cuda") * 0.02
    p, s = ops.quantize_w4_gpu(w, GROUP)
    base = ops.W4Weight(p, s, GROUP, ("mma",))
    out = []
    for _ in range(int(-(-gib * 2 ** 30 // w4_bytes(k, n)))):
        c = ops.W4Weight.__new__(ops.W4Weight)
        c.__dict__.update(base.__dict__)
        c.packed_mma, c.scales = base.packed_mma.clone(), base.scales.clone()
        out.append(c)
    return out


def sweep_gemv(a):
    """M=1 GEMV (v6) per decode shape: graph-timed us per call of the automatic plan and of every tile split
    CS (lowbit_set_launch_override k_splits: 1, 2, 4 workgroups per 16-row tile) x waves per workgroup."""
    import torch
    from lowbit import _native, ops
    torch.cuda.set_device(0)
    lib = _native.lib()
    rows = []
    for k, n in SWEEP_SHAPES:
        cl = cloned_copies(torch, ops, k, n)
        x = torch.randn(1, k, device="cuda").half()
        t = lambda: round(graph_time_us(torch, lambda i: ops.gemv(x, cl[i % len(cl)], 6), max(400, len(cl))), 2)
        _native.check(lib.lowbit_set_launch_override(0, 0, 0))
        r = {"K": k, "N": n, "auto_us": t(), "cs_waves_us": {}}
        kc = k // 128
        for cs in (1, 2, 4):
            for waves in (1, 2, 4, 8, 16):
                if kc % cs == 0 and waves <= kc // cs:
                    _native.check(lib.lowbit_set_launch_override(waves, 0, cs))
                    r["cs_waves_us"][f"{cs}x{waves}"] = t()
        _native.check(lib.lowbit_set_launch_override(0, 0, 0))
        rows.append(r)
        print(json.dumps(r), flush=True)
        del cl
        torch.cuda.empty_cache()
    if a.out:
        pathlib.Path(a.out).write_text(json.dumps(rows, indent=1))


LDS_RING_SHAPES = [(896, 4864), (1536, 256), (1536, 1536), (1536, 8960), (1536, 17920), (8960, 1536), (2048, 256),
                   (2048, 2048), (2048, 2560), (2048, 11008), (2048, 22016), (11008, 2048), (3584, 18944),
                   (18944, 3584)]


def sweep_ldsring(a):
    """M=1 GEMV (v6) per decode shape: graph-timed us per call with the weight ring in registers (automatic plan)
    against the ring in LDS (lowbit_set_gemv_lds_ring: 4, 8, 12, 16 slots per wave) at the automatic wave count and
    at every wave count 1..16 (lowbit_set_launch_override, the automatic tile split)."""
    import torch
    from lowbit import _native, ops
    torch.cuda.set_device(0)
    lib = _native.lib()
    rows = []
    for k, n in LDS_RING_SHAPES:
        cl = cloned_copies(torch, ops, k, n)
        x = torch.randn(1, k, device="cuda").half()
        t = lambda: round(graph_time_us(torch, lambda i: ops.gemv(x, cl[i % len(cl)], 6), max(400, len(cl))), 2)
        _native.check(lib.lowbit_set_launch_override(0, 0, 0))
        _native.check(lib.lowbit_set_gemv_lds_ring(-1))
        r = {"K": k, "N": n, "registers_us": t(), "lds_us": {}}
        for lr in (4, 8, 12, 16):
            _native.check(lib.lowbit_set_gemv_lds_ring(lr))
            for waves in (0, 1, 2, 4, 8, 16):
                if waves and waves > k // 128:
                    continue
                _native.check(lib.lowbit_set_launch_override(waves, 0, 0))
                r["lds_us"][f"{lr}x{waves}"] = t()
        _native.check(lib.lowbit_set_launch_override(0, 0, 0))
        _native.check(lib.lowbit_set_gemv_lds_ring(0))
        best = min(r["lds_us"], key=r["lds_us"].get)
        r["best_lds"] = [best, r["lds_us"][best]]
        rows.append(r)
        print(json.dumps(r), flush=True)
        del cl
        torch.cuda.empty_cache()
    if a.out:
        pathlib.Path(a.out).write_text(json.dumps(rows, indent=1))


ORDER_SHAPES = [(11008, 2048), (8960, 1536), (18944, 3584), (2048, 2048), (3584, 3584), (2048, 2560), (1536, 2048),
                (3584, 4608)]


def sweep_order(a):
    """MFMA GEMM (v5) with a K split, M = 2..64: graph-timed us per call with the row groups fastest in the
    workgroup order (lowbit_set_gemm_order 1) and with the splits fastest (2), over >= 1 GiB of cold copies."""
    import torch
    from lowbit import _native, ops
    torch.cuda.set_device(0)
    lib = _native.lib()
    rows = []
    for k, n in ORDER_SHAPES:
        cl = cloned_copies(torch, ops, k, n)
        r = {"K": k, "N": n, "us": {}}
        for m in SKINNY_BLOCK_M:
            x = torch.randn(m, k, device="cuda").half()
            for order in (1, 2):
                _native.check(lib.lowbit_set_gemm_order(order))
                r["us"][f"{m}:{order}"] = round(graph_time_us(torch, lambda i: ops.gemv(x, cl[i % len(cl)], 5),
                                                              max(400, len(cl))), 2)
        _native.check(lib.lowbit_set_gemm_order(0))
        rows.append(r)
        print(json.dumps(r), flush=True)
        del cl
        torch.cuda.empty_cache()
    if a.out:
        pathlib.Path(a.out).write_text(json.dumps(rows, indent=1))


def sweep_tiles(a):
    """MFMA GEMM (v5) per decode shape and M in 2..64: graph-timed us per call of the row-group kernel (automatic
    shape), of one tile per workgroup with 2, 4 and 8 waves, and of the automatic choice (lowbit_set_gemm_kernel)."""
    import torch
    from lowbit import _native, ops
    torch.cuda.set_device(0)
    lib = _native.lib()
    rows = []
    for k, n in SWEEP_SHAPES:
        cl = cloned_copies(torch, ops, k, n)
        for m in (2, 4, 8, 16, 24, 32, 40, 48, 56, 64):
            x = torch.randn(m, k, device="cuda").half()
            t = lambda: round(graph_time_us(torch, lambda i: ops.gemv(x, cl[i % len(cl)], 5), max(300, len(cl))), 2)
            r = {"K": k, "N": n, "M": m}
            for name, kern, waves in (("rows", 1, 0), ("tiles_2", 2, 2), ("tiles_4", 2, 4), ("tiles_8", 2, 8),
                                      ("auto", 0, 0)):
                _native.check(lib.lowbit_set_gemm_kernel(kern))
                _native.check(lib.lowbit_set_launch_override(waves, 0, 0))
                r[name] = t()
            _native.check(lib.lowbit_set_gemm_kernel(0))
            _native.check(lib.lowbit_set_launch_override(0, 0, 0))
            rows.append(r)
            print(json.dumps(r), flush=True)
        del cl
        torch.cuda.empty_cache()
    if a.out:
        pathlib.Path(a.out).write_text(json.dumps(rows, indent=1))


def sweep_tilewaves(a):
    """MFMA GEMM (v5) row groups on layers of 560 to 2368 tiles, M in {16, 32, 48, 64}: graph-timed us per call of the
    automatic plan, of 4 tile-waves per K-group (lowbit_set_gemm_tile_waves(4), the rest automatic) and of 3, 4, 5, 6
    and 8 tile-waves with 1, 2 or 4 K-groups, where the library builds them."""
    import torch
    from lowbit import _native, ops
    torch.cuda.set_device(0)
    lib = _native.lib()

    def built(tw, ks, mt):                                 # kernels.hpp gemm_fits with one tile per wave, 2 slots
        if tw == 3:
            return ks <= 2 or mt <= 2
        if tw == 4:
            return ks <= 2 or mt <= 3
        return ks <= 2 and (tw * ks <= 12 or mt <= 3)

    rows = []
    for k, n in ((3584, 18944), (2048, 22016), (1536, 17920), (3584, 37888), (2048, 11008), (1536, 8960),
                 (3584, 16384)):
        cl = cloned_copies(torch, ops, k, n)
        for m in (16, 32, 48, 64):
            x = torch.randn(m, k, device="cuda").half()
            t = lambda: round(graph_time_us(torch, lambda i: ops.gemv(x, cl[i % len(cl)], 5), max(400, len(cl))), 2)
            r = {"K": k, "N": n, "M": m, "auto": t()}
            try:
                _native.check(lib.lowbit_set_gemm_tile_waves(4))
                r["tw4"] = t()
                for tw in (3, 4, 5, 6, 8):
                    for ks in (1, 2, 4):
                        if not built(tw, ks, (m + 15) // 16):
                            continue
                        _native.check(lib.lowbit_set_gemm_tile_waves(tw))
                        _native.check(lib.lowbit_set_launch_override(4 * ks, 2, 0))
                        r[f"tw{tw}_kg{ks}"] = t()
                        _native.check(lib.lowbit_set_launch_override(0, 0, 0))
            finally:
                _native.check(lib.lowbit_set_gemm_tile_waves(0))
                _native.check(lib.lowbit_set_launch_override(0, 0, 0))
            rows.append(r)
            print(json.dumps(r), flush=True)
        del cl
        torch.cuda.empty_cache()
    if a.out:
        pathlib.Path(a.out).write_text(json.dumps(rows, indent=1))


def sweep_splits(a):
    """MFMA GEMM (v5) on the 1.5B / 3B / 7B decode projections, M in {2, 16, 32, 48, 64}: graph-timed us per call of
    the automatic plan, of one tile per workgroup (lowbit_set_gemm_kernel(2)) and of the row groups
    (lowbit_set_gemm_kernel(1)) with every K split S in {1, 2, 4, 8, 16} x K-groups ks in {1, 2, 4} forced through
    lowbit_set_launch_override(4 ks, 0, S), the rest automatic."""
    import torch
    from lowbit import _native, ops
    torch.cuda.set_device(0)
    lib = _native.lib()
    rows = []
    for k, n in ((1536, 2048), (1536, 1536), (2048, 2560), (2048, 2048), (3584, 3584), (3584, 512), (2048, 256),
                 (1536, 256), (3584, 4608), (8960, 1536), (11008, 2048), (18944, 3584)):
        cl = cloned_copies(torch, ops, k, n, gib=0.5)
        for m in (2, 16, 32, 48, 64):
            x = torch.randn(m, k, device="cuda").half()
            t = lambda: round(graph_time_us(torch, lambda i: ops.gemv(x, cl[i % len(cl)], 5), max(200, len(cl))), 2)
            r = {"K": k, "N": n, "M": m, "auto": t()}
            try:
                _native.check(lib.lowbit_set_gemm_kernel(2))
                r["tiles"] = t()
                _native.check(lib.lowbit_set_gemm_kernel(1))
                for sp in (1, 2, 4, 8, 16):
                    for ks in (1, 2, 4):
                        if sp * ks <= k // 128:
                            _native.check(lib.lowbit_set_launch_override(4 * ks, 0, sp))
                            r[f"s{sp}k{ks}"] = t()
            finally:
                _native.check(lib.lowbit_set_gemm_kernel(0))
                _native.check(lib.lowbit_set_launch_override(0, 0, 0))
            rows.append(r)
            print(json.dumps(r), flush=True)
        del cl
        torch.cuda.empty_cache()
    if a.out:
        pathlib.Path(a.out).write_text(json.dumps(rows, indent=1))


def sweep_prefill(a):
    """Prefill, M in {128, 256, 512, 2048} on the Qwen2.5-3B layer (merged q|k|v and gate|up, o, down) and the 7B MLP
    projections: us/call of dequantize + hipBLASLt, fp16 hipBLASLt, the int4 prefill GEMM (automatic launch plan), the
    v5 MFMA kernel in 64-row slices (ops.gemm_chunked, M <= 512) and linear() (auto route), each a graph cycling
    >= 1 GiB of int4 copies (fp16: >= 1 GiB of fp16 copies)."""
    import torch
    from lowbit import ops
    torch.cuda.set_device(0)
    shapes = [("3b.qkv", 2048, 2560), ("3b.o", 2048, 2048), ("3b.gate_up", 2048, 22016), ("3b.down", 11008, 2048),
              ("7b.gate_up", 3584, 18944), ("7b.down", 18944, 3584)]
    rows = []
    for name, k, n in shapes:
        projs = [(name, k, n)]
        pool, pool16, _, copies = build_pool(torch, ops, projs, fp16=True, seed=k + n)
        e = ops.ext()
        for m in (128, 256, 512, 2048):
            x = torch.randn(m, k, device="cuda").half()
            r = {"shape": name, "K": k, "N": n, "M": m, "copies": copies}
            it = max(40, copies)
            r["dequant_blas_us"] = round(graph_time_us(torch, lambda i: torch.nn.functional.linear(
                x, ops.dequant(pool[i % copies][name], "mma")), it), 2)
            r["fp16_blas_us"] = round(graph_time_us(torch, lambda i: torch.nn.functional.linear(
                x, pool16[i % copies][name]), it), 2)
            r["int4_prefill_us"] = round(graph_time_us(torch, lambda i: ops.prefill(x, pool[i % copies][name]), it), 2)
            r["v5_chunked_us"] = (round(graph_time_us(torch, lambda i: ops.gemm_chunked(x, pool[i % copies][name]), it), 2)
                                  if m <= 512 else None)
            r["linear_us"] = round(graph_time_us(torch, lambda i: ops.linear(x, pool[i % copies][name]), it), 2)
            r["linear_path"] = "prefill" if ops.prefill_path(m, pool[0][name]) else "dequant+blas"
            r["int4_prefill_tflops"] = round(2 * m * n * k / (r["int4_prefill_us"] * 1e-6) / 1e12, 1)
            r["fp16_blas_tflops"] = round(2 * m * n * k / (r["fp16_blas_us"] * 1e-6) / 1e12, 1)
            rows.append(r)
            print(json.dumps(r), flush=True)
        del pool, pool16
        torch.cuda.empty_cache()
    if a.out:
        pathlib.Path(a.out).write_text(json.dumps(rows, indent=1))


def pmc_workload(a):
    """For rocprofv3 --pmc: one elementwise copy of exactly 1 GiB (read 1 GiB, write 1 GiB: the calibration of
    FETCH_SIZE / WRITE_SIZE), then a.steps eager steps of the contract workload (14 GEMV launches each)."""
    import torch
    from lowbit import ops
    torch.cuda.set_device(0)
    src = torch.ones(2 ** 28, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    del src, dst
    projs = step_projections()
    pool, _, _, copies = build_pool(torch, ops, projs)
    gen = torch.Generator(device="cuda").manual_seed(1)
    xs = {name: torch.randn(1, k, generator=gen, device="cuda").half() for name, k, n in projs}
    for i in range(a.steps):
        layer = pool[i % copies]
        for name, k, n in projs:
            ops.linear(xs[name], layer[name])
    torch.cuda.synchronize()
    print(json.dumps({"pmc_workload": True, "steps": a.steps, "launches_per_step": len(projs),
                      "step_bytes": sum(alg_bytes(k, n) for _, k, n in projs)}), flush=True)


PMC_SKINNY_SHAPES = [("3b.gate_up", 2048, 11008), ("3b.down", 11008, 2048), ("7b.gate_up", 3584, 18944),
                     ("7b.down", 18944, 3584)]
PMC_SKINNY_M = (16, 32, 64)


def pmc_skinny_workload(a):
    """For rocprofv3 --pmc on the skinny path: one elementwise copy of exactly 1 GiB (the counters' calibration), then
    per (shape, M) in PMC_SKINNY_SHAPES x PMC_SKINNY_M one eager MFMA GEMM (v5) call on each of C cold copies of the
    weight (C covering >= 1 GiB), in that order; prints the order so a counter summary can attribute each dispatch."""
    import torch
    from lowbit import ops
    torch.cuda.set_device(0)
    src = torch.ones(2 ** 28, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    del src, dst
    order = []
    for name, k, n in PMC_SKINNY_SHAPES:
        copies = cloned_copies(torch, ops, k, n)
        for m in PMC_SKINNY_M:
            x = torch.randn(m, k, device="cuda").half()
            for c in copies:
                ops.gemv(x, c, 5)
            order.append({"shape": name, "K": k, "N": n, "M": m, "launches": len(copies),
                          "alg_bytes": alg_bytes(k, n, m), "flops": 2 * m * n * k})
        torch.cuda.synchronize()
        del copies
        torch.cuda.empty_cache()
    print(json.dumps({"pmc_skinny_workload": True, "kernel": "gemm_mfma", "order": order}), flush=True)


# BASELINE configs 4 and 5: prompt length, greedy tokens, tokens per step of the teacher-forced feeds, clip search
E2E = {"1.5b": dict(prompt=64, new=256, chunks=(1, 16, 48), feed=480, clip=False),
       "3b": dict(prompt=512, new=256, chunks=(1, 16, 48), feed=480, clip=True),
       "tiny": dict(prompt=32, new=32, chunks=(1, 16, 48), feed=96, clip=True)}


def e2e(a):
    """Random-init Qwen2.5 decoder, batch 1, every decode step one hipGraph. Two pairs of variants:
    * transformers' own modules (lowbit.decode.GraphDecoder): fp16, then the same model with W4Linear projections
      (the reference's drop-in, lowbit/model.py), plus fake-quant (dequantized weights in nn.Linear) for agreement;
    * FusedQwen2 (lowbit.fused: RMSNorm, RoPE + cache write and attention kernels, merged q|k|v and gate|up with fused
      epilogues), fp16 projections (hipBLASLt) vs W4A16 projections; everything but the projections is shared.
    Per variant: TTFT (eager prefill of the prompt: dequantize + hipBLASLt for W4), greedy decode tokens/s, tokens/s
    feeding a fixed random stream 1, 16 and 48 tokens per step (GEMV / MFMA / MFMA kernels), peak HBM. W4 variants
    are compared with fake-quant on identical inputs (teacher-forced argmax agreement, max logit difference relative
    to the logits' RMS)."""
    import torch
    from lowbit import decode, fused, model as lbmodel
    cfg = E2E[a.e2e]
    torch.cuda.set_device(0)
    m = decode.random_model(a.e2e, seed=0)
    vocab = m.config.vocab_size
    gen = torch.Generator(device="cuda").manual_seed(2024)
    prompt = torch.randint(0, vocab, (1, cfg["prompt"]), generator=gen, device="cuda")
    feed = torch.randint(0, vocab, (cfg["feed"],), generator=gen, device="cuda")
    max_len = cfg["prompt"] + max(cfg["new"], cfg["feed"]) + 64
    clip = CLIP_GRID if cfg["clip"] else None
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731

    def measure(make, label, speed=True):
        """make(chunk) -> a decoder (prefill / capture / step / greedy)."""
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        r = {"label": label}
        dec = make(1)
        ttft = []
        for _ in range(3 if speed else 1):
            e0, e1 = ev(), ev()
            e0.record()
            dec.prefill(prompt).argmax(-1)
            e1.record()
            torch.cuda.synchronize()
            ttft.append(e0.elapsed_time(e1))
        dec.capture()
        times, toks = [], None
        for _ in range(3 if speed else 1):
            first = dec.prefill(prompt).argmax(-1)
            e0, e1 = ev(), ev()
            e0.record()
            toks = dec.greedy(first, cfg["new"])
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1))
        ms = sorted(times)[len(times) // 2]
        r["ttft_ms"] = round(sorted(ttft)[len(ttft) // 2], 3)
        r["greedy"] = {"prompt_tokens": cfg["prompt"], "new_tokens": cfg["new"],
                       "tokens_per_s": round((cfg["new"] - 1) / (ms / 1000), 1),
                       "ms_per_token": round(ms / (cfg["new"] - 1), 4)}
        del dec
        logits = {}
        for c in cfg["chunks"]:
            dc = make(c)
            best = None
            for rep in range(2 if speed else 1):
                dc.prefill(prompt)
                if dc.graph is None:
                    dc.capture()
                rows = []
                e0, e1 = ev(), ev()
                e0.record()
                for i in range(0, cfg["feed"], c):
                    out = dc.step(feed[i:i + c])
                    if rep == 0:
                        rows.append(out.half().clone())
                e1.record()
                torch.cuda.synchronize()
                t = e0.elapsed_time(e1)
                best = t if best is None else min(best, t)
                if rep == 0:
                    logits[c] = torch.cat(rows)
            r[f"feed_{c}"] = {"tokens_per_step": c, "tokens": cfg["feed"],
                              "tokens_per_s": round(cfg["feed"] / (best / 1000), 1)}
            del dc
        r["peak_hbm_bytes"] = torch.cuda.max_memory_allocated()
        print(json.dumps({"e2e": a.e2e, **r}), flush=True)
        return r, toks, logits

    hf_dec = lambda model: (lambda c: decode.GraphDecoder(model, max_len, c))  # noqa: E731
    res = {"e2e": a.e2e, "model": f"random-init Qwen2.5-{a.e2e} architecture (no checkpoint), fp16",
           "clip_search": cfg["clip"], "workload": cfg}
    out, tok, lg = {}, {}, {}
    out["hf_fp16"], tok["hf_fp16"], lg["hf_fp16"] = measure(hf_dec(m), "hf_fp16")
    fq = fused.FusedQwen2(m, max_len, quant="fp16")
    out["fused_fp16"], tok["fused_fp16"], lg["fused_fp16"] = measure(lambda c: fused.FusedDecoder(fq, c), "fused_fp16")
    del fq
    fq = fused.FusedQwen2(m, max_len, quant="int4", clip_grid=clip)
    out["fused_int4"], tok["fused_int4"], lg["fused_int4"] = measure(lambda c: fused.FusedDecoder(fq, c), "fused_int4")
    del fq
    torch.cuda.empty_cache()
    layers = lbmodel.quantize_layers(m, GROUP, clip)
    lbmodel.apply_fake_quant(layers)
    out["hf_fake_quant"], tok["hf_fake_quant"], lg["hf_fake_quant"] = measure(hf_dec(m), "hf_fake_quant", speed=False)
    res["layers_replaced"], res["int4_linear_bytes"] = lbmodel.apply_int4(layers)
    out["hf_int4"], tok["hf_int4"], lg["hf_int4"] = measure(hf_dec(m), "hf_int4")

    def prefix(x, y):
        diff = (x != y).nonzero()
        return int(diff[0, 0]) if diff.numel() else int(x.numel())

    def agree(x, y):
        r = {}
        for c in cfg["chunks"]:
            f, q = lg[y][c].float(), lg[x][c].float()
            rms = f.pow(2).mean().sqrt()
            r[str(c)] = {"argmax_agreement": round(float((f.argmax(-1) == q.argmax(-1)).float().mean()), 4),
                         "max_logit_diff_rel": round(float((f - q).abs().max() / rms), 5)}
        return r

    res["agreement"] = {"hf_int4_vs_hf_fake_quant": agree("hf_int4", "hf_fake_quant"),
                        "fused_int4_vs_hf_fake_quant": agree("fused_int4", "hf_fake_quant"),
                        "fused_fp16_vs_hf_fp16": agree("fused_fp16", "hf_fp16")}
    res["greedy_common_prefix"] = {"hf_int4_vs_hf_fake_quant": prefix(tok["hf_int4"], tok["hf_fake_quant"]),
                                   "fused_int4_vs_hf_fake_quant": prefix(tok["fused_int4"], tok["hf_fake_quant"]),
                                   "fused_fp16_vs_hf_fp16": prefix(tok["fused_fp16"], tok["hf_fp16"]),
                                   "of": cfg["new"]}
    sp = lambda x, y, k: round(out[x][k]["tokens_per_s"] / out[y][k]["tokens_per_s"], 3)  # noqa: E731
    keys = ["greedy"] + [f"feed_{c}" for c in cfg["chunks"]]
    res["speedup_w4_over_fp16"] = {"transformers_modules": {k: sp("hf_int4", "hf_fp16", k) for k in keys},
                                   "fused_layer": {k: sp("fused_int4", "fused_fp16", k) for k in keys},
                                   "fused_w4_over_transformers_fp16": {k: sp("fused_int4", "hf_fp16", k) for k in keys}}
    res["ttft_ms"] = {k: v["ttft_ms"] for k, v in out.items()}
    res["variants"] = out
    print(json.dumps({k: v for k, v in res.items() if k != "variants"}), flush=True)
    if a.out:
        pathlib.Path(a.out).parent.mkdir(parents=True, exist_ok=True)
        pathlib.Path(a.out).write_text(json.dumps(res, indent=1))


def decode_trace(a):
    """Profiler workload for one e2e variant: the model, the prompt prefill, one captured step, `steps` replays."""
    import torch
    from lowbit import decode, fused, model as lbmodel
    cfg = E2E[a.e2e]
    torch.cuda.set_device(0)
    m = decode.random_model(a.e2e, seed=0)
    steps, chunk = min(a.steps, 256), a.chunk
    max_len = cfg["prompt"] + steps * chunk + 64
    clip = CLIP_GRID if cfg["clip"] else None
    if a.decode_trace.startswith("fused"):
        dec = fused.FusedDecoder(fused.FusedQwen2(m, max_len, quant=a.decode_trace.split("_")[1], clip_grid=clip),
                                 chunk)
        del m
    else:
        if a.decode_trace == "hf_int4":
            lbmodel.apply_int4(lbmodel.quantize_layers(m, GROUP, clip))
        dec = decode.GraphDecoder(m, max_len, chunk)
    torch.cuda.empty_cache()
    vocab = decode.qwen25_config(a.e2e).vocab_size
    prompt = torch.randint(0, vocab, (1, cfg["prompt"]), generator=torch.Generator(device="cuda").manual_seed(2024),
                           device="cuda")
    first = dec.prefill(prompt).argmax(-1)
    dec.capture()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if chunk == 1:
        dec.greedy(first, steps)
        tokens = steps - 1
    else:
        feed = torch.randint(0, vocab, (steps * chunk,), generator=torch.Generator(device="cuda").manual_seed(7),
                             device="cuda")
        for i in range(steps):
            dec.step(feed[i * chunk:(i + 1) * chunk])
        tokens = steps * chunk
    torch.cuda.synchronize()
    print(json.dumps({"decode_trace": a.decode_trace, "e2e": a.e2e, "steps": steps, "chunk": chunk,
                      "ms_per_token": round(1000 * (time.perf_counter() - t0) / tokens, 4)}), flush=True)


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {a.gpus}); the W4A16 path is not sharded in this build",
              file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs on one GPU only; launch it without torch.distributed.run", file=sys.stderr)
        sys.exit(2)
    if a.pmc_workload:
        pmc_workload(a)
    elif a.pmc_skinny:
        pmc_skinny_workload(a)
    elif a.per_shape_only:
        per_shape_workload(a)
    elif a.sweep == "skinny":
        sweep_skinny(a)
    elif a.sweep == "prefill":
        sweep_prefill(a)
    elif a.sweep == "gemv":
        sweep_gemv(a)
    elif a.sweep == "ldsring":
        sweep_ldsring(a)
    elif a.sweep == "order":
        sweep_order(a)
    elif a.sweep == "tiles":
        sweep_tiles(a)
    elif a.sweep == "tilewaves":
        sweep_tilewaves(a)
    elif a.sweep == "splits":
        sweep_splits(a)
    elif a.e2e and a.decode_trace:
        decode_trace(a)
    elif a.e2e:
        e2e(a)
    elif a.host_cost:
        host_cost(a)
    elif a.trace_child:
        a.no_cpu = a.no_fp16 = a.no_detail = True
        a.trace = None
        contract(a)
    else:
        # the traced run first, while this process has not touched the GPU
        a.trace = None if a.no_trace else traced_gemv(a)
        progress("traced run " + ("done" if a.trace else "unavailable: roofline from graph time"))
        contract(a)


if __name__ == "__main__":
    main()
