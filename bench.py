"""Benchmark of the quantized linear hot path on one MI355X.

Headline: AQ4 g128 matvec, M=1, K=4096, N=14336,
bf16 activations, fp32 accumulation, in GB/s of algorithmic HBM traffic
(N*K/2 + 4*N*K/128 + 2*M*K + 2*M*N bytes per launch).

One "step" is one sweep of forward calls over R rotated weight copies
(R chosen so the copies total more than 1 GB, defeating the 256 MB Infinity
Cache), captured once into a HIP graph and replayed, so that the timed region
holds back-to-back kernels with inputs already resident in HBM.  The kernel's
average duration is timed with HIP events on the stream the kernels run on.

Extra configurations (FP8 matvec, the FP8 small-M sweep M = 1..32 over the
four Llama-3-8B layer shapes, a plain streaming-read floor at the headline
sizes, the M=2048 FP8 GEMM and the 32-layer AQ4 decode stack; "gemm_shapes"
adds the other prefill projections, short prompts (M = 256, 512) and M < 128, "vendor_gemm" the same FP8
GEMMs through hipBLASLt for reference, "floor_sweep" every read shape of the
read-floor kernel at the headline's bytes) are reported under "configs".  The CPU
baseline is this build's own C restatement (oracle/), not a reference CPU
path: the reference has none.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs a,b]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "ullm-project_amd"))

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5030.0  # dense, 256 CU x 2.4 GHz x 8192 flop/clk/CU
ROTATE_BYTES = 1 << 30


def fp8_bytes(m, n, k):
    return n * k + 4 * n + 2 * m * k + 2 * m * n


def aq4_bytes(m, n, k):
    return n * k // 2 + 4 * n * k // 128 + 2 * m * k + 2 * m * n


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Runner:
    """Creates rotated weight copies and times graph replays of forwards."""

    def __init__(self, uh, torch, device):
        self.uh = uh
        self.torch = torch
        self.dev = device
        self.stream = torch.cuda.Stream(device=device)

    def weights(self, encoding, n, k, copies, seed=0):
        torch = self.torch
        g = torch.Generator(device=self.dev)
        out = []
        for i in range(copies):
            g.manual_seed(seed * 1000 + i)
            w = torch.randn((n, k), generator=g, device=self.dev,
                            dtype=torch.float32) * 0.02
            out.append(self.uh.LinearWeight.quantize(w, encoding))
            del w
        torch.cuda.synchronize()
        return out

    def time_sweep(self, calls, steps, warmup):
        """calls: list of zero-arg callables issuing one forward each on the
        current stream.  Returns (ms per step, us per call, timing mode)."""
        torch = self.torch
        mode = "graph"
        with torch.cuda.stream(self.stream):
            for c in calls:  # first touch outside capture
                c()
            self.stream.synchronize()
            graph = None
            try:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=self.stream):
                    for c in calls:
                        c()
            except Exception as exc:  # capture unsupported: eager launches
                log(f"graph capture failed ({exc}); timing eager launches")
                graph = None
                mode = "eager"
                torch.cuda.synchronize()

            def step():
                if graph is not None:
                    graph.replay()
                else:
                    for c in calls:
                        c()

            for _ in range(warmup):
                step()
            self.stream.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record(self.stream)
            for _ in range(steps):
                step()
            end.record(self.stream)
            end.synchronize()
        ms = start.elapsed_time(end)
        return ms / steps, 1000.0 * ms / (steps * len(calls)), mode


def bench_matvec(r, encoding, m, n, k, steps, warmup, seed=0):
    torch, uh = r.torch, r.uh
    per = aq4_bytes(m, n, k) if encoding == uh.ENCODING_AQ4_G128 else fp8_bytes(m, n, k)
    copies = max(4, -(-ROTATE_BYTES // per))
    ws = r.weights(encoding, n, k, copies, seed)
    g = torch.Generator(device=r.dev)
    g.manual_seed(seed + 7)
    x = torch.randn((m, k), generator=g, device=r.dev).to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=r.dev)
    calls = [(lambda w=w: w.forward(x, y)) for w in ws]
    ms_step, us_call, mode = r.time_sweep(calls, steps, warmup)
    gbs = per / (us_call * 1e-6) / 1e9
    for w in ws:
        w.destroy()
    return {"m": m, "n": n, "k": k, "bytes_per_launch": per, "copies": copies,
            "us_per_launch": us_call, "ms_per_step": ms_step, "GB_s": gbs,
            "frac_hbm": gbs / HBM_PEAK_GBS, "timing": mode}


def bench_gemm(r, m, n, k, steps, warmup):
    torch, uh = r.torch, r.uh
    # At least 4 weight copies totalling more than 1 GB, so each call streams
    # its weights from HBM rather than the 256 MB Infinity Cache.
    copies = max(4, -(-ROTATE_BYTES // (n * k + 4 * n)))
    ws = r.weights(uh.ENCODING_FP8_E4M3_ROW, n, k, copies, seed=3)
    g = torch.Generator(device=r.dev)
    g.manual_seed(11)
    x = torch.randn((m, k), generator=g, device=r.dev).to(torch.bfloat16)
    xq, xs = uh.quantize_activations(x)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=r.dev)
    torch.cuda.synchronize()
    calls = [(lambda w=w: w.forward(xq, y, x_scales=xs)) for w in ws]
    ms_step, us_call, mode = r.time_sweep(calls, steps, warmup)
    tflops = 2.0 * m * n * k / (us_call * 1e-6) / 1e12
    # End to end from bf16 activations: per-token quantization into the
    # caller's workspace, then the GEMM (two kernels per call).  The bf16
    # activations rotate over enough copies (> 256 MB) that each call's
    # quantization reads them from HBM, as a prefill step would.
    xcopies = max(16, -(-(256 << 20) // (2 * m * k)) + 1)
    xs_b = [torch.randn((m, k), generator=g, device=r.dev).to(torch.bfloat16)
            for _ in range(xcopies)]
    wsb = torch.empty((ws[0].workspace_size(m, mode=uh.ACT_FP8_PER_TOKEN),),
                      dtype=torch.uint8, device=r.dev)
    ncalls = max(copies, xcopies)
    calls = [(lambda w=ws[i % copies], xb=xs_b[i % xcopies]:
              w.forward(xb, y, mode=uh.ACT_FP8_PER_TOKEN, workspace=wsb))
             for i in range(ncalls)]
    _, us_e2e, _ = r.time_sweep(calls, steps, warmup)
    # The quantization alone over the same rotated activations (HBM-fed).
    xq_b = torch.empty((m, k), dtype=torch.uint8, device=r.dev)
    xs_s = torch.empty((m,), dtype=torch.float32, device=r.dev)
    calls = [(lambda xb=xb: uh.quantize_activations(xb, xq_b, xs_s, stream=r.stream))
             for xb in xs_b]
    _, us_quant, _ = r.time_sweep(calls, steps, warmup)
    del xs_b
    for w in ws:
        w.destroy()
    return {"m": m, "n": n, "k": k, "copies": copies, "us_per_launch": us_call,
            "TFLOPS": tflops, "frac_fp8_peak": tflops / FP8_PEAK_TFLOPS,
            "us_with_act_quant": us_e2e, "act_copies": xcopies,
            "us_act_quant_alone": us_quant,
            "TFLOPS_with_act_quant": 2.0 * m * n * k / (us_e2e * 1e-6) / 1e12,
            "timing": mode}


def bench_add_quant(r, m, k, steps, warmup):
    """The add that precedes a prefill projection fused into the per-token
    quantization (ullm_linear_add_quantize_activations: reads a and b once,
    writes the bf16 sum and the codes) against the two passes it replaces
    (torch's bf16 add, then ullm_linear_quantize_activations)."""
    torch, uh = r.torch, r.uh
    copies = 8  # 8 x 3 x 16.8 MB at M=2048, K=4096: past the Infinity Cache
    g = torch.Generator(device=r.dev)
    g.manual_seed(23)
    ab = [(torch.randn((m, k), generator=g, device=r.dev).to(torch.bfloat16),
           torch.randn((m, k), generator=g, device=r.dev).to(torch.bfloat16),
           torch.empty((m, k), dtype=torch.bfloat16, device=r.dev)) for _ in range(copies)]
    torch.cuda.synchronize()
    fused = [(lambda t=t: uh.add_quantize_activations(t[0], t[1], t[2], stream=r.stream))
             for t in ab]
    _, us_fused, mode = r.time_sweep(fused, steps, warmup)

    def two_pass(t):
        torch.add(t[0], t[1], out=t[2])
        uh.quantize_activations(t[2], stream=r.stream)

    _, us_two, _ = r.time_sweep([(lambda t=t: two_pass(t)) for t in ab], steps, warmup)
    return {"m": m, "k": k, "us_fused": us_fused, "us_add_then_quantize": us_two,
            "bytes_fused": 4 * m * k + m * k + 4 * m, "timing": mode}


def bench_vendor_gemm(r, m, n, k, steps, warmup):
    """The same FP8 GEMM through the vendor library (hipBLASLt via
    torch._scaled_mm: E4M3 x E4M3 with per-tensor scales, bf16 out), over the
    same number of rotated weight copies: a reference point for the FP8
    matrix-core rate this part reaches on this shape.  Not a product path."""
    torch = r.torch
    copies = max(4, -(-ROTATE_BYTES // (n * k)))
    g = torch.Generator(device=r.dev)
    g.manual_seed(17)
    x = torch.randn((m, k), generator=g, device=r.dev).to(torch.float8_e4m3fn)
    ws = [(torch.randn((n, k), generator=g, device=r.dev) * 8).to(torch.float8_e4m3fn)
          for _ in range(copies)]
    one = torch.ones((), dtype=torch.float32, device=r.dev)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=r.dev)

    def call(w):
        torch._scaled_mm(x, w.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16,
                         out=y)

    calls = [(lambda w=w: call(w)) for w in ws]
    _, us_call, mode = r.time_sweep(calls, steps, warmup)
    del ws
    tflops = 2.0 * m * n * k / (us_call * 1e-6) / 1e12
    return {"m": m, "n": n, "k": k, "copies": copies, "us_per_launch": us_call,
            "TFLOPS": tflops, "frac_fp8_peak": tflops / FP8_PEAK_TFLOPS,
            "timing": mode, "library": "hipBLASLt via torch._scaled_mm"}


def bench_read_floor(r, nbytes, steps, warmup):
    """Plain streaming reads of `nbytes` per launch (libullm_bench.so's
    stream_read_kernel in three shapes of waves x loads in flight x bytes per
    wave; the fastest is reported) over rotated random buffers totalling
    more than 1 GB, timed like the matvecs: what a launch that reads that
    many bytes costs with no unpacking or arithmetic."""
    import ctypes
    torch = r.torch
    bench_lib = ctypes.CDLL(str(ROOT / "ullm-project_amd" / "lib" / "libullm_bench.so"))
    fn = bench_lib.ullm_bench_stream_read
    fn.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_void_p,
                   ctypes.c_void_p]
    fn.restype = ctypes.c_int
    nbytes = nbytes // 16 * 16
    copies = max(4, -(-ROTATE_BYTES // nbytes))
    g = torch.Generator(device=r.dev)
    g.manual_seed(99)
    bufs = [torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), generator=g,
                          device=r.dev, dtype=torch.int32) for _ in range(copies)]
    sink = torch.empty(((nbytes >> 10) + 1,), dtype=torch.int32, device=r.dev)

    def call(b, shape):
        st = fn(b.data_ptr(), nbytes, shape, sink.data_ptr(),
                torch.cuda.current_stream().cuda_stream)
        if st != 0:
            raise RuntimeError(f"stream_read launch failed: {st}")

    shapes = {0: "4 waves x 4 loads, 4 KiB/wave", 1: "4 waves x 8 loads, 8 KiB/wave",
              2: "8 waves x 8 loads, 8 KiB/wave"}
    best = None
    for shape, name in shapes.items():
        calls = [(lambda b=b, sh=shape: call(b, sh)) for b in bufs]
        ms_step, us_call, mode = r.time_sweep(calls, steps, warmup)
        if best is None or us_call < best[0]:
            best = (us_call, name, mode)
    del bufs
    us_call, name, mode = best
    gbs = nbytes / (us_call * 1e-6) / 1e9
    return {"bytes_per_launch": nbytes, "copies": copies,
            "us_per_launch": us_call, "GB_s": gbs,
            "frac_hbm": gbs / HBM_PEAK_GBS, "timing": mode,
            "kernel": f"stream_read_kernel ({name})"}


def bench_read_sweep(r, nbytes, steps, warmup):
    """Every read shape of libullm_bench.so's sweep (1-16 waves per workgroup,
    1-32 1 KiB loads in flight per wave, 1-32 KiB per wave) over rotated
    random buffers of `nbytes`: how far the floor the `floor` leg reports is
    from the fastest plain read of those bytes this harness can time; and
    torch's reductions over the same buffers for comparison."""
    import ctypes
    torch = r.torch
    bench_lib = ctypes.CDLL(str(ROOT / "ullm-project_amd" / "lib" / "libullm_bench.so"))
    fn = bench_lib.ullm_bench_stream_read_shape
    fn.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                   ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    nbytes = nbytes // 16 * 16
    copies = max(4, -(-ROTATE_BYTES // nbytes))
    g = torch.Generator(device=r.dev)
    g.manual_seed(98)
    bufs = [torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), generator=g,
                          device=r.dev, dtype=torch.int32) for _ in range(copies)]
    sink = torch.empty(((nbytes >> 10) + 1,), dtype=torch.int32, device=r.dev)

    def call(b, w, d, c):
        st = fn(b.data_ptr(), nbytes, w, d, c, sink.data_ptr(),
                torch.cuda.current_stream().cuda_stream)
        if st != 0:
            raise RuntimeError(f"stream_read_shape launch failed: {st}")

    shapes = []
    for w in (1, 2, 4, 8, 16):
        for d in (1, 2, 4, 8, 16, 32):
            for kib in (1, 2, 4, 8, 16, 32):
                if kib % d == 0:
                    calls = [(lambda b=b, w=w, d=d, c=kib * 1024: call(b, w, d, c)) for b in bufs]
                    _, us, _ = r.time_sweep(calls, steps, warmup)
                    shapes.append((us, w, d, kib))
    # The vendor's own kernels reading the same buffers: torch's reductions
    # (one pass over the bytes, a few bytes out), as an outside check on the
    # floor this harness reports.
    vendor = {}
    half = nbytes // 8  # int32 elements in half the bytes
    dst = torch.empty((half,), dtype=torch.int32, device=r.dev)
    for name, fn_v in (("torch.sum (f32 view)", lambda b: torch.sum(b.view(torch.float32))),
                       ("torch.amax (i32)", lambda b: torch.amax(b)),
                       ("copy_ of half the bytes (read + write)",
                        lambda b: dst.copy_(b[:half]))):
        calls = [(lambda b=b, f=fn_v: f(b)) for b in bufs]
        _, us, mode = r.time_sweep(calls, steps, warmup)
        vendor[name] = {"us": round(us, 3), "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "timing": mode}
    del bufs
    shapes.sort()
    return {"bytes_per_launch": nbytes, "copies": copies, "shapes": len(shapes),
            "vendor_reads": vendor,
            "best_us": shapes[0][0], "best_GB_s": nbytes / (shapes[0][0] * 1e-6) / 1e9,
            "worst_us": shapes[-1][0],
            "fastest": [{"us": round(u, 3), "waves": w, "depth": d, "kib_per_wave": k}
                        for u, w, d, k in shapes[:8]]}


def bench_stack(r, steps, warmup):
    """BASELINE config #5: 32-layer AQ4 Llama-3-8B-shaped linear stack +
    lm_head, batch 8 single-token decode; one step = 129 forward calls."""
    import stack
    st = stack.DecodeStack(r.uh, r.torch, r.dev, batch=8)
    g = r.torch.Generator(device=r.dev)
    g.manual_seed(5)
    st.h0.copy_(r.torch.randn(st.h0.shape, generator=g, device=r.dev))
    ms_step, _, mode = r.time_sweep([st.step], steps, warmup)
    logits = st.logits.float()
    finite = bool(r.torch.isfinite(logits).all())
    rms = float(logits.pow(2).mean().sqrt())
    st.destroy()
    per = stack.step_bytes()
    gbs = per / (ms_step * 1e-3) / 1e9
    return {"layers": 32, "batch": 8, "bytes_per_step": per,
            "us_per_step": ms_step * 1e3, "GB_s": gbs,
            "frac_hbm": gbs / HBM_PEAK_GBS, "tokens_per_s": 8 / (ms_step * 1e-3),
            "logits_finite": finite, "logits_rms": rms, "timing": mode}


def measured_traffic(workload):
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE + WRITE_SIZE and
    committed under profiles/ (None when no such summary exists)."""
    path = ROOT / "profiles" / f"{workload}_traffic.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# Threads the CPU leg uses: the host share of one GPU on the GPU boxes this
# runs on (16 threads per GPU), or fewer when the process may use fewer CPUs.
CPU_SHARE_THREADS = 16


def cpu_baseline(seconds=10.0):
    """The oracle's AQ4 matvec on the host cores, same shape, bounded time.
    The oracle source is compiled here with -march=native (for this host's
    CPU), OpenMP over output rows."""
    import tempfile
    import numpy as np
    from oracle import oracle as orc
    m, n, k = 1, 14336, 4096
    affinity = len(os.sched_getaffinity(0))
    threads = min(CPU_SHARE_THREADS, affinity)
    with tempfile.TemporaryDirectory() as tmp:
        orc.use_library(orc.build_native(Path(tmp)))
        rs = np.random.default_rng(0)
        w = (rs.standard_normal((n, k)) * 0.02).astype(np.float32)
        p, s, z = orc.aq4_quantize(w)
        xb = orc.bf16_from_f32(rs.standard_normal((m, k)).astype(np.float32))
        orc.aq4_gemv(xb, p, s, z, threads=threads)
        t0 = time.perf_counter()
        calls = 0
        while time.perf_counter() - t0 < seconds:
            orc.aq4_gemv(xb, p, s, z, threads=threads)
            calls += 1
        dt = (time.perf_counter() - t0) / calls
    return {"value": aq4_bytes(m, n, k) / dt / 1e9, "unit": "GB/s",
            "cores": threads, "kind": "port",
            "host_logical_cpus": os.cpu_count(), "affinity_cpus": affinity,
            "cpu_model": _cpu_model(), "build": "gcc -O3 -march=native -fopenmp",
            "sample": f"{calls} AQ4 matvecs M=1 K=4096 N=14336 "
                      f"(oracle fp32 loop, OpenMP {threads} threads: the 16-thread host "
                      f"share of one GPU, capped by the {affinity} CPUs this process "
                      f"may use; {dt * 1e3:.1f} ms each)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="aq4,fp8,sweep,floor,gemm,stack")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a plain 256 MiB torch copy (a known-size "
                         "reference kernel for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.cpu_seconds <= 0:
        args.cpu_seconds = 0.05
    if args.gpus != 1:
        print("bench.py measures one GPU only: the kernels run on one GPU "
              "(a multi-GPU deployment would shard N per GPU); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import ullm_hip as uh
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    available, _, diag = uh.backend_probe()
    if not available:
        raise SystemExit(f"HIP backend unavailable: {diag}")
    r = Runner(uh, torch, dev)
    want = set(args.configs.split(","))
    if args.calibrate_copy:
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    head = bench_matvec(r, uh.ENCODING_AQ4_G128, 1, 14336, 4096, args.steps,
                        args.warmup)
    log("aq4 M=1 K=4096 N=14336:", head)
    configs = {"aq4_m1_k4096_n14336": head}
    if "fp8" in want:
        configs["fp8_m1_k4096_n4096"] = bench_matvec(
            r, uh.ENCODING_FP8_E4M3_ROW, 1, 4096, 4096, args.steps, args.warmup)
        log("fp8:", configs["fp8_m1_k4096_n4096"])
    if "sweep" in want:
        for kk, nn, name in ((4096, 6144, "qkv"), (4096, 4096, "o"),
                             (4096, 28672, "gate_up"), (14336, 4096, "down")):
            for m in (1, 2, 4, 8, 16, 32):
                res = bench_matvec(r, uh.ENCODING_FP8_E4M3_ROW, m, nn, kk,
                                   max(10, args.steps // 5), 2)
                configs[f"fp8_sweep_{name}_m{m}"] = res
                log(name, m, res["GB_s"])
    if "floor" in want:
        for name, nbytes in (("aq4_m1_k4096_n14336", aq4_bytes(1, 14336, 4096)),
                             ("fp8_m1_k4096_n4096", fp8_bytes(1, 4096, 4096)),
                             ("fp8_m1_k14336_n4096", fp8_bytes(1, 4096, 14336)),
                             ("aq4_m8_k4096_n4096", aq4_bytes(8, 4096, 4096)),
                             ("aq4_m8_k4096_n6144", aq4_bytes(8, 6144, 4096)),
                             ("aq4_m8_k4096_n28672", aq4_bytes(8, 28672, 4096))):
            configs[f"read_floor_{name}"] = bench_read_floor(
                r, nbytes, args.steps, args.warmup)
            log("read floor", name, configs[f"read_floor_{name}"])
    if "floor_sweep" in want:
        configs["read_sweep_aq4_m1_k4096_n14336"] = bench_read_sweep(
            r, aq4_bytes(1, 14336, 4096), max(10, args.steps // 2), 2)
        log("read sweep:", configs["read_sweep_aq4_m1_k4096_n14336"])
    if "stack_proj" in want:
        # The stack's projections one at a time (AQ4, M = 8, contiguous x),
        # over rotated copies like the headline.
        for name, kk, nn in (("qkv", 4096, 6144), ("o", 4096, 4096),
                             ("gate_up", 4096, 28672), ("down", 14336, 4096),
                             ("lm_head", 4096, 128256)):
            res = bench_matvec(r, uh.ENCODING_AQ4_G128, 8, nn, kk,
                               max(10, args.steps // 5), 2)
            configs[f"aq4_stack_{name}_m8"] = res
            log("stack projection", name, res["us_per_launch"], res["GB_s"])
    if "stack" in want:
        configs["aq4_stack_32l_batch8"] = bench_stack(r, max(5, args.steps // 5), 2)
        log("stack:", configs["aq4_stack_32l_batch8"])
    if "gemm" in want:
        configs["fp8_gemm_m2048_k4096_n28672"] = bench_gemm(
            r, 2048, 28672, 4096, max(5, args.steps // 5), 3)
        log("gemm:", configs["fp8_gemm_m2048_k4096_n28672"])
    if "gemm" in want:
        configs["add_quantize_m2048_k4096"] = bench_add_quant(r, 2048, 4096, 20, 3)
        log("add + quantize:", configs["add_quantize_m2048_k4096"])
    if "vendor_gemm" in want:
        try:
            configs["vendor_fp8_gemm_m2048_k4096_n28672"] = bench_vendor_gemm(
                r, 2048, 28672, 4096, max(5, args.steps // 5), 3)
            log("vendor gemm:", configs["vendor_fp8_gemm_m2048_k4096_n28672"])
        except Exception as exc:  # the vendor path is informational only
            log(f"vendor gemm unavailable: {exc}")
    if "gemm_shapes" in want:
        # The other prefill projections, short prompts whose grids split K
        # over workgroups, and M below one 128-row block.
        for m, n, k in ((2048, 6144, 4096), (2048, 4096, 4096),
                        (2048, 4096, 14336), (256, 4096, 4096),
                        (512, 4096, 14336), (64, 4096, 4096),
                        (64, 28672, 4096), (120, 14336, 4096)):
            res = bench_gemm(r, m, n, k, max(3, args.steps // 10), 1)
            configs[f"fp8_gemm_m{m}_k{k}_n{n}"] = res
            log("gemm", m, n, k, res["us_per_launch"])
            if "vendor_gemm" in want:
                try:
                    v = bench_vendor_gemm(r, m, n, k, max(3, args.steps // 10), 1)
                    configs[f"vendor_fp8_gemm_m{m}_k{k}_n{n}"] = v
                    log("vendor gemm", m, n, k, v["us_per_launch"])
                except Exception as exc:  # informational only
                    log(f"vendor gemm {m} {n} {k} unavailable: {exc}")

    cpu = cpu_baseline(args.cpu_seconds)
    us = head["us_per_launch"]
    line = {
        "metric": "AQ4 g128 matvec HBM throughput (M=1, K=4096, N=14336)",
        "value": round(head["GB_s"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic: weights N(0,0.02) quantized on device, x ~ N(0,1) bf16",
        "config": {"workload": "aq4_matvec_m1_k4096_n14336",
                   "rotated_weight_copies": head["copies"],
                   "launches_per_step": head["copies"],
                   "timing": head["timing"]},
        "roofline": {"bound": "hbm", "achieved": round(head["GB_s"], 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["GB_s"] / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("aq4_gemv_m1_k4096_n14336"),
                     "kernel_us": round(us, 3),
                     "kernel": "aq4_gemv_ms_kernel"},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
