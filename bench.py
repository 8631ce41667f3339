#!/usr/bin/env python3
"""Benchmark: int8 GEMM + requant at M=N=K=4096 on one MI355X.

One step = one miaie_gemm_i8_rq launch: A 4096x4096 int8 times B 4096x4096
int8, both row-major (NN), int32 accumulate, Y = sat_int8((acc + 2^9) >> 10),
over inputs already resident in HBM.  W untimed warm-up steps, then K timed
steps bracketed by a drain of the context stream on both sides, timed with
HIP events recorded on that same stream.  Prints ONE JSON line.

Also in the line (not the headline):
  extras.conv2d_3x3      int8 3x3 conv2d, N=8 56x56 Cin=Cout=64 (GOPS, roofline)
  extras.gemm_bf16_8192  bf16 8192^3 GEMM, fp32 accumulate/output (TFLOP/s)
  extras.mlp_i8          chained int8 MLP 2048x4096 -> 11008 -> 4096 (TOP/s)
  extras.gemm_i8_m_shard one GPU's 512- and 256-row share of the 4096^3 GEMM
                         sharded over M, with the tile the planner picks
  extras.mfma_ceiling    register-only MFMA rate on this GPU, constant and
                         random operands (aiehlc_amd/probes/mfma_ceiling)
  extras.gemm_in_kernel  the headline kernel's in-kernel clocks (prologue,
                         cycles per k-tile, epilogue, workgroup end spread,
                         clock per XCD; aiehlc_amd/probes/gemm_span)
  extras.launch_floor    an empty kernel with the conv's and the GEMM's grid and
                         LDS size (aiehlc_amd/probes/launch_floor): time per
                         back-to-back launch from one host thread, the host's
                         issue time per launch, and the device's time per
                         launch with the queue already filled; the conv line
                         carries the device figure as its floor and the time
                         above it; host_launch_paths: the host's time per
                         launch through each HIP launch API
  extras.reference_flow_16x16, extras.reference_flow_8x8
                         the reference's own timed example flow (aieml_mm.cc:
                         an int32 tile moved in, run, waited for, moved out)
                         through the aie-rt facade, beside the 215 us (16x16)
                         and 15 us (8x8) the reference prints for it
  extras.vendor_library  the same int8 4096^3 and bf16 8192^3 products through
                         hipBLASLt (torch._int_mm / torch.matmul) on this GPU
  cpu_baseline           the reference's CPU golden loop (i-j-k, int32
                         accumulate, B in the [N][K] layout of
                         example/matrixmultiply/aieml_mm.cc:194-230), restated
                         in oracle/miaie_oracle.c, on this host's cores

roofline.traffic (L2<->fabric bytes per launch, MALL hits included) and
roofline.frac_rocprof are read from profiles/gemm_i8_rq_4096_traffic.txt, which
records the rocprofv3 FETCH_SIZE / WRITE_SIZE and kernel-trace runs they come
from.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import re
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# MI355X published dense peaks
PEAK_INT8_TOPS = 5000.0
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_i8_rq_4096_traffic.txt")
CEILING_EXE = os.path.join(ROOT, "aiehlc_amd", "probes", "mfma_ceiling")
FLOOR_EXE = os.path.join(ROOT, "aiehlc_amd", "probes", "launch_floor")
CONV_SPAN_EXE = os.path.join(ROOT, "aiehlc_amd", "probes", "conv_span")
GEMM_SPAN_EXE = os.path.join(ROOT, "aiehlc_amd", "probes", "gemm_span")
FLOWS_EXE = os.path.join(ROOT, "aiehlc_amd", "harness", "xaie_flows")
METRIC = "int8 GEMM TOPS (% MFMA peak) at 4096^3; int8 conv2d 3x3 GOPS; vs host CPU"


class HipTimer:
    """hipEvent pair recorded on a given stream (the miaie context's stream)."""

    def __init__(self, stream: int):
        self.hip = C.CDLL("libamdhip64.so")
        self.stream = C.c_void_p(stream)
        self.e0, self.e1 = C.c_void_p(), C.c_void_p()
        for e in (self.e0, self.e1):
            self._ok(self.hip.hipEventCreate(C.byref(e)), "hipEventCreate")

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: {rc}")

    def start(self):
        self._ok(self.hip.hipEventRecord(self.e0, self.stream), "hipEventRecord")

    def stop_ms(self) -> float:
        self._ok(self.hip.hipEventRecord(self.e1, self.stream), "hipEventRecord")
        self._ok(self.hip.hipEventSynchronize(self.e1), "hipEventSynchronize")
        ms = C.c_float()
        self._ok(self.hip.hipEventElapsedTime(C.byref(ms), self.e0, self.e1), "hipEventElapsedTime")
        return float(ms.value)


def settle(ctx, fn, seconds: float) -> int:
    """Run fn back to back, untimed, for about `seconds` of wall time, so the
    GPU leaves its idle clocks and reaches the steady clock its power limit
    allows before anything is timed.  Measured on one box: after 5 warm-up
    launches the next 50 ran at 2.09-2.13 POP/s, after 500 at 2.35 POP/s.
    Returns the number of launches."""
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            fn()
        n += 20
        ctx.wait(120_000)
    return n


def timed(ctx, timer, fn, steps: int, warmup: int) -> float:
    """Average ms per call over `steps` back-to-back calls, after `warmup`."""
    for _ in range(warmup):
        fn()
    ctx.wait(120_000)
    timer.start()
    for _ in range(steps):
        fn()
    ms = timer.stop_ms()
    ctx.wait(120_000)
    return ms / steps


def single_launch_us(ctx, timer, fn, reps: int, flush=None) -> float:
    """Median over `reps` single launches, each alone between its own pair of
    events on a drained stream.  With `flush`, that call runs first (outside
    the events) so the launch starts from cold caches."""
    ts = []
    for _ in range(reps):
        if flush is not None:
            flush()
        ctx.wait(120_000)
        timer.start()
        fn()
        ts.append(timer.stop_ms() * 1e3)
    ts.sort()
    return ts[len(ts) // 2]


def read_traffic() -> dict:
    """The committed rocprofv3 summary of the headline kernel: L2<->fabric
    bytes per launch (FETCH_SIZE + WRITE_SIZE, scaled by a copy of known size;
    reads served by the MALL are counted in FETCH_SIZE too), the kernel-trace
    average duration and the bench's own event time in that profiled run."""
    out = {"bytes": None, "source": None, "rocprof_avg_kernel_us": None, "event_us": None}
    if not os.path.exists(TRAFFIC_FILE):
        return out
    text = open(TRAFFIC_FILE).read()
    out["source"] = os.path.relpath(TRAFFIC_FILE, ROOT)
    for key, pat, conv in (("bytes", r"^l2_fabric_bytes_per_launch:\s*(\d+)", int),
                           ("rocprof_avg_kernel_us", r"^rocprof_avg_kernel_us:\s*([\d.]+)", float),
                           ("event_us", r"^bench_event_us_same_run:\s*([\d.]+)", float)):
        m = re.search(pat, text, re.M)
        out[key] = conv(m.group(1)) if m else None
    return out


def cpu_baseline(seconds: float) -> dict:
    """The reference golden loop on the host over the 4096^3 problem.

    value: all of C with OpenMP over rows (threads = min(16, cores)).  Also a
    single-thread slab and the reference host's -Os build on a slab."""
    import oracle
    from aiehlc_amd import synth

    M = N = K = 4096
    threads = min(16, os.cpu_count() or 1)
    A = synth.int8((M, K), 1)
    Bt = np.ascontiguousarray(synth.int8((K, N), 2).T)  # NN -> the reference's [N][K] layout, untimed
    Cb = np.zeros((M, N), dtype=np.int32)

    def run(lib, rows, nt):
        t0 = time.perf_counter()
        lib.oracle_gemm_i8_nt_rows(A.ctypes.data, Bt.ctypes.data, Cb.ctypes.data, M, N, K, K, K, N, 0, rows, nt)
        return time.perf_counter() - t0

    lib = oracle._lib()
    # size the multi-threaded sample to about `seconds` of wall time (capped at all of C)
    probe = max(threads, 64)
    t = run(lib, probe, threads)
    rows = int(min(M, max(probe, probe * seconds / max(t, 1e-3))))
    rows -= rows % threads
    rows = max(rows, threads)
    t = run(lib, rows, threads)
    tops = 2.0 * rows * N * K / t / 1e12
    t1 = run(lib, 16, 1)
    tops1 = 2.0 * 16 * N * K / t1 / 1e12
    t_os = run(oracle._lib("liboracle_os.so"), 16, 1)
    tops_os = 2.0 * 16 * N * K / t_os / 1e12
    others = other_cpu_goldens(threads)
    return {
        "value": round(tops, 6),
        "unit": "TOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"rows 0..{rows} of C (of 4096) of the 4096^3 int8 GEMM: the reference's i-j-k int32 golden "
                  f"loop (aieml_mm.cc:194-230) on int8 operands, B transposed to [N][K] untimed, gcc -O2 "
                  f"-fopenmp over rows, {threads} threads, {t:.2f} s wall ({t * threads:.1f} thread-s); no requant",
        "single_thread_value": round(tops1, 6),
        "single_thread_sample": f"rows 0..16, 1 thread, gcc -O2, {t1:.2f} s",
        "single_thread_Os_value": round(tops_os, 6),
        "single_thread_Os_sample": f"rows 0..16, 1 thread, gcc -Os (the reference host's flag, script/aiehlc.sh:343), "
                                   f"{t_os:.2f} s",
        "host_cpu": host_cpu(),
        "other_configs": others,
    }


def host_cpu() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return f"{line.split(':', 1)[1].strip()} ({os.cpu_count()} logical CPUs visible)"
    except OSError:
        pass
    return f"unknown ({os.cpu_count()} logical CPUs visible)"


def other_cpu_goldens(threads: int) -> dict:
    """The oracle's golden loops on the other configs (same seeded inputs as
    the GPU side): config 1 (64^3, one thread), the conv in full, and
    256-row slabs of the MLP and of the bf16 GEMM, extrapolated to the whole
    output by row count (stated)."""
    import oracle
    from aiehlc_amd import synth

    out = {}
    A, B = synth.int8((64, 64), 1), synth.int8((64, 64), 2)
    t0 = time.perf_counter()
    for _ in range(100):
        oracle.gemm_i8(A, B, nthreads=1)
    t = (time.perf_counter() - t0) / 100
    out["config1_gemm_64"] = {"seconds": round(t, 7), "gops": round(2.0 * 64**3 / t / 1e9, 3), "threads": 1}
    X, W = synth.int8((8, 56, 56, 64), 3), synth.int8((64, 3, 3, 64), 4)
    sh = synth.shifts(64, 7)
    t0 = time.perf_counter()
    oracle.conv2d_nhwc_i8(X, W, sh, nthreads=threads)
    t = time.perf_counter() - t0
    out["config4_conv2d"] = {"seconds": round(t, 4), "gops": round(2.0 * 8 * 56 * 56 * 64 * 64 * 9 / t / 1e9, 2),
                             "threads": threads, "sample": "the whole output, direct 7-loop nest"}
    # the generators are counter-based, so the first 256 rows of X (and of
    # the bf16 A below) are generated alone
    Xm, W1, W2 = synth.int8((256, 4096), 3), synth.int8((4096, 11008), 5), synth.int8((11008, 4096), 6)
    t0 = time.perf_counter()
    oracle.mlp_i8(Xm, W1, W2, 11, 12, rows=(0, 256), nthreads=threads)
    t = time.perf_counter() - t0
    out["config5_mlp"] = {"seconds_extrapolated": round(t * 2048 / 256, 3),
                          "tops": round(2.0 * 2 * 256 * 4096 * 11008 / t / 1e12, 5), "threads": threads,
                          "sample": f"rows 0..256 of 2048 in {t:.2f} s, extrapolated x8"}
    del Xm, W1, W2
    Ab = synth.bf16_normal((256, 8192), 1, 1.0 / np.sqrt(8192))
    Bb = synth.bf16_normal((8192, 8192), 2, 1.0 / np.sqrt(8192))
    t0 = time.perf_counter()
    oracle.gemm_bf16(Ab, Bb, rows=(0, 256), nthreads=threads)
    t = time.perf_counter() - t0
    out["config3_gemm_bf16"] = {"seconds_extrapolated": round(t * 8192 / 256, 3),
                                "tflops": round(2.0 * 256 * 8192 * 8192 / t / 1e12, 5), "threads": threads,
                                "sample": f"rows 0..256 of 8192 (fp32 accumulate) in {t:.2f} s, extrapolated x32"}
    return out


def probe_json(exe: str) -> dict | None:
    """Run one of the standalone probes (aiehlc_amd/probes) and parse its JSON."""
    if not os.path.exists(exe):
        return None
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    if r.returncode != 0:
        return {"error": r.stderr.strip()[-300:]}
    return json.loads(r.stdout)


def cpp_conv_loop(reps: int, streams: int = 1) -> tuple[float, float | None] | None:
    """Config-4 conv from the C++ harness.  streams == 1: (us per call back to
    back on one stream, the host's issue time per call).  streams > 1:
    independent calls dealt round-robin over that many streams (each
    stream's output checked against the first's), (us per call issued from
    one host thread, us per call with one issuing thread per stream)."""
    exe = os.path.join(ROOT, "aiehlc_amd", "harness", "miaie_examples")
    if not os.path.exists(exe):
        return None
    r = subprocess.run([exe, "conv", str(reps), str(streams)], capture_output=True, text=True, timeout=120)
    if streams == 1:
        m = re.search(r"back-to-back: ([0-9.]+) us per call", r.stdout)
        mi = re.search(r"back-to-back: [0-9.]+ us per call over \d+ calls \(host issue ([0-9.]+) us per call\)",
                       r.stdout)
    else:
        m = re.search(r"on \d+ streams: ([0-9.]+) us per call", r.stdout)
        mi = re.search(r"on \d+ streams from \d+ threads: ([0-9.]+) us per call", r.stdout)
    if r.returncode != 0 or not m:
        return None
    return float(m.group(1)), (float(mi.group(1)) if mi else None)


def mfma_ceiling() -> dict | None:
    return probe_json(CEILING_EXE)


def reference_flow(sub: str = "mm", n: int = 16, expected_us: float = 215.0, reps: int = 500) -> dict | None:
    """The reference's own timed example: aieml_mm.cc's XAie_* sequence
    (move A||B into the tile, run, wait for done, move C out, MemSyncForCPU;
    the span its stopwatch covers, :148-190) for an n x n int32 NT tile,
    through the aie-rt facade on this GPU.  The reference prints that this
    span "should be 15us(8*8) 215 us(16*16)" on its AIE-ML board
    (aieml_mm.cc:257)."""
    if not os.path.exists(FLOWS_EXE):
        return None
    r = subprocess.run([FLOWS_EXE, sub, str(reps)], capture_output=True, text=True, timeout=120)
    m = re.search(r"median over (\d+) runs: ([0-9.]+) us \(min ([0-9.]+) us\)", r.stdout)
    first = re.search(r"Output took ([0-9.]+) us", r.stdout)
    if r.returncode != 0 or not m:
        return {"error": (r.stdout + r.stderr).strip()[-300:]}
    med = float(m.group(2))
    return {"flow": f"aieml_mm.cc {n}x{n} int32 NT: XAie_MoveData in, XAie_Run, XAie_CoreWaitForDone, XAie_MoveData out, "
                    f"XAie_MemSyncForCPU (aiehlc_amd/harness/xaie_flows {sub})",
            "median_us": med, "min_us": float(m.group(3)), "first_us": float(first.group(1)) if first else None,
            "runs": int(m.group(1)),
            "reference_expected_us": expected_us,
            "reference_expected_source": "aieml_mm.cc:257 (printed expectation on VEK280 AIE-ML with caches on)",
            "speedup_vs_reference_expected": round(expected_us / med, 2)}


def vendor_library(steps: int) -> dict:
    """The same GEMMs through ROCm's libraries (hipBLASLt behind torch), on
    the same GPU in the same process: the bar a tuned vendor kernel sets
    under the same clocks.  Timed with torch's events on torch's stream."""
    try:
        import torch
    except Exception as ex:  # torch is plumbing here; report and carry on
        return {"error": repr(ex)[:200]}
    dev = torch.device("cuda:0")

    def t_ms(fn, n):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    out = {"library": "torch " + torch.__version__ + " (hipBLASLt)"}
    try:
        M = 4096
        g = torch.Generator(device=dev)
        g.manual_seed(5)
        A = torch.randint(-128, 128, (M, M), dtype=torch.int8, device=dev, generator=g)
        B = torch.randint(-128, 128, (M, M), dtype=torch.int8, device=dev, generator=g)
        Bc = B.t().contiguous().t()  # same matrix, column-major storage
        for name, b in (("int8_4096_rowmajor_B", B), ("int8_4096_colmajor_B", Bc)):
            ms = t_ms(lambda: torch._int_mm(A, b), steps)
            out[name] = {"op": "torch._int_mm (int32 out)", "tops": round(2.0 * M ** 3 / (ms * 1e-3) / 1e12, 1)}
        del A, B, Bc
        Mb = 8192
        a = torch.randn(Mb, Mb, device=dev, generator=g).to(torch.bfloat16)
        b = torch.randn(Mb, Mb, device=dev, generator=g).to(torch.bfloat16)
        ms = t_ms(lambda: torch.matmul(a, b), max(20, steps // 10))
        out["bf16_8192"] = {"op": "torch.matmul (bf16 out)", "tflops": round(2.0 * Mb ** 3 / (ms * 1e-3) / 1e12, 1)}
        del a, b
        torch.cuda.empty_cache()
    except Exception as ex:
        out["error"] = repr(ex)[:300]
    return out


def extra_conv(ctx, timer, args) -> dict:
    """Config 4: int8 conv2d 3x3, N=8 56x56 Cin=Cout=64."""
    import aiehlc_amd as mi

    Nb, H, W, Ci, Co = 8, 56, 56, 64, 64
    dX, dW, dS, dYc = (ctx.empty((Nb, H, W, Ci), np.int8), ctx.empty((Co, 3, 3, Ci), np.int8),
                       ctx.upload(mi.synth.shifts(Co, 7)), ctx.empty((Nb, H, W, Co), np.int8))
    ctx.fill_i8(dX, Nb * H * W * Ci, 3)
    ctx.fill_i8(dW, Co * 9 * Ci, 4)
    conv1 = lambda: ctx.conv2d_i8_nhwc(dX, dW, dS, dYc, Nb, H, W, Ci, Co, 3, 3, 1, 1)
    ms_c = timed(ctx, timer, conv1, max(args.steps, 200), args.warmup)
    # single launches, hot and cold: "cold" writes 512 MiB first (twice the
    # 256 MB MALL; the L2s start every kernel invalidated anyway), so the
    # convolution reads X and W from HBM
    flush_bytes = 512 << 20
    dF = ctx.alloc(flush_bytes)
    us_hot1 = single_launch_us(ctx, timer, conv1, 50)
    us_cold1 = single_launch_us(ctx, timer, conv1, 50, lambda: ctx.fill_i8(dF, flush_bytes, 11))
    dF.free()
    # the same convolution recorded 20 times into one graph (miaie_graph_*):
    # replays have no host launch gap between the convolutions
    chain = 20
    with ctx.record() as g:
        for _ in range(chain):
            conv1()
    ms_cg = timed(ctx, timer, g.launch, max(10, args.steps // 5), 2) / chain
    g.destroy()
    for b in (dX, dW, dS, dYc):
        b.free()
    conv_ops = 2.0 * Nb * H * W * Co * Ci * 9
    conv_bytes = Nb * H * W * Ci + Co * 9 * Ci + Co + Nb * H * W * Co
    roof = min(PEAK_INT8_TOPS, conv_ops / conv_bytes * PEAK_HBM_GBS / 1e3)
    # the same convolution called back to back through the C ABI from the C++
    # harness (the Python loop above adds a ctypes call per launch, which can
    # be slower than the device)
    cpp = cpp_conv_loop(3000)
    # independent convolutions on two and three streams: one stream's launch
    # work overlaps the others' (throughput of a server with that many
    # requests in flight)
    cpp2 = cpp_conv_loop(3000, 2)
    cpp3 = cpp_conv_loop(3000, 3)
    # the kernel's own execution time from in-kernel clocks (the same kernel
    # template, instantiated with clock records, in its own process)
    span = probe_json(CONV_SPAN_EXE)
    issue_c = None
    if cpp is not None:
        (us_c, issue_c), step_from = cpp, ("C++ harness, 3000 back-to-back miaie_conv2d_i8_nhwc calls "
                                           "(aiehlc_amd/harness/miaie_examples conv 3000)")
    else:
        us_c, step_from = ms_c * 1e3, "Python loop over the ctypes binding, HIP events"

    if isinstance(span, dict) and "span_us" in span:
        s_us = span["span_us"]
        span["alg_GBps"] = round(conv_bytes / (s_us * 1e-6) / 1e9, 1)
        span["frac"] = round(conv_ops / (s_us * 1e-6) / 1e12 / roof, 4)
        if span.get("device_us"):
            span["device_frac"] = round(conv_ops / (span["device_us"] * 1e-6) / 1e12 / roof, 4)
    return {
        "config": "N=8 H=W=56 Cin=Cout=64 3x3 stride 1 pad 1, NHWC x OHWI, per-channel shift in [8,12]",
        "kernel": "conv2d_i8_rows<3,3,64,4,32> (4 output rows x 32 channels per workgroup, image-per-XCD grid)",
        "us_per_step": round(us_c, 3),
        "us_per_step_from": step_from,
        "gops": round(conv_ops / (us_c * 1e-6) / 1e9, 1),
        "alg_GBps": round(conv_bytes / (us_c * 1e-6) / 1e9, 1),
        "roofline": {"bound": "hbm", "achieved": round(conv_bytes / (us_c * 1e-6) / 1e9, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "alg_bytes": conv_bytes,
                     "roof_tops": round(roof, 1),
                     "frac": round(conv_ops / (us_c * 1e-6) / 1e12 / roof, 4)},
        "host_issue_us_per_call": issue_c,
        "python_loop_us_per_step": round(ms_c * 1e3, 3),
        "independent_batches": {
            f"{n}_streams": {
                "us_per_conv": round(c[1], 3), "gops": round(conv_ops / (c[1] * 1e-6) / 1e9, 1),
                "frac": round(conv_ops / (c[1] * 1e-6) / 1e12 / roof, 4),
                "us_per_conv_one_issuing_thread": round(c[0], 3)}
            for n, c in ((2, cpp2), (3, cpp3)) if c is not None and c[1] is not None},
        "independent_batches_how": "3000 independent convolutions (one batch of 8 images each) dealt round-robin "
                                   "over 2 or 3 contexts with a stream each, each stream's calls issued by its own "
                                   "host thread (aiehlc_amd/harness/miaie_examples conv 3000 N); every stream's "
                                   "output is checked against the first's; a throughput figure for a server with N "
                                   "requests in flight, not the time of one call (us_per_step)",
        "graph_chain": {"convs_per_replay": chain, "us_per_conv": round(ms_cg * 1e3, 3),
                        "gops": round(conv_ops / (ms_cg * 1e-3) / 1e9, 1),
                        "frac": round(conv_ops / (ms_cg * 1e-3) / 1e12 / roof, 4)},
        "single_launch_us": {"hot": round(us_hot1, 3), "cold_hbm": round(us_cold1, 3),
                             "how": "median of 50 launches, each alone between two events on a drained stream; "
                                    "cold_hbm writes 512 MiB before each launch (outside the events)"},
        "in_kernel": span,
        "note": "us_per_step is the host's clock around back-to-back calls and the drain after them, so it "
                "includes the device's work between launches (an empty kernel of the same grid: "
                "extras.launch_floor.conv2d_rows_grid.device_us) and would show a host slower than the device "
                "(host_issue_us_per_call); in_kernel.device_us is the same kernel's time per launch with the queue "
                "already filled, in_kernel.span_us the first wave's start to the last wave's end by the GPU's wall "
                "clock (aiehlc_amd/probes/conv_span); graph_chain replays 20 recorded convolutions per launch",
    }


def extra_m_shard(ctx, timer, args) -> dict:
    """One GPU's share of the 4096^3 GEMM sharded 8 and 16 ways over M: the
    planner picks 128x128 tiles so the grid still covers the CUs."""
    import aiehlc_amd as mi

    N = K = 4096
    shard = {}
    for Ms in (512, 256):
        dAs, dBs, dYs = ctx.empty((Ms, K), np.int8), ctx.empty((K, N), np.int8), ctx.empty((Ms, N), np.int8)
        ctx.fill_i8(dAs, Ms * K, 1)
        ctx.fill_i8(dBs, K * N, 2)
        ms_s = timed(ctx, timer, lambda: ctx.gemm_i8_rq(dAs, dBs, dYs, Ms, N, K, 10, False, None, mi.B_NN),
                     args.steps, args.warmup)
        sops = 2.0 * Ms * N * K
        shard[f"M{Ms}"] = {"shape": [Ms, N, K], "plan": ctx.plan_gemm_i8(Ms, N, K), "us": round(ms_s * 1e3, 2),
                           "tops": round(sops / (ms_s * 1e-3) / 1e12, 1),
                           "frac_of_peak": round(sops / (ms_s * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4)}
        for b in (dAs, dBs, dYs):
            b.free()
    return shard


def extra_ragged(ctx, timer, args) -> dict:
    """Shapes that no tile divides (M and N of 4000): the pipelined kernels
    with the last tile row and column moved back over their neighbours, int8
    (Y only, shift 10) and bf16, beside the same kernels at 4096."""
    import aiehlc_amd as mi

    out = {}
    for M, N, K in ((4000, 4000, 4096), (2000, 2000, 1024)):
        dA, dB, dY = ctx.empty((M, K), np.int8), ctx.empty((K, N), np.int8), ctx.empty((M, N), np.int8)
        ctx.fill_i8(dA, M * K, 1)
        ctx.fill_i8(dB, K * N, 2)
        fn = lambda: ctx.gemm_i8_rq(dA, dB, dY, M, N, K, 10, False, None, mi.B_NN)
        settle(ctx, fn, min(args.settle, 0.2))
        ms = timed(ctx, timer, fn, max(20, args.steps // 5), 5)
        ops = 2.0 * M * N * K
        out[f"int8_{M}x{N}x{K}"] = {"plan": ctx.plan_gemm_i8(M, N, K), "us": round(ms * 1e3, 2),
                                    "tops": round(ops / (ms * 1e-3) / 1e12, 1)}
        for b in (dA, dB, dY):
            b.free()
    M = N = 4000
    K = 4096
    dA, dB, dC = ctx.empty((M, K), np.uint16), ctx.empty((K, N), np.uint16), ctx.empty((M, N), np.float32)
    ctx.copy_h2d(dA, mi.synth.bf16_normal((M, K), 1, 1.0 / np.sqrt(K)))
    ctx.copy_h2d(dB, mi.synth.bf16_normal((K, N), 2, 1.0 / np.sqrt(K)))
    fn = lambda: ctx.gemm_bf16_f32(dA, dB, dC, M, N, K)
    settle(ctx, fn, min(args.settle, 0.2))
    ms = timed(ctx, timer, fn, 20, 5)
    out[f"bf16_{M}x{N}x{K}"] = {"kernel": "gemm_bf16_pair16", "us": round(ms * 1e3, 2),
                                "tflops": round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1)}
    for b in (dA, dB, dC):
        b.free()
    return out


def extra_conv_shapes(ctx, timer, args) -> dict:
    """int8 conv2d 3x3 (stride 1, pad 1, per-channel shifts) on CNN layer
    shapes beyond config 4, with the kernel the planner picks for each: wide
    rows, deep layers (few pixels, long k) and large layers.  Back-to-back
    calls through the Python binding (its ctypes call adds about 0.5 us per
    call on small shapes)."""
    import aiehlc_amd as mi

    out = {}
    for N, H, Ci, Co in ((8, 112, 64, 64), (8, 112, 128, 128), (8, 56, 256, 256), (8, 28, 512, 512),
                         (8, 14, 256, 256), (8, 7, 512, 512)):
        dX, dW, dS, dY = (ctx.empty((N, H, H, Ci), np.int8), ctx.empty((Co, 3, 3, Ci), np.int8),
                          ctx.empty((Co,), np.uint8), ctx.empty((N, H, H, Co), np.int8))
        ctx.fill_i8(dX, N * H * H * Ci, 3)
        ctx.fill_i8(dW, Co * 9 * Ci, 4)
        ctx.copy_h2d(dS, mi.synth.shifts(Co, 7))
        fn = lambda: ctx.conv2d_i8_nhwc(dX, dW, dS, dY, N, H, H, Ci, Co, 3, 3, 1, 1)
        settle(ctx, fn, min(args.settle, 0.1))
        ms = timed(ctx, timer, fn, 100, 10)
        ops = 2.0 * N * H * H * Co * Ci * 9
        byts = N * H * H * (Ci + Co) + Co * 9 * Ci + Co
        out[f"{N}x{H}x{H}x{Ci}->{Co}"] = {"kernel": mi.plan_conv2d_i8(N, H, H, Ci, Co), "us": round(ms * 1e3, 2),
                                          "tops": round(ops / (ms * 1e-3) / 1e12, 1),
                                          "frac_of_int8_peak": round(ops / (ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 3)}
        for b in (dX, dW, dS, dY):
            b.free()
    return out


def extra_bf16(ctx, timer, args) -> dict:
    """Config 3: bf16 8192^3, fp32 accumulate and output."""
    import aiehlc_amd as mi

    Mb = 8192
    dAb, dBb, dCb = (ctx.empty((Mb, Mb), np.uint16), ctx.empty((Mb, Mb), np.uint16),
                     ctx.empty((Mb, Mb), np.float32))
    ctx.copy_h2d(dAb, mi.synth.bf16_normal((Mb, Mb), 1, 1.0 / np.sqrt(Mb)))
    ctx.copy_h2d(dBb, mi.synth.bf16_normal((Mb, Mb), 2, 1.0 / np.sqrt(Mb)))
    bf16_step = lambda: ctx.gemm_bf16_f32(dAb, dBb, dCb, Mb, Mb, Mb)
    settle(ctx, bf16_step, args.settle)
    n_b = max(20, args.steps // 10)
    ms_b = timed(ctx, timer, bf16_step, n_b, 5)
    for b in (dAb, dBb, dCb):
        b.free()
    tf = 2.0 * Mb ** 3 / (ms_b * 1e-3) / 1e12
    return {"kernel": "gemm_bf16_pair16", "ms_per_step": round(ms_b, 4),
            "tflops": round(tf, 1), "frac_of_peak": round(tf / PEAK_BF16_TFLOPS, 4),
            "timed_launches": n_b, "warmup": 5,
            "how": f"{args.settle} s of untimed launches, 5 warm-ups, then {n_b} back-to-back "
                   "launches between two events"}


def extra_mlp(ctx, timer, args) -> dict:
    """Config 5: the chained int8 MLP 2048x4096 -> 11008 -> 4096."""
    Mm, Km, Fm, Nm = 2048, 4096, 11008, 4096
    dXm, d1, d2 = ctx.empty((Mm, Km), np.int8), ctx.empty((Km, Fm), np.int8), ctx.empty((Fm, Nm), np.int8)
    dH, dYm = ctx.empty((Mm, Fm), np.int8), ctx.empty((Mm, Nm), np.int8)
    ctx.fill_i8(dXm, Mm * Km, 3)
    ctx.fill_i8(d1, Km * Fm, 5)
    ctx.fill_i8(d2, Fm * Nm, 6)
    mlp_step = lambda: ctx.mlp_i8(dXm, d1, d2, dH, dYm, Mm, Km, Fm, Nm, 11, 12)
    # from idle clocks the first ~120 calls ran 10% slower: settle first
    settle(ctx, mlp_step, args.settle)
    n_m = max(20, args.steps // 2)
    ms_m = timed(ctx, timer, mlp_step, n_m, 5)
    for b in (dXm, d1, d2, dH, dYm):
        b.free()
    mops = 2.0 * 2 * Mm * Km * Fm
    return {"kernel": "gemm_i8_pipe16_mixed<NN, Y_HI_RELU> (32 x 8 tiles of 256x256, 22 x 8 of 256x128) + "
                      "gemm_i8_pipe16<256, 128, 4, NN, Y_HI>",
            "ms_per_step": round(ms_m, 4), "timed_calls": n_m,
            "how": f"{args.settle} s of untimed calls, 5 warm-ups, then {n_m} back-to-back calls between two events",
            "tops": round(mops / (ms_m * 1e-3) / 1e12, 1),
            "frac_of_peak": round(mops / (ms_m * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4)}


EXTRAS = {"conv": extra_conv, "m_shard": extra_m_shard, "bf16": extra_bf16, "mlp": extra_mlp, "ragged": extra_ragged,
          "conv_shapes": extra_conv_shapes}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--settle", type=float, default=0.3,
                    help="seconds of untimed launches before the warm-up steps (GPU leaves its idle clocks)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extras", action="store_true", help="headline workload only")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", choices=sorted(EXTRAS), default=None,
                    help="run one extra workload alone and print its JSON (for profiling it by itself)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run miaie_copy_d2d of MIB MiB, --steps times (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "how the GEMM, conv and MLP would shard over several GPUs is described, not run", file=sys.stderr)
        return 2

    import aiehlc_amd as mi

    ctx = mi.Context(0)
    timer = HipTimer(ctx.stream)
    if args.calibrate_copy:
        nb = args.calibrate_copy << 20
        src, dst = ctx.alloc(nb), ctx.alloc(nb)
        ctx.fill_i8(src, nb, 9)
        ms = timed(ctx, timer, lambda: ctx.copy_d2d(dst, src, nb), args.steps, args.warmup)
        print(json.dumps({"calibrate_copy_bytes": nb, "ms_per_copy": round(ms, 5),
                          "GBps_read_plus_write": round(2 * nb / (ms * 1e-3) / 1e9, 1)}), flush=True)
        ctx.close()
        return 0

    if args.only:
        print(json.dumps({"only": args.only, args.only: EXTRAS[args.only](ctx, timer, args)}), flush=True)
        ctx.close()
        return 0

    # ---- headline: int8 GEMM + requant, 4096^3 NN, shift 10
    M = N = K = 4096
    dA, dB, dY = ctx.empty((M, K), np.int8), ctx.empty((K, N), np.int8), ctx.empty((M, N), np.int8)
    ctx.fill_i8(dA, M * K, 1)
    ctx.fill_i8(dB, K * N, 2)
    ctx.wait(60_000)
    def step():
        ctx.gemm_i8_rq(dA, dB, dY, M, N, K, 10, False, None, mi.B_NN)

    settled = settle(ctx, step, args.settle)
    ms = timed(ctx, timer, step, args.steps, args.warmup)
    ops = 2.0 * M * N * K
    tops = ops / (ms * 1e-3) / 1e12
    for b in (dA, dB, dY):
        b.free()
    prof = read_traffic()

    extras = {}
    if not args.no_extras:
        extras["conv2d_3x3"] = extra_conv(ctx, timer, args)
        extras["gemm_i8_m_shard"] = extra_m_shard(ctx, timer, args)
        extras["gemm_bf16_8192"] = extra_bf16(ctx, timer, args)
        extras["mlp_i8"] = extra_mlp(ctx, timer, args)
        extras["gemm_ragged"] = extra_ragged(ctx, timer, args)
        extras["conv2d_other_shapes"] = extra_conv_shapes(ctx, timer, args)
    ctx.close()
    if not args.no_extras:
        extras["mfma_ceiling"] = mfma_ceiling()
        # the headline kernel's in-kernel clocks: prologue / k-tile / epilogue
        # cycles, workgroup start and end spread, per-XCD clock
        # (aiehlc_amd/probes/gemm_span, the same kernel template with clock records)
        extras["gemm_in_kernel"] = probe_json(GEMM_SPAN_EXE)
        extras["reference_flow_16x16"] = reference_flow()
        extras["reference_flow_8x8"] = reference_flow("mm8", 8, 15.0)
        floor = probe_json(FLOOR_EXE)
        extras["launch_floor"] = floor
        conv = extras.get("conv2d_3x3")
        cf = (floor or {}).get("conv2d_rows_grid")
        if conv and isinstance(cf, dict) and "device_us" in cf:
            # the same grid and LDS with an empty kernel body, in its own
            # process: the device's time per launch with the queue filled,
            # and the host's time to issue one launch
            conv["launch_floor_us"] = cf["device_us"]
            conv["launch_host_issue_us"] = cf["host_issue_us"]
            conv["us_above_floor"] = round(conv["us_per_step"] - cf["device_us"], 3)
        extras["vendor_library"] = vendor_library(args.steps)

    roofline = {
        "bound": "mfma",
        "kernel": "gemm_i8_pipe16<256, 256, 4, NN, Y_HI> (rocprof: miaie::gemm::gemm_i8_pipe16<256, 256, 4, false, 2, false, false, false>)",
        "achieved": round(tops, 2),
        "peak": PEAK_INT8_TOPS,
        "unit": "TOP/s",
        "frac": round(tops / PEAK_INT8_TOPS, 4),
        # L2<->fabric bytes per launch (FETCH_SIZE + WRITE_SIZE; MALL hits
        # are counted), from the committed profile
        "traffic": prof["bytes"],
        "traffic_source": prof["source"],
        # the same fraction from the committed rocprofv3 kernel-trace average,
        # and the bench's own event time per launch in that profiled run (the
        # box differs from this one: boxes of the pool spread by about 10%)
        "frac_rocprof": (round(ops / (prof["rocprof_avg_kernel_us"] * 1e-6) / 1e12 / PEAK_INT8_TOPS, 4)
                         if prof["rocprof_avg_kernel_us"] else None),
        "rocprof_avg_kernel_us": prof["rocprof_avg_kernel_us"],
        "profiled_run_event_us": prof["event_us"],
        "alg_ops_per_launch": ops,
        "alg_bytes_per_launch": M * K + K * N + M * N,
    }
    ceil = extras.get("mfma_ceiling") or {}
    # against the register-only rate of the instruction the kernel issues
    if isinstance(ceil.get("i8_16x16x64_random"), dict):
        roofline["frac_of_measured_random_operand_ceiling"] = round(tops / ceil["i8_16x16x64_random"]["tops"], 4)
    line = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (SplitMix64-seeded int8, generated on the device)",
        "settle": {"seconds": args.settle, "untimed_launches": settled,
                   "why": "the GPU starts at idle clocks; these launches (before the warm-up steps) bring it to the "
                          "steady clock its 1400 W power limit allows"},
        "config": {"workload": "int8 GEMM + requant, M=N=K=4096, A and B row-major (NN), int32 accumulate, "
                               "Y = sat_int8((acc + 2^9) >> 10)", "M": M, "N": N, "K": K, "shift": 10},
        "roofline": roofline,
        "extras": extras,
        "cpu_baseline": None if args.no_cpu else cpu_baseline(args.cpu_seconds),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
