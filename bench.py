#!/usr/bin/env python3
"""Headline benchmark: sustained fp16 GEMM TFLOPS at 4096^3 on one MI355X.

Workload (the reference's scored configuration, results/ralph_loop_fable/src/
main.cpp:43-62 and :83-90): C = A . B, A and B fp16 4096x4096 row-major,
fp32 accumulation, fp16 C; synthetic uniform[-1,1) inputs from a fixed seed,
already resident in HBM.

Before the timed region the GEMM runs back to back, untimed, for `--settle-ms`
(default 2500 ms): under a sustained matrix-core load MI355X starts at a
reduced clock and raises it over some tens of milliseconds to its sustained,
power-limited level (about 1.6-1.7 GHz for this GEMM); the reference's 10
warm-up launches (about 1 ms here) would leave the timed launches inside that
ramp.  The settle phase is also where the clock is sampled (below): the
driver's metrics table refreshes about once per second.

Timed region: `--warmup` untimed launches, a device synchronisation, then
`--steps` launches back to back on the kernel's stream between one HIP event
pair, then a device synchronisation (all in C++, libvk_bench.so).
ms_per_step = event time / steps (the mean launch duration);
value = 2*m*n*k / ms_per_step.  The reference's
own loop (an event pair and a host sync around every launch, main.cpp:52-62)
runs afterwards (100 launches; `--no-reference-loop` skips it) and is reported
as `reference_loop`.  The two differ on MI355X: back to back, the GEMM holds
the board at its power limit and the clock drops; the idle gaps of the
synchronised loop let it recover, so its per-launch times are shorter.

Clock: the SCLK, memory clock, socket power and GFX activity are sampled
from the driver's metrics table on a host thread (libvk_bench.so,
vkb_clock_*) over the settle phase after its first 300 ms (the same call back
to back, as in the timed region; the table refreshes about once per second, so
the 10 ms timed region itself rarely holds a sample), and reported under
`clock`; `roofline.frac_clock` is the achieved rate over the peak at that
clock (CUs x FLOP per clock per CU x SCLK), beside `frac` against the spec
peak at 2.4 GHz.

Other configurations of the same GEMM: `--workload` (see WORKLOADS) or
explicit --m/--n/--k/--dtype/--dist.

Prints ONE JSON line.  Extra objects:
  roofline     -- the kernel against its bound: dense fp16 or fp32 peak (TFLOP/s),
                  or HBM bandwidth (GB/s) when the GEMM's arithmetic intensity
                  is below the ridge point; `traffic` (HBM bytes per launch) from
                  the committed rocprofv3 counter summary in profiles/, else null;
  cpu_baseline -- the harness's version 0 (libvk_v0.so: widen, blocked
                  cblas-style sgemm, narrow; the reference's v0 is OpenBLAS)
                  timed on this host's cores on a bounded sample of the
                  workload, plus `c1`: version 0 on fp32 512^3 over the
                  reference's 10 CPU rounds (main.cpp:64-77).
The timed output is checked against torch's fp32 GEMM before anything is
printed: an element beyond the accumulation bound ends the run with status 1
and no JSON line.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_F16_TFLOPS = 2516.6   # 256 CU x 4096 FLOP/clk (dense fp16 MFMA) x 2.4 GHz
PEAK_F32_TFLOPS = 157.3    # published dense fp32 figure (matrix cores and vector FMAs alike)
PEAK_HBM_GBS = 8000.0
METRIC = "sustained fp16 GEMM TFLOPS at 4096³ (100-iter avg) + % of MFMA peak"

# name -> (m, n, k, dtype, dist)
WORKLOADS = {
    "square4096": (4096, 4096, 4096, "f16", "uniform"),       # the headline
    "square4096_normal": (4096, 4096, 4096, "f16", "normal"),  # reference-parity N(0,1) inputs
    "mlp_up": (4096, 11008, 4096, "f16", "uniform"),
    "mlp_down": (4096, 4096, 11008, "f16", "uniform"),
    "square8192": (8192, 8192, 8192, "f16", "normal0.5"),
    "skinny": (16, 8192, 8192, "f16", "uniform"),
    "skinny128": (128, 8192, 8192, "f16", "uniform"),
    "f32_4096": (4096, 4096, 4096, "f32", "uniform"),
    "f32_512": (512, 512, 512, "f32", "uniform"),
}


DIST_TEXT = {"uniform": "uniform[-1,1)", "normal": "N(0,1)", "normal0.5": "N(0,0.5)"}


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--version", type=int, default=None, help="kernel version (default: the library default)")
    p.add_argument("--workload", choices=sorted(WORKLOADS), default="square4096")
    p.add_argument("--m", type=int, default=None)
    p.add_argument("--n", type=int, default=None)
    p.add_argument("--k", type=int, default=None)
    p.add_argument("--dtype", choices=["f16", "f32"], default=None)
    p.add_argument("--dist", choices=["uniform", "normal", "normal0.5"], default=None)
    p.add_argument("--out", choices=["f16", "f32"], default=None)
    p.add_argument("--seed", type=int, default=20261201)
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="CPU baseline budget (repeats of the v0 GEMM until this much time)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--settle-ms", type=float, default=2500.0,
                   help="run the GEMM back to back for this long before the warm-up (untimed): "
                        "MI355X starts a sustained matrix-core load at a reduced clock and raises "
                        "it to its sustained level over some tens of milliseconds")
    p.add_argument("--no-reference-loop", action="store_true",
                   help="skip the reference's per-launch synchronised loop after the timed region "
                        "(100 more launches of the same kernel)")
    a = p.parse_args()
    m, n, k, dt, dist = WORKLOADS[a.workload]
    a.m = a.m or m
    a.n = a.n or n
    a.k = a.k or k
    a.dtype = a.dtype or dt
    a.dist = a.dist or dist
    return a


def read_traffic(kernel_name: str, workload: str):
    """HBM bytes per launch from profiles/traffic.txt lines:
    `<kernel> <workload> fetch_bytes=<F> write_bytes=<W>` (already scaled by
    the copy-kernel calibration; see the file's header)."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("#") or not line.strip():
            continue
        parts = line.split()
        if len(parts) >= 4 and parts[0] == kernel_name and parts[1] == workload:
            kv = dict(x.split("=", 1) for x in parts[2:] if "=" in x)
            try:
                return int(float(kv["fetch_bytes"]) + float(kv["write_bytes"]))
            except (KeyError, ValueError):
                return None
    return None


def load_bench_lib():
    """libvk_bench.so: the harness timing loops (include/vk_bench.h)."""
    path = os.path.join(ROOT, "vibekernel_amd", "lib", "libvk_bench.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: run __graft_entry__.build()")
    L = ctypes.CDLL(path)
    ci, sz, vp = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p
    L.vkb_reference_loop.argtypes = [ci, ci, ci, sz, sz, sz, vp, vp, vp, vp, ci, ci,
                                     ctypes.POINTER(ctypes.c_float)]
    L.vkb_reference_loop.restype = ci
    L.vkb_back_to_back.argtypes = [ci, ci, ci, sz, sz, sz, vp, vp, vp, vp, ci,
                                   ctypes.POINTER(ctypes.c_float)]
    L.vkb_back_to_back.restype = ci
    fp = ctypes.POINTER(ctypes.c_float)
    L.vkb_stream_loop.argtypes = [ci, ci, ci, sz, sz, sz, vp, vp, vp, vp, ci, ci, fp]
    L.vkb_stream_loop.restype = ci
    L.vkb_clock_open.restype = ci
    L.vkb_clock_start.argtypes = [ci]
    L.vkb_clock_start.restype = ci
    L.vkb_clock_stop.argtypes = [ctypes.POINTER(ClockStats)]
    L.vkb_clock_stop.restype = ci
    L.vkb_clock_error.restype = ctypes.c_char_p
    return L


class ClockStats(ctypes.Structure):
    """vkb_clock_stats (include/vk_bench.h)."""
    _fields_ = [("samples", ctypes.c_int), ("window_ms", ctypes.c_double), ("gfx_mhz_mean", ctypes.c_double),
                ("gfx_mhz_min", ctypes.c_double), ("gfx_mhz_max", ctypes.c_double),
                ("uclk_mhz_mean", ctypes.c_double), ("socket_w_mean", ctypes.c_double),
                ("gfx_activity_mean", ctypes.c_double)]


class Clock:
    """Driver-metrics sampling around a region (None values when unavailable)."""

    def __init__(self, lib):
        self.lib = lib
        self.ok = lib.vkb_clock_open() == 0
        self.error = None if self.ok else lib.vkb_clock_error().decode()

    def start(self, interval_us=2000):
        return self.ok and self.lib.vkb_clock_start(interval_us) == 0

    def stop(self):
        st = ClockStats()
        if self.lib.vkb_clock_stop(ctypes.byref(st)) != 0 or st.samples == 0:
            return None
        return {"sclk_mhz": round(st.gfx_mhz_mean, 1), "sclk_mhz_min": round(st.gfx_mhz_min, 1),
                "sclk_mhz_max": round(st.gfx_mhz_max, 1), "mclk_mhz": round(st.uclk_mhz_mean, 1),
                "socket_w": round(st.socket_w_mean, 1), "gfx_busy_pct": round(st.gfx_activity_mean, 1),
                "samples": st.samples, "window_ms": round(st.window_ms, 2)}


def load_v0():
    """libvk_v0.so: the harness's version 0 (include/vk_v0.h)."""
    path = os.path.join(ROOT, "vibekernel_amd", "lib", "libvk_v0.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: run __graft_entry__.build()")
    L = ctypes.CDLL(path)
    sz, vp = ctypes.c_size_t, ctypes.c_void_p
    L.vk_v0_sgemm.argtypes = [sz, sz, sz, vp, vp, vp]
    L.vk_v0_hgemm.argtypes = [sz, sz, sz, vp, vp, vp]
    L.vk_v0_threads.restype = ctypes.c_int
    return L


def cpu_baseline(m, n, k, dtype, seed, budget_s):
    """The harness's version 0 (libvk_v0.so, the product's CPU ground truth:
    fp16 -> widen, blocked OpenMP sgemm with fma over ascending k, narrow;
    matmul_f16_v0_cblas.cpp:13-25 / matmul_f32_v0_cblas.cpp:8-12) timed on
    this host; repeats the GEMM until `budget_s` seconds have been spent (at
    least once).  Beyond 2^38 FLOP the sample is a row band of A (same n and
    k, fewer rows): the rate per FLOP of a blocked SGEMM does not depend on
    the row count once it spans many cache blocks.  Also times C1 of the
    configurations: version 0 on fp32 512^3, the reference's 10 CPU rounds
    (main.cpp:64-77)."""
    import numpy as np
    L = load_v0()
    full_m = m
    while 2.0 * m * n * k > 2.0 ** 38 and m % 2 == 0 and m > 256:
        m //= 2
    rng = np.random.default_rng(seed)
    if dtype == "f16":
        A = rng.uniform(-1, 1, (m, k)).astype(np.float16).view(np.uint16)
        B = rng.uniform(-1, 1, (k, n)).astype(np.float16).view(np.uint16)
        C = np.empty((m, n), np.uint16)
        fn = lambda: L.vk_v0_hgemm(m, n, k, A.ctypes.data, B.ctypes.data, C.ctypes.data)  # noqa: E731
    else:
        A = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        B = rng.uniform(-1, 1, (k, n)).astype(np.float32)
        C = np.empty((m, n), np.float32)
        fn = lambda: L.vk_v0_sgemm(m, n, k, A.ctypes.data, B.ctypes.data, C.ctypes.data)  # noqa: E731
    fn()  # first touch / thread pool start, untimed
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 1000:
            break
    per = el / reps
    # C1: fp32 512^3, 10 rounds, each timed (main.cpp:64-77)
    A1 = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    B1 = rng.uniform(-1, 1, (512, 512)).astype(np.float32)
    C1 = np.empty((512, 512), np.float32)
    L.vk_v0_sgemm(512, 512, 512, A1.ctypes.data, B1.ctypes.data, C1.ctypes.data)
    ms = []
    for _ in range(10):
        t = time.perf_counter()
        L.vk_v0_sgemm(512, 512, 512, A1.ctypes.data, B1.ctypes.data, C1.ctypes.data)
        ms.append((time.perf_counter() - t) * 1e3)
    c1_ms = sum(ms) / len(ms)
    cores = L.vk_v0_threads()
    return {
        "value": round(2.0 * m * n * k / per / 1e12, 4),
        "unit": "TFLOPS",
        "cores": cores,
        "kind": "port",
        "sample": (("full " if m == full_m else f"{m}-row band of the {full_m}-row ") +
                   f"{m}x{n}x{k} {dtype} GEMM through the harness's version 0 (libvk_v0.so: "
                   f"blocked OpenMP sgemm, fp32 fma accumulation), {reps} repeat(s), "
                   f"{el:.1f} s, {per * 1e3:.1f} ms per GEMM"),
        "host_threads_available": len(os.sched_getaffinity(0)),
        "c1": {"workload": "fp32 512x512x512 version 0, 10 rounds (the reference's CPU loop)",
               "mean_ms": round(c1_ms, 4), "min_ms": round(min(ms), 4),
               "tflops": round(2.0 * 512 ** 3 / (c1_ms * 1e-3) / 1e12, 4), "cores": cores},
    }


def check_output(A, B, C, out):
    """Every element of the timed output within the fp32 accumulation bound of
    torch's fp32 product (2 * 2 k u |A||B|: both sides' rounding), plus half
    an fp16 ulp of the result for fp16 output.  Returns (ok, max_abs,
    worst ratio of error to bound)."""
    import torch
    k = A.shape[1]
    ref = torch.matmul(A.float(), B.float())
    absab = torch.matmul(A.float().abs(), B.float().abs())
    bound = 4.0 * k * 2.0 ** -24 * absab
    if out == "f16":
        # half an fp16 ulp of the reference value (normal range: 2^(e-11))
        mag = ref.abs().clamp_min(2.0 ** -14)
        bound = bound + torch.exp2(torch.floor(torch.log2(mag)) - 11) * 1.0001
    err = (C.float() - ref).abs()
    ratio = float((err / bound).max())
    return bool(torch.isfinite(C.float()).all()) and ratio <= 1.0, float(err.max()), ratio


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one MI355X "
              "(the GEMM is single-GPU; multi-GPU sharding is a design note only)", file=sys.stderr)
        return 2

    import torch
    import vibekernel_amd as vk

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    vk.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    m, n, k = args.m, args.n, args.k
    dtype = args.dtype
    out = args.out or dtype
    if args.version is not None:
        version = args.version
    elif dtype == "f32":
        # The fp32 configuration is defined on the vector ALUs (a
        # register-blocked VALU SGEMM, the CUDA-core-tier analog); the
        # matrix-core fp32 kernel (version 2) is measured with --version 2.
        version = 1
    else:
        version = vk.pick_version(m, n, k, dtype, out)
    kname = vk.name(version, dtype)
    if kname is None:
        print(f"bench.py: unknown {dtype} version {version}", file=sys.stderr)
        return 1

    tdt = torch.float16 if dtype == "f16" else torch.float32
    odt = torch.float16 if out == "f16" else torch.float32
    g = torch.Generator(device=dev).manual_seed(args.seed)

    def draw(shape):
        if args.dist == "uniform":
            x = torch.rand(shape, generator=g, device=dev, dtype=torch.float32) * 2 - 1
        else:
            x = torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
            if args.dist == "normal0.5":
                x = x * 0.5
        return x.to(tdt)

    A = draw((m, k))
    B = draw((k, n))
    C = torch.empty((m, n), dtype=odt, device=dev)
    stream = torch.cuda.current_stream(dev)

    bench = load_bench_lib()
    in_code = vk.DTYPE_F16 if dtype == "f16" else vk.DTYPE_F32
    out_code = vk.DTYPE_F16 if out == "f16" else vk.DTYPE_F32
    sptr = ctypes.c_void_p(stream.cuda_stream)
    call = (version, in_code, out_code, m, n, k, ctypes.c_void_p(A.data_ptr()),
            ctypes.c_void_p(B.data_ptr()), ctypes.c_void_p(C.data_ptr()), sptr)

    clock = Clock(bench)

    # Untimed settle phase: back-to-back launches until the clock has reached
    # its sustained level (see --settle-ms); the clock is sampled after its
    # first 300 ms.
    settle_launches = 0
    settle_clock = None
    if args.settle_ms > 0:
        # Chunks of back-to-back launches (about 50 ms each, sized from the
        # previous chunk's event time) until the host clock says settle_ms
        # have passed; the sampler runs from 300 ms on.
        probe = ctypes.c_float(0.0)
        chunk, sampling = 20, False
        t0 = time.perf_counter()
        while True:
            st = bench.vkb_back_to_back(*call, chunk, ctypes.byref(probe))
            if st != 0:
                if sampling:
                    clock.stop()
                print(f"bench.py: settle phase failed with status {st}", file=sys.stderr)
                return 1
            settle_launches += chunk
            el = (time.perf_counter() - t0) * 1e3
            if el >= args.settle_ms:
                break
            if not sampling and el >= min(300.0, args.settle_ms / 2):
                sampling = clock.start()
            chunk = max(1, int(50.0 / max(probe.value / chunk, 1e-3)))
        if sampling:
            settle_clock = clock.stop()

    # Timed region (C++, on the kernel's stream): warm-up, device sync, then
    # `steps` launches back to back between one event pair, device sync.
    # Wall clock around it as a cross-check; the clock sampled throughout.
    tot = ctypes.c_float(0.0)
    torch.cuda.synchronize()
    sampling = clock.start()
    w0 = time.perf_counter()
    st = bench.vkb_stream_loop(*call, args.warmup, args.steps, ctypes.byref(tot))
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    timed_clock = clock.stop() if sampling else None
    if st != 0:
        print(f"bench.py: timed loop failed with status {st}", file=sys.stderr)
        return 1
    mean_ms = tot.value / args.steps
    flop = 2.0 * m * n * k
    tflops = flop / (mean_ms * 1e-3) / 1e12

    # The timed output against torch's fp32 GEMM, before anything is printed
    # (the parity tests hold the oracle comparison).
    ok, max_abs_vs_torch, bound_ratio = check_output(A, B, C, out)
    if not ok:
        print(f"bench.py: the timed output is wrong: max |C - fp32 reference| = {max_abs_vs_torch:.3e}, "
              f"{bound_ratio:.2f} x the accumulation bound; no result reported", file=sys.stderr)
        return 1

    # After the timed region: the reference's loop (event pair and host sync
    # around every launch, main.cpp:52-62), reported beside the value.
    ref_loop = None
    if not args.no_reference_loop:
        ref_n = 100
        ref_per = (ctypes.c_float * ref_n)()
        sampling = clock.start()
        st = bench.vkb_reference_loop(*call, 2, ref_n, ref_per)
        ref_clock = clock.stop() if sampling else None
        if st != 0:
            print(f"bench.py: reference loop failed with status {st}", file=sys.stderr)
            return 1
        ref_ms = sum(ref_per) / ref_n
        ref_loop = {"iters": ref_n, "warmup": 2, "mean_ms": round(ref_ms, 5), "min_ms": round(min(ref_per), 5),
                    "max_ms": round(max(ref_per), 5), "tflops": round(flop / (ref_ms * 1e-3) / 1e12, 2),
                    "clock": ref_clock,
                    "protocol": "event pair + host sync around each launch (main.cpp:52-62), after the timed region"}

    peak = PEAK_F16_TFLOPS if dtype == "f16" else PEAK_F32_TFLOPS
    props = torch.cuda.get_device_properties(dev)
    cus = int(props.multi_processor_count)
    # FLOP per clock per CU: dense fp16 MFMA 4096; fp32 (vector FMA or fp32
    # MFMA) 256.  The peak at the measured SCLK is what the clock allowed.
    flop_clk_cu = 4096 if dtype == "f16" else 256
    sclk_src = None
    if timed_clock and timed_clock["samples"] >= 3:
        sclk, sclk_src = timed_clock["sclk_mhz"], "timed region"
    elif settle_clock:
        sclk, sclk_src = settle_clock["sclk_mhz"], "settle phase (same call back to back, after its first 300 ms)"
    else:
        sclk = None
    peak_at_sclk = cus * flop_clk_cu * sclk * 1e6 / 1e12 if sclk else None
    workload = f"gemm_{dtype}_{m}x{n}x{k}"
    esz = 2 if dtype == "f16" else 4
    algo_bytes = (m * k + k * n) * esz + m * n * (2 if out == "f16" else 4)
    intensity = flop / algo_bytes
    if intensity < peak * 1e12 / (PEAK_HBM_GBS * 1e9):
        # below the ridge point: the bound is HBM bandwidth
        gbs = algo_bytes / (mean_ms * 1e-3) / 1e9
        roofline = {
            "bound": "hbm",
            "achieved": round(gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4),
            "traffic": read_traffic(kname, workload),
            "kernel": kname,
            "algorithmic_bytes_per_launch": algo_bytes,
        }
    else:
        roofline = {
            "bound": "valu" if "valu" in kname else "mfma",
            "achieved": round(tflops, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(tflops / peak, 4),
            "traffic": read_traffic(kname, workload),
            "kernel": kname,
            "algorithmic_flop_per_launch": flop,
            "peak_at_sclk": round(peak_at_sclk, 1) if peak_at_sclk else None,
            "frac_clock": round(tflops / peak_at_sclk, 4) if peak_at_sclk else None,
            "sclk_mhz": sclk,
        }
    headline = (m, n, k, dtype) == WORKLOADS["square4096"][:4]
    metric = METRIC if headline else (
        f"sustained {dtype} GEMM TFLOPS at {m}x{n}x{k} (mean over {args.steps} launches) "
        f"+ % of the {roofline['bound'].upper()} roofline")
    res = {
        "metric": metric,
        "value": round(tflops, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "accumulate": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"{workload} row-major NN, fp32 accumulate, {out} out, "
                    f"{DIST_TEXT[args.dist]} seed {args.seed}",
            "preset": args.workload if (m, n, k, dtype) == WORKLOADS[args.workload][:4] else "custom",
            "m": m, "n": n, "k": k,
            "version": version,
            "kernel": kname,
            "out_dtype": out,
        },
        "pct_of_peak": round(100.0 * tflops / peak, 2),
        "wall_ms_per_step": round(wall * 1e3 / (args.steps + args.warmup), 5),
        "settle": {"ms": args.settle_ms, "launches": settle_launches,
                   "note": "the timed dispatches are launches settle.launches + warmup .. + steps - 1 of the run"},
        "reference_loop": ref_loop,
        "clock": {
            "timed": timed_clock,
            "settle": settle_clock,
            "sclk_for_frac_clock": sclk_src,
            "source": "amd-smi gpu_metrics (current_gfxclks averaged over XCDs, current_uclk, "
                      "current_socket_power, average_gfx_activity) polled every 2 ms on a host thread; "
                      "the table refreshes about once per second",
            "error": clock.error,
        },
        "device": {"name": props.name, "cus": cus, "host_cores": os.cpu_count(),
                   "host_threads_available": len(os.sched_getaffinity(0))},
        "max_abs_vs_torch_f32": max_abs_vs_torch,
        "error_over_bound": round(bound_ratio, 4),
        "reference_best_a100_frac_of_peak": 0.897,
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(m, n, k, dtype, args.seed, args.cpu_seconds)
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
