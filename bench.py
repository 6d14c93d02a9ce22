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
as `reference_loop`.  Its per-launch times are longer on MI355X (measured:
104.9 us against 93.3 back to back at 4096^3): each holds the host round trip
of its event synchronisation, which the back-to-back region hides.

Clock: the SCLK, memory clock, socket power and GFX activity are sampled
from the driver's metrics table on a host thread (libvk_bench.so,
vkb_clock_*) from 300 ms into the settle phase until the timed region ends.
The table refreshes about once per second, so the settle phase ends on a
refresh: after --settle-ms the same launches continue in ~4 ms chunks until
the sampler sees a new table, and the timed region starts at once.  Every
sample is reported under `clock.samples` with its age (host time of the read
that saw it minus the timed region's start); `roofline.frac_clock` is the
achieved rate over the peak at the SCLK of the sample nearest the timed
region's start (CUs x FLOP per clock per CU x SCLK), beside `frac` against
the spec peak at 2.4 GHz.

Library ceiling (after the timed region, the output check and the reference
loop; `--no-library-ceiling` skips it; never part of any product path): the
same product on the same A and B through torch.matmul (fp32 accumulation;
for fp32 inputs with TF32 off) under the same protocol -- a settle phase of the same length
ending on a metrics refresh, `--warmup` launches, a device synchronisation,
`--steps` launches back to back between one event pair -- once per BLAS
backend torch offers on ROCm (hipBLASLt, rocBLAS, Composable Kernel), reported as
`library_ceiling` with each backend's ms_per_step, SCLK and frac_clock, and
its output checked against the same bound.  It says how far the chip lets a
vendor library go at this shape under the same clock conditions.

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
import math
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
    p.add_argument("--no-library-ceiling", action="store_true",
                   help="skip timing torch.matmul (hipBLASLt, rocBLAS, CK) under the same protocol afterwards")
    p.add_argument("--library-tune", action="store_true",
                   help="let torch's TunableOp pick the fastest library solution for the shape before "
                        "the library ceiling is timed (tuning takes some seconds)")
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
    L.vkb_clock_samples.argtypes = [ctypes.POINTER(ClockSample), ci]
    L.vkb_clock_samples.restype = ci
    L.vkb_clock_now_ms.restype = ctypes.c_double
    return L


class ClockSample(ctypes.Structure):
    """vkb_clock_sample (include/vk_bench.h)."""
    _fields_ = [("t_ms", ctypes.c_double), ("gfx_mhz", ctypes.c_double), ("uclk_mhz", ctypes.c_double),
                ("socket_w", ctypes.c_double), ("gfx_activity", ctypes.c_double), ("xcd_mhz", ctypes.c_double * 8)]


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

    def count(self):
        return self.lib.vkb_clock_samples(None, 0) if self.ok else 0

    def now_ms(self):
        return self.lib.vkb_clock_now_ms()

    def samples(self):
        n = self.count()
        if n <= 0:
            return []
        buf = (ClockSample * n)()
        n = min(n, self.lib.vkb_clock_samples(buf, n))
        return [buf[i] for i in range(n)]


def _aggregate(samples):
    """Mean SCLK, memory clock, socket power and GFX activity of samples."""
    if not samples:
        return None
    g = [s.gfx_mhz for s in samples]
    u = [s.uclk_mhz for s in samples if s.uclk_mhz > 0]
    w = [s.socket_w for s in samples if s.socket_w > 0]
    b = [s.gfx_activity for s in samples if s.gfx_activity >= 0]
    mean = lambda xs: round(sum(xs) / len(xs), 1) if xs else None  # noqa: E731
    return {"sclk_mhz": mean(g), "sclk_mhz_min": round(min(g), 1), "sclk_mhz_max": round(max(g), 1),
            "mclk_mhz": mean(u), "socket_w": mean(w), "gfx_busy_pct": mean(b), "samples": len(samples)}


def measure(clock, chunk, timed, settle_ms, per_launch_ms_hint=0.1):
    """The timed protocol for one launch sequence.

    chunk(n) runs n launches back to back and returns their event time in ms
    (synchronised); timed() runs the timed region (warm-up, device sync,
    steps back to back between one event pair) and returns its event time in
    ms.  Settle phase: chunks of ~50 ms until settle_ms have passed on the
    host clock, the sampler running from min(300 ms, settle_ms / 2) on; then
    chunks of ~4 ms until the sampler sees a metrics refresh (at most 1.5 s
    more), and the timed region starts at once.  Returns (timed ms, record)
    with every sample's age relative to the timed region's start."""
    rec = {"settle_ms": settle_ms, "settle_launches": 0, "aligned_to_refresh": False}
    per = max(per_launch_ms_hint, 1e-3)
    sampling = False
    if settle_ms > 0:
        n, t0 = max(1, int(5.0 / per)), time.perf_counter()
        while True:
            ms = chunk(n)
            rec["settle_launches"] += n
            per = max(ms / n, 1e-3)
            el = (time.perf_counter() - t0) * 1e3
            if el >= settle_ms:
                break
            if not sampling and el >= min(300.0, settle_ms / 2):
                sampling = clock.start(1000)
            n = max(1, int(50.0 / per))
        if sampling:
            seen, t1 = clock.count(), time.perf_counter()
            n = max(1, int(4.0 / per))
            while clock.count() == seen and time.perf_counter() - t1 < 1.5:
                chunk(n)
                rec["settle_launches"] += n
            rec["aligned_to_refresh"] = clock.count() > seen
    else:
        sampling = clock.start(1000)
    t_start = clock.now_ms() if clock.ok else None
    total = timed()
    t_end = clock.now_ms() if clock.ok else None
    samples = clock.samples() if sampling else []
    if sampling:
        clock.stop()
    rec["timed_window_ms"] = round(t_end - t_start, 3) if t_start is not None else None
    rec["samples"] = [{"age_ms": round(s.t_ms - t_start, 2), "sclk_mhz": round(s.gfx_mhz, 1),
                       "xcd_mhz": [round(x) for x in s.xcd_mhz],
                       "socket_w": round(s.socket_w, 1), "gfx_busy_pct": round(s.gfx_activity, 1)}
                      for s in samples]
    rec["settle"] = _aggregate([s for s in samples if s.t_ms < t_start])
    rec["timed"] = _aggregate([s for s in samples if t_start <= s.t_ms <= t_end])
    rec["nearest"] = min(rec["samples"], key=lambda s: abs(s["age_ms"])) if samples else None
    return total, rec


def library_ceiling(A, B, out, args, cus, flop_clk_cu, peak, clock):
    """torch.matmul on the same operands under measure()'s protocol, once per
    BLAS backend torch offers on ROCm.  Comparison only."""
    import torch
    tdt = torch.float16 if out == "f16" else torch.float32
    C2 = torch.empty((A.shape[0], B.shape[1]), dtype=tdt, device=A.device)
    flop = 2.0 * A.shape[0] * B.shape[1] * A.shape[1]
    bk = torch.backends.cuda
    saved_backend = bk.preferred_blas_library()
    saved_red = bk.matmul.allow_fp16_reduced_precision_reduction
    saved_tf32 = bk.matmul.allow_tf32
    bk.matmul.allow_fp16_reduced_precision_reduction = False  # fp32 accumulation throughout
    bk.matmul.allow_tf32 = False  # fp32 inputs multiplied in fp32
    res = {}
    tuned = False
    try:
        if args.library_tune:
            torch.cuda.tunable.enable(True)
            torch.cuda.tunable.tuning_enable(True)
            torch.cuda.tunable.set_filename(os.path.join(os.environ.get("TMPDIR", "/tmp"), "vk_tunableop.csv"))
            tuned = True

        def mm():
            if A.dtype == C2.dtype:
                torch.matmul(A, B, out=C2)
            else:  # fp16 in, fp32 out
                torch.mm(A, B, out_dtype=torch.float32, out=C2)

        # torch's names on ROCm: "hipblaslt" (hipBLASLt), "hipblas" (rocBLAS
        # through hipBLAS), "ck" (Composable Kernel GEMMs)
        for name, backend in (("hipblaslt", "hipblaslt"), ("rocblas", "hipblas"), ("ck", "ck")):
            try:
                bk.preferred_blas_library(backend)
            except Exception as e:  # noqa: BLE001 -- a backend this build lacks is reported, not fatal
                res[name] = {"error": str(e)}
                continue
            try:
                mm()
                torch.cuda.synchronize()
            except Exception as e:  # noqa: BLE001
                res[name] = {"error": str(e)}
                continue

            def chunk(n):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(n):
                    mm()
                e1.record()
                e1.synchronize()
                return e0.elapsed_time(e1)

            def timed():
                for _ in range(args.warmup):
                    mm()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(args.steps):
                    mm()
                e1.record()
                e1.synchronize()
                torch.cuda.synchronize()
                return e0.elapsed_time(e1)

            C2.fill_(float("nan"))
            total, rec = measure(clock, chunk, timed, args.settle_ms)
            ms = total / args.steps
            tf = flop / (ms * 1e-3) / 1e12
            ok, max_abs, ratio = check_output(A, B, C2, out)
            if not ok:
                # e.g. a backend that returns without computing this shape
                res[name] = {"rejected": "output not within the accumulation bound of torch's fp32 product",
                             "ms_per_step": round(ms, 5),
                             "error_over_bound": round(ratio, 4) if math.isfinite(ratio) else None}
                continue
            near = rec["nearest"]
            sclk = near["sclk_mhz"] if near else None
            pk = cus * flop_clk_cu * sclk * 1e6 / 1e12 if sclk else None
            res[name] = {"ms_per_step": round(ms, 5), "tflops": round(tf, 2), "frac": round(tf / peak, 4),
                         "sclk_mhz": sclk, "sclk_age_ms": near["age_ms"] if near else None,
                         "frac_clock": round(tf / pk, 4) if pk else None,
                         "output_within_bound": ok, "error_over_bound": round(ratio, 4), "clock": rec}
    finally:
        bk.preferred_blas_library(saved_backend)
        bk.matmul.allow_fp16_reduced_precision_reduction = saved_red
        bk.matmul.allow_tf32 = saved_tf32
        if tuned:
            torch.cuda.tunable.tuning_enable(False)
            torch.cuda.tunable.enable(False)
    timed_ok = {k: v for k, v in res.items() if "tflops" in v}
    best = max(timed_ok, key=lambda k: timed_ok[k]["tflops"]) if timed_ok else None
    return {"best_backend": best,
            "tflops": timed_ok[best]["tflops"] if best else None,
            "ms_per_step": timed_ok[best]["ms_per_step"] if best else None,
            "frac_clock": timed_ok[best]["frac_clock"] if best else None,
            "tunableop": tuned,
            "protocol": "torch.matmul on the same A, B (fp32 accumulation, allow_fp16_reduced_precision_"
                        "reduction off), same settle length ending on a metrics refresh, same warm-up and "
                        "steps back to back between one event pair; after the product's measurements",
            "backends": res}


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


def _finite(x):
    """The record with every non-finite float replaced by None (strict JSON)."""
    if isinstance(x, float):
        return x if math.isfinite(x) else None
    if isinstance(x, dict):
        return {k: _finite(v) for k, v in x.items()}
    if isinstance(x, (list, tuple)):
        return [_finite(v) for v in x]
    return x


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

    # Settle phase and timed region (see measure()): the timed region is C++
    # on the kernel's stream -- warm-up, device sync, `steps` launches back to
    # back between one event pair, device sync.  Wall clock around it as a
    # cross-check.
    probe = ctypes.c_float(0.0)

    def chunk(n):
        st = bench.vkb_back_to_back(*call, n, ctypes.byref(probe))
        if st != 0:
            raise RuntimeError(f"settle phase failed with status {st}")
        return probe.value

    tot = ctypes.c_float(0.0)
    wall = [0.0]

    def timed():
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        st = bench.vkb_stream_loop(*call, args.warmup, args.steps, ctypes.byref(tot))
        torch.cuda.synchronize()
        wall[0] = time.perf_counter() - w0
        if st != 0:
            raise RuntimeError(f"timed loop failed with status {st}")
        return tot.value

    try:
        total_ms, clock_rec = measure(clock, chunk, timed, args.settle_ms)
    except RuntimeError as e:
        print(f"bench.py: {e}", file=sys.stderr)
        return 1
    wall = wall[0]
    mean_ms = total_ms / args.steps
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
    near = clock_rec["nearest"]
    sclk = near["sclk_mhz"] if near else None
    sclk_src = (f"the metrics sample nearest the timed region's start (age {near['age_ms']} ms; "
                f"negative: before the start)") if near else None
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
        "settle": {"ms": args.settle_ms, "launches": clock_rec["settle_launches"],
                   "ends_on_metrics_refresh": clock_rec["aligned_to_refresh"],
                   "note": "the timed dispatches are launches settle.launches + warmup .. + steps - 1 of the run"},
        "reference_loop": ref_loop,
        "clock": {
            "timed": clock_rec["timed"],
            "settle": clock_rec["settle"],
            "samples": clock_rec["samples"],
            "nearest": near,
            "timed_window_ms": clock_rec["timed_window_ms"],
            "sclk_for_frac_clock": sclk_src,
            "source": "amd-smi gpu_metrics (current_gfxclks averaged over XCDs, current_uclk, "
                      "current_socket_power, average_gfx_activity) polled every 1 ms on a host thread; "
                      "the table refreshes about once per second; age_ms = host time of the read that "
                      "saw a refresh minus the timed region's start",
            "error": clock.error,
        },
        "device": {"name": props.name, "cus": cus, "host_cores": os.cpu_count(),
                   "host_threads_available": len(os.sched_getaffinity(0))},
        "max_abs_vs_torch_f32": max_abs_vs_torch,
        "error_over_bound": round(bound_ratio, 4),
        "reference_best_a100_frac_of_peak": 0.897,
        "roofline": roofline,
    }
    if not args.no_library_ceiling:
        lib_ceiling = library_ceiling(A, B, out, args, cus, flop_clk_cu, peak, clock)
        if lib_ceiling["tflops"]:
            lib_ceiling["product_over_library"] = round(tflops / lib_ceiling["tflops"], 4)
        res["library_ceiling"] = lib_ceiling
    else:
        res["library_ceiling"] = None
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(m, n, k, dtype, args.seed, args.cpu_seconds)
    else:
        res["cpu_baseline"] = None
    print(json.dumps(_finite(res)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
