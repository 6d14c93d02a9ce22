#!/usr/bin/env python3
"""Per-workgroup timeline of version 7 (measurement tool).

Loads the timeline build of the library (`make -C vibekernel_amd/csrc
timeline` -> vibekernel_amd/lib/libvk_gemm_timeline.so, where version 7's
kernel records, for one wave of each wave group, its XCD (the XCC_ID
hardware register) and the 100 MHz real-time clock at entry, at the first
MFMA, at the end of the k-loop, after its C stores are issued and after they
complete), runs the GEMM back to back for --settle-ms, then 20 launches
between an event pair, and reads the last launch's records.  The driver's
metrics table is sampled meanwhile (libvk_bench.so), with the SCLK of every
XCD.  Prints one JSON object:

  span_us            first entry to last store completion of the launch
  prologue_us        entry -> first MFMA (mean over wave groups)
  epilogue_us        end of k-loop -> stores complete (mean)
  by_xcd             per XCD: its SCLK (the sample nearest the timed
                     launches), workgroups, mean and latest end of the
                     k-loop, mean k-loop duration, and the k-loop's cycles
                     per 64-deep k-tile at that SCLK against the 2048 MFMA
                     cycles a SIMD's two waves need per k-tile
                     (loop_mfma_efficiency)

    python vibekernel_amd/harness/timeline.py [--m 4096 --n 4096 --k 4096]

Not part of the product path: the timeline build exists for this tool only.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "..", "lib")


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--m", type=int, default=4096)
    p.add_argument("--n", type=int, default=4096)
    p.add_argument("--k", type=int, default=4096)
    p.add_argument("--settle-ms", type=float, default=2500.0)
    p.add_argument("--seed", type=int, default=20261201)
    a = p.parse_args()
    m, n, k = a.m, a.n, a.k
    if m % 256 or n % 256 or k % 64:
        print("timeline.py: version 7 needs M, N multiples of 256 and K of 64", file=sys.stderr)
        return 2

    import numpy as np
    import torch  # before the libraries: they bind to torch's HIP runtime

    if not torch.cuda.is_available():
        print("timeline.py: no GPU visible", file=sys.stderr)
        return 1
    path = os.path.join(LIB, "libvk_gemm_timeline.so")
    if not os.path.exists(path):
        print(f"timeline.py: {path} is missing (make -C vibekernel_amd/csrc timeline)", file=sys.stderr)
        return 1
    T = ctypes.CDLL(path, mode=ctypes.RTLD_LOCAL)
    sz, vp = ctypes.c_size_t, ctypes.c_void_p
    T.vk_gemm.argtypes = [ctypes.c_int] * 3 + [sz] * 3 + [vp] * 4
    T.vk_gemm.restype = ctypes.c_int
    T.vk_timeline_read.argtypes = [vp, ctypes.c_int]
    T.vk_timeline_read.restype = ctypes.c_int
    sys.path.insert(0, os.path.join(HERE, "..", ".."))
    import bench as B  # the clock sampler bindings (libvk_bench.so)

    bl = B.load_bench_lib()
    clock = B.Clock(bl)

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(a.seed)
    A = (torch.rand((m, k), generator=g, device=dev) * 2 - 1).half()
    Bm = (torch.rand((k, n), generator=g, device=dev) * 2 - 1).half()
    C = torch.empty((m, n), dtype=torch.float16, device=dev)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = (7, 1, 1, m, n, k, ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(Bm.data_ptr()),
            ctypes.c_void_p(C.data_ptr()), s)

    def run(count):
        for _ in range(count):
            st = T.vk_gemm(*args)
            if st != 0:
                raise RuntimeError(f"vk_gemm status {st}")

    sampling = False
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < a.settle_ms:
        run(20)
        torch.cuda.synchronize()
        if not sampling and (time.perf_counter() - t0) * 1e3 >= min(300.0, a.settle_ms / 2):
            sampling = clock.start(1000)
    t_start = clock.now_ms() if clock.ok else None
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    run(20)
    e1.record()
    torch.cuda.synchronize()
    samples = clock.samples() if sampling else []
    if sampling:
        clock.stop()
    near = min(samples, key=lambda x: abs(x.t_ms - t_start)) if samples else None

    groups = (m // 256) * (n // 256)
    rec = min(groups, 4096)
    buf = np.zeros(rec * 2 * 8, dtype=np.uint64)
    if T.vk_timeline_read(buf.ctypes.data, rec * 2) != 0:
        print("timeline.py: vk_timeline_read failed", file=sys.stderr)
        return 1
    r = buf.reshape(rec, 2, 8)
    ts = r[:, :, :5].astype(np.float64) / 100.0  # 100 MHz ticks -> us
    ts -= ts[:, :, 0].min()
    xcc = r[:, 0, 5].astype(int)
    nkt = k // 64
    out = {
        "workload": f"gemm_f16_{m}x{n}x{k} version 7 (timeline build), uniform[-1,1) seed {a.seed}",
        "event_us_per_launch": round(e0.elapsed_time(e1) * 1e3 / 20, 2),
        "span_us": round(float(ts[:, :, 4].max()), 2),
        "entry_skew_us_max": round(float(ts[:, :, 0].max()), 2),
        "prologue_us": round(float((ts[:, :, 1] - ts[:, :, 0]).mean()), 2),
        "loop_us_mean": round(float((ts[:, :, 2] - ts[:, :, 1]).mean()), 2),
        "loop_end_us_min_mean_max": [round(float(f(ts[:, :, 2])), 2) for f in (np.min, np.mean, np.max)],
        "epilogue_us": round(float((ts[:, :, 4] - ts[:, :, 2]).mean()), 2),
        "sclk_sample_age_ms": round(near.t_ms - t_start, 1) if near else None,
        "socket_w": near.socket_w if near else None,
        "by_xcd": [],
    }
    for x in range(8):
        sel = xcc == x
        if not sel.any():
            continue
        mhz = float(near.xcd_mhz[x]) if near else 0.0
        loop = float((ts[sel, :, 2] - ts[sel, :, 1]).mean())
        cyc = loop * mhz / nkt if mhz else None
        out["by_xcd"].append({
            "xcd": x, "sclk_mhz": mhz, "workgroups": int(sel.sum()),
            "loop_end_us_mean": round(float(ts[sel, :, 2].mean()), 2),
            "loop_end_us_max": round(float(ts[sel, :, 2].max()), 2),
            "loop_us_mean": round(loop, 2),
            "cycles_per_ktile": round(cyc, 1) if cyc else None,
            "loop_mfma_efficiency": round(2048.0 / cyc, 4) if cyc else None,
        })
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
