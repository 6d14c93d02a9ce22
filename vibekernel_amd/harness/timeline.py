#!/usr/bin/env python3
"""Per-workgroup timeline of version 7, or of version 8 with --skinny
(measurement tool).

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

With --skinny (default shape 16 x 8192 x 8192) version 8's workgroups record
their XCD, k part, k-steps and the clock at entry, at the end of the k-loop
and when they leave; by_xcd then gives each XCD's mean and latest k-loop
end and the B bytes its workgroups streamed per microsecond of k-loop.

    python vibekernel_amd/harness/timeline.py --skinny [--m 16 --n 8192 --k 8192]

With --f32 (default 4096^3) fp32 version 2's four-wave kernel: every wave
records its XCD, the clock at entry, k-loop start and end and after its
stores complete, and in shader-clock cycles its k-loop and the part spent
from each k-tile's last group to the end of its barrier; the report gives
cycles per 32-deep k-tile against the 16384 a SIMD's MFMAs need.

    python vibekernel_amd/harness/timeline.py --f32 [--m 4096 --n 4096 --k 4096]

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
    p.add_argument("--skinny", action="store_true", help="version 8 (default shape 16 x 8192 x 8192)")
    p.add_argument("--f32", action="store_true", help="fp32 version 2, four-wave kernel (default shape 4096^3)")
    p.add_argument("--lib", default=None, help="the timeline build to load (default vibekernel_amd/lib/libvk_gemm_timeline.so)")
    p.add_argument("--dump", default=None, help="with --skinny: write every workgroup's record to this file")
    p.add_argument("--m", type=int, default=None)
    p.add_argument("--n", type=int, default=None)
    p.add_argument("--k", type=int, default=None)
    p.add_argument("--settle-ms", type=float, default=2500.0)
    p.add_argument("--seed", type=int, default=20261201)
    a = p.parse_args()
    dm, dn, dk = (16, 8192, 8192) if a.skinny else (4096, 4096, 4096)
    m, n, k = a.m or dm, a.n or dn, a.k or dk
    if a.skinny and (m > 256 or n % 128 or k % 32):
        print("timeline.py: --skinny takes M <= 256, N a multiple of 128 and K of 32", file=sys.stderr)
        return 2
    if a.f32 and (m % 256 or n % 256 or k % 32 or (m // 256) * (n // 256) > 1024):
        print("timeline.py: --f32 needs M, N multiples of 256 (at most 1024 tiles) and K of 32", file=sys.stderr)
        return 2
    if not a.skinny and not a.f32 and (m % 256 or n % 256 or k % 64):
        print("timeline.py: version 7 needs M, N multiples of 256 and K of 64", file=sys.stderr)
        return 2

    import numpy as np
    import torch  # before the libraries: they bind to torch's HIP runtime

    if not torch.cuda.is_available():
        print("timeline.py: no GPU visible", file=sys.stderr)
        return 1
    path = a.lib or os.path.join(LIB, "libvk_gemm_timeline.so")
    if not os.path.exists(path):
        print(f"timeline.py: {path} is missing (make -C vibekernel_amd/csrc timeline)", file=sys.stderr)
        return 1
    T = ctypes.CDLL(path, mode=ctypes.RTLD_LOCAL)
    sz, vp = ctypes.c_size_t, ctypes.c_void_p
    T.vk_gemm.argtypes = [ctypes.c_int] * 3 + [sz] * 3 + [vp] * 4
    T.vk_gemm.restype = ctypes.c_int
    T.vk_timeline_read.argtypes = [vp, ctypes.c_int]
    T.vk_timeline_read.restype = ctypes.c_int
    T.vk_timeline_sk_read.argtypes = [vp, ctypes.c_int]
    T.vk_timeline_sk_read.restype = ctypes.c_int
    T.vk_timeline_f32_read.argtypes = [vp, ctypes.c_int]
    T.vk_timeline_f32_read.restype = ctypes.c_int
    sys.path.insert(0, os.path.join(HERE, "..", ".."))
    import bench as B  # the clock sampler bindings (libvk_bench.so)

    bl = B.load_bench_lib()
    clock = B.Clock(bl)

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(a.seed)
    dt = torch.float32 if a.f32 else torch.float16
    A = (torch.rand((m, k), generator=g, device=dev) * 2 - 1).to(dt)
    Bm = (torch.rand((k, n), generator=g, device=dev) * 2 - 1).to(dt)
    C = torch.empty((m, n), dtype=dt, device=dev)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dcode = 2 if a.f32 else 1  # vk_dtype: 1 fp16, 2 fp32
    args = (2 if a.f32 else 8 if a.skinny else 7, dcode, dcode, m, n, k, ctypes.c_void_p(A.data_ptr()),
            ctypes.c_void_p(Bm.data_ptr()), ctypes.c_void_p(C.data_ptr()), s)

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
    if a.skinny:
        return skinny_report(T, a, m, n, k, e0, e1, near, t_start)
    if a.f32:
        return f32_report(T, a, m, n, k, e0, e1, near, t_start)

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


def skinny_report(T, a, m, n, k, e0, e1, near, t_start) -> int:
    """Version 8's records: (entry, k-loop end, leave, XCD, k-steps, k part)."""
    import numpy as np

    nc = 128  # columns per workgroup (f16_skinny_sk.hip pick_nc)
    groups = -(-n // nc)
    ks = 1
    while ks < 8 and groups * ks * 2 <= 256 and k // 32 // (ks * 2) >= 4:
        ks *= 2
    rec = min(groups * ks, 4096)
    buf = np.zeros(rec * 6, dtype=np.uint64)
    if T.vk_timeline_sk_read(buf.ctypes.data, rec) != 0:
        print("timeline.py: vk_timeline_sk_read failed", file=sys.stderr)
        return 1
    r = buf.reshape(rec, 6)
    ts = r[:, :3].astype(np.float64) / 100.0  # 100 MHz ticks -> us
    ts -= ts[:, 0].min()
    xcc, steps, part = r[:, 3].astype(int), r[:, 4].astype(int), r[:, 5].astype(int)
    bbytes = steps * 32 * nc * 2  # B bytes each workgroup streamed
    loop = ts[:, 1] - ts[:, 0]
    out = {
        "workload": f"gemm_f16_{m}x{n}x{k} version 8 (timeline build), uniform[-1,1) seed {a.seed}",
        "event_us_per_launch": round(e0.elapsed_time(e1) * 1e3 / 20, 2),
        "workgroups": int(rec), "k_parts": ks,
        "span_us": round(float(ts[:, 2].max()), 2),
        "loop_end_us_min_mean_max": [round(float(f(ts[:, 1])), 2) for f in (np.min, np.mean, np.max)],
        "leave_after_loop_us_mean_max": [round(float(f(ts[:, 2] - ts[:, 1])), 2) for f in (np.mean, np.max)],
        "sclk_sample_age_ms": round(near.t_ms - t_start, 1) if near else None,
        "by_xcd": [], "by_part": [],
    }
    for x in range(8):
        sel = xcc == x
        if not sel.any():
            continue
        out["by_xcd"].append({
            "xcd": x, "sclk_mhz": float(near.xcd_mhz[x]) if near else None, "workgroups": int(sel.sum()),
            "entry_us_mean_max": [round(float(ts[sel, 0].mean()), 2), round(float(ts[sel, 0].max()), 2)],
            "loop_us_mean_max": [round(float(loop[sel].mean()), 2), round(float(loop[sel].max()), 2)],
            "loop_end_us_mean": round(float(ts[sel, 1].mean()), 2),
            "loop_end_us_max": round(float(ts[sel, 1].max()), 2),
            "b_gb_per_s_per_workgroup": round(float((bbytes[sel] / loop[sel]).mean()) / 1e3, 2),
            "b_tb_per_s_of_xcd": round(float(bbytes[sel].sum() / ts[sel, 1].max()) / 1e6, 3),
        })
    for q in range(ks):
        sel = part == q
        out["by_part"].append({"part": q, "steps": int(steps[sel].max()) if sel.any() else 0,
                               "xcds": sorted(set(int(v) for v in xcc[sel])),
                               "loop_us_mean": round(float(loop[sel].mean()), 2) if sel.any() else None,
                               "loop_end_us_mean": round(float(ts[sel, 1].mean()), 2) if sel.any() else None})
    if a.dump:
        np.savetxt(a.dump, np.column_stack([ts, xcc, steps, part]), fmt="%.3f %.3f %.3f %d %d %d",
                   header="entry_us loop_end_us leave_us xcd steps part")
    print(json.dumps(out), flush=True)
    return 0


def f32_report(T, a, m, n, k, e0, e1, near, t_start) -> int:
    """fp32 version 2's records per wave: (entry, loop start, loop end, stores
    complete, XCD, loop cycles, last-group-and-barrier cycles, k-tiles)."""
    import numpy as np

    waves = (m // 256) * (n // 256) * 4
    buf = np.zeros(waves * 8, dtype=np.uint64)
    if T.vk_timeline_f32_read(buf.ctypes.data, waves) != 0:
        print("timeline.py: vk_timeline_f32_read failed", file=sys.stderr)
        return 1
    r = buf.reshape(waves, 8)
    ts = r[:, :4].astype(np.float64) / 100.0  # 100 MHz ticks -> us
    ts -= ts[:, 0].min()
    xcc = r[:, 4].astype(int)
    loop_c, bar_c, nk = r[:, 5].astype(np.float64), r[:, 6].astype(np.float64), r[:, 7].astype(np.float64)
    loop_us = ts[:, 2] - ts[:, 1]
    ideal = 256 * 64.0  # one wave per SIMD: 256 MFMAs of 64 cycles per k-tile
    out = {
        "workload": f"gemm_f32_{m}x{n}x{k} fp32 version 2, four-wave kernel (timeline build), seed {a.seed}",
        "event_us_per_launch": round(e0.elapsed_time(e1) * 1e3 / 20, 2),
        "span_us": round(float(ts[:, 3].max()), 2),
        "entry_skew_us_max": round(float(ts[:, 0].max()), 2),
        "prologue_us": round(float((ts[:, 1] - ts[:, 0]).mean()), 2),
        "loop_us_mean": round(float(loop_us.mean()), 2),
        "loop_end_us_min_mean_max": [round(float(f(ts[:, 2])), 2) for f in (np.min, np.mean, np.max)],
        "epilogue_us_mean_max": [round(float(f(ts[:, 3] - ts[:, 2])), 2) for f in (np.mean, np.max)],
        "memtime_mhz": round(float((loop_c / loop_us).mean()), 1),
        "cycles_per_ktile": round(float((loop_c / nk).mean()), 1),
        "last_group_and_barrier_cycles_per_ktile": round(float((bar_c / nk).mean()), 1),
        "loop_mfma_efficiency": round(float((ideal * nk / loop_c).mean()), 4),
        "sclk_sample_age_ms": round(near.t_ms - t_start, 1) if near else None,
        "by_xcd": [],
    }
    for x in range(8):
        sel = xcc == x
        if not sel.any():
            continue
        out["by_xcd"].append({
            "xcd": x, "sclk_mhz": float(near.xcd_mhz[x]) if near else None, "waves": int(sel.sum()),
            "loop_us_mean": round(float(loop_us[sel].mean()), 2),
            "loop_end_us_max": round(float(ts[sel, 2].max()), 2),
            "exit_us_max": round(float(ts[sel, 3].max()), 2),
            "cycles_per_ktile": round(float((loop_c[sel] / nk[sel]).mean()), 1),
            "last_group_and_barrier_cycles_per_ktile": round(float((bar_c[sel] / nk[sel]).mean()), 1),
        })
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
