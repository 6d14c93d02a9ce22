"""Shared helpers of the GPU parity tests: seeded inputs, the C-ABI call and
the tolerance rules (all stated here, next to the numbers)."""
import sys

import numpy as np

U32 = 2.0 ** -24  # unit roundoff of binary32


def announce(*parts):
    """Name the case on the real stderr before a GPU step, flushed, so a run
    that dies mid-test still says which case it was."""
    print("[gpu-case]", *parts, file=sys.__stderr__, flush=True)


def make_inputs(m, n, k, dist, seed, dtype=np.float16):
    rng = np.random.default_rng(seed)
    if dist == "uniform":
        A = rng.uniform(-1, 1, (m, k))
        B = rng.uniform(-1, 1, (k, n))
    elif dist == "normal":
        A = rng.standard_normal((m, k))
        B = rng.standard_normal((k, n))
    elif dist == "normal0.5":
        A = rng.normal(0, 0.5, (m, k))
        B = rng.normal(0, 0.5, (k, n))
    elif dist == "int":
        A = rng.integers(-2, 3, (m, k))
        B = rng.integers(-2, 3, (k, n))
    else:
        raise ValueError(dist)
    return np.ascontiguousarray(A.astype(dtype)), np.ascontiguousarray(B.astype(dtype))


def run_gemm(version, A, B, out_dtype, device="cuda:0", poison=True):
    """Upload, run one kernel version through the C ABI, download."""
    import torch
    import vibekernel_amd as vk
    m, k = A.shape
    n = B.shape[1]
    tA = torch.from_numpy(A).to(device)
    tB = torch.from_numpy(B).to(device)
    tdt = torch.float16 if out_dtype == "f16" else torch.float32
    tC = torch.empty((m, n), dtype=tdt, device=device)
    if poison:
        tC.fill_(float("nan"))  # the kernel must overwrite every element
    announce(f"version={version} m={m} n={n} k={k} out={out_dtype}")
    vk.matmul(m, n, k, tA, tB, tC, version)
    torch.cuda.synchronize()
    return tC.cpu().numpy()


def fp32_bound(A, B, factor=2.0):
    """Forward error bound of an fp32-accumulated product: k * u * |A| |B|
    (one rounding per accumulated term), times a safety factor for the MFMA's
    internal adds."""
    k = A.shape[1]
    return factor * k * U32 * (np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64)))


def check_f32_out(C, A, B, C64):
    assert not np.isnan(C).any(), "NaN left in C (element not written)"
    err = np.abs(C.astype(np.float64) - C64)
    bound = fp32_bound(A, B)
    bad = err > bound + 1e-30
    assert not bad.any(), f"{bad.sum()} elements beyond the fp32 bound; max err {err.max():.3e}"
    return err.max()


def f16_half_ulp(R):
    """Half the larger of the two fp16 gaps around R: the widest an exact
    value can sit from its round-to-nearest result (at a power of two the gap
    away from zero is twice the gap toward it)."""
    R = R.astype(np.float16)
    up = np.abs(np.nextafter(R, np.float16(np.inf)).astype(np.float64) - R.astype(np.float64))
    dn = np.abs(R.astype(np.float64) - np.nextafter(R, np.float16(-np.inf)).astype(np.float64))
    return np.maximum(up, dn) / 2


def check_f16_out(C, A, B, C64):
    assert not np.isnan(C.astype(np.float32)).any(), "NaN left in C (element not written)"
    R = C64.astype(np.float16)
    half_ulp = f16_half_ulp(R)
    err = np.abs(C.astype(np.float64) - C64)
    bound = fp32_bound(A, B) + half_ulp * 1.0001
    bad = err > bound
    assert not bad.any(), f"{bad.sum()} fp16 elements beyond bound; max err {err.max():.3e}"
