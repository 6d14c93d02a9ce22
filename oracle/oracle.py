"""ctypes front end of the CPU oracle (oracle/vk_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/ and by
``__graft_entry__.smoke()`` to verify its result.  bench.py's cpu_baseline leg
times the harness's own version 0 (libvk_v0.so), not this oracle.
The product never imports it.

Every function follows a reference file (paths relative to the reference
repository root):

* :func:`sgemm`  -- results/ralph_loop_fable/src/matmul_f32/matmul_f32_v0_cblas.cpp:8-12
* :func:`hgemm`  -- results/ralph_loop_fable/src/matmul_f16/matmul_f16_v0_cblas.cpp:11-26
* :func:`mean_rel_err` -- results/naive_cycle4/include/playground/test_data.hpp:145-162
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")

ERR_SKIP_ZERO = 0
ERR_LEGACY = 1
STATUS_OK, STATUS_INF, STATUS_NAN, STATUS_EMPTY = 0, 1, 2, 3

_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with oracle/Makefile (gcc + OpenMP)."""
    args = ["make", "-C", _HERE]
    if force:
        args.append("-B")
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sz, vp, u16p, f32p, f64p = (ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_void_p)
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f16_to_f32_array.argtypes = [u16p, f32p, sz]
        L.orc_f32_to_f16_array.argtypes = [f32p, u16p, sz]
        for name in ("orc_sgemm", "orc_hgemm", "orc_hgemm_f32out", "orc_dgemm_h", "orc_dgemm_f"):
            getattr(L, name).argtypes = [sz, sz, sz, vp, vp, vp]
            getattr(L, name).restype = None
        for name in ("orc_mean_rel_err_h", "orc_mean_rel_err_f"):
            getattr(L, name).argtypes = [vp, vp, sz, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
            getattr(L, name).restype = ctypes.c_float
        L.orc_mean_rel_err_f64.argtypes = [f64p, f64p, sz]
        L.orc_mean_rel_err_f64.restype = ctypes.c_double
        L.orc_max_abs_err_f.argtypes = [f32p, f32p, sz]
        L.orc_max_abs_err_f.restype = ctypes.c_double
        L.orc_num_threads.restype = ctypes.c_int
        L.orc_set_num_threads.argtypes = [ctypes.c_int]
        L.orc_set_num_threads.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _as_u16(a: np.ndarray) -> np.ndarray:
    """fp16 arrays are passed as their bit patterns."""
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    assert a.dtype == np.uint16
    return np.ascontiguousarray(a)


def num_threads() -> int:
    return int(lib().orc_num_threads())


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(int(n))


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = _as_u16(h)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    """Round to nearest even; returns a float16 array."""
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(_ptr(f), _ptr(out), f.size)
    return out.view(np.float16)


def sgemm(A: np.ndarray, B: np.ndarray) -> np.ndarray:
    """cblas_sgemm(RowMajor, NoTrans, NoTrans, m, n, k, 1, A, k, B, n, 0, C, n)."""
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    m, k = A.shape
    k2, n = B.shape
    assert k == k2
    C = np.empty((m, n), dtype=np.float32)
    lib().orc_sgemm(m, n, k, _ptr(A), _ptr(B), _ptr(C))
    return C


def hgemm(A: np.ndarray, B: np.ndarray, out: str = "f16") -> np.ndarray:
    """fp16 v0: widen A and B (exact), sgemm, narrow C with RNE (out="f16")
    or keep the fp32 result (out="f32")."""
    A = _as_u16(A)
    B = _as_u16(B)
    m, k = A.shape
    k2, n = B.shape
    assert k == k2
    if out == "f16":
        C = np.empty((m, n), dtype=np.uint16)
        lib().orc_hgemm(m, n, k, _ptr(A), _ptr(B), _ptr(C))
        return C.view(np.float16)
    C = np.empty((m, n), dtype=np.float32)
    lib().orc_hgemm_f32out(m, n, k, _ptr(A), _ptr(B), _ptr(C))
    return C


def dgemm(A: np.ndarray, B: np.ndarray) -> np.ndarray:
    """fp64 brute force; A and B fp16 or fp32."""
    m, k = A.shape
    k2, n = B.shape
    assert k == k2
    C = np.empty((m, n), dtype=np.float64)
    if A.dtype == np.float16 or A.dtype == np.uint16:
        A, B = _as_u16(A), _as_u16(B)
        lib().orc_dgemm_h(m, n, k, _ptr(A), _ptr(B), _ptr(C))
    else:
        A = np.ascontiguousarray(A, dtype=np.float32)
        B = np.ascontiguousarray(B, dtype=np.float32)
        lib().orc_dgemm_f(m, n, k, _ptr(A), _ptr(B), _ptr(C))
    return C


def mean_rel_err(GT: np.ndarray, C: np.ndarray, mode: int = ERR_SKIP_ZERO):
    """test_data.hpp:145-162 statistic.  Returns (value, status)."""
    st = ctypes.c_int(0)
    if GT.dtype in (np.float16, np.uint16):
        g, c = _as_u16(GT).ravel(), _as_u16(C).ravel()
        assert g.size == c.size
        v = lib().orc_mean_rel_err_h(_ptr(g), _ptr(c), g.size, mode, ctypes.byref(st))
    else:
        g = np.ascontiguousarray(GT, dtype=np.float32).ravel()
        c = np.ascontiguousarray(C, dtype=np.float32).ravel()
        assert g.size == c.size
        v = lib().orc_mean_rel_err_f(_ptr(g), _ptr(c), g.size, mode, ctypes.byref(st))
    return float(v), int(st.value)


def mean_rel_err_f64(GT: np.ndarray, C: np.ndarray) -> float:
    g = np.ascontiguousarray(GT, dtype=np.float64).ravel()
    c = np.ascontiguousarray(C, dtype=np.float64).ravel()
    return float(lib().orc_mean_rel_err_f64(_ptr(g), _ptr(c), g.size))


def max_abs_err(GT: np.ndarray, C: np.ndarray) -> float:
    g = np.ascontiguousarray(GT, dtype=np.float32).ravel()
    c = np.ascontiguousarray(C, dtype=np.float32).ravel()
    return float(lib().orc_max_abs_err_f(_ptr(g), _ptr(c), g.size))
