"""ctypes binding of libvk_gemm.so (the C ABI declared in include/vk_gemm.h).

The library is built in-tree by ``vibekernel_amd.build`` (hipcc, gfx950) into
``vibekernel_amd/lib/libvk_gemm.so``.  Loading fails loudly when it is missing:
there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libvk_gemm.so")

DTYPE_F16 = 1
DTYPE_F32 = 2

VK_OK = 0
STATUS_NAMES = {
    0: "VK_OK",
    -1: "VK_ERR_VERSION",
    -2: "VK_ERR_DTYPE",
    -3: "VK_ERR_SHAPE",
    -4: "VK_ERR_ALIGN",
    -5: "VK_ERR_NULL",
    -6: "VK_ERR_WORKSPACE",
    -7: "VK_ERR_HIP",
    -8: "VK_ERR_RANGE",
}

# Every symbol include/vk_gemm.h declares (checked by the CPU test suite).
EXPORTED_SYMBOLS = (
    "vk_gemm",
    "vk_gemm_ws",
    "vk_gemm_noalloc",
    "vk_gemm_workspace_bytes",
    "vk_gemm_name",
    "vk_gemm_query",
    "vk_gemm_list",
    "vk_gemm_check",
    "vk_gemm_release",
    "vk_status_string",
    "vk_gemm_abi_version",
)


class VkError(RuntimeError):
    def __init__(self, status: int, what: str = ""):
        self.status = status
        name = STATUS_NAMES.get(status, str(status))
        super().__init__(f"{what}: {name} ({status_string(status)})" if what else name)


class vk_caps(ctypes.Structure):
    _fields_ = [
        ("version", ctypes.c_int),
        ("in_dtype", ctypes.c_int),
        ("out_dtype_mask", ctypes.c_int),
        ("div_m", ctypes.c_uint32),
        ("div_n", ctypes.c_uint32),
        ("div_k", ctypes.c_uint32),
        ("max_m", ctypes.c_uint64),
        ("align_bytes", ctypes.c_uint32),
        ("tile_m", ctypes.c_uint32),
        ("tile_n", ctypes.c_uint32),
        ("tile_k", ctypes.c_uint32),
        ("threads", ctypes.c_uint32),
        ("lds_bytes", ctypes.c_uint32),
        ("tolerance_tier", ctypes.c_int),
        ("uses_workspace", ctypes.c_int),
    ]


@dataclass(frozen=True)
class Caps:
    version: int
    in_dtype: int
    out_dtypes: tuple
    div_m: int
    div_n: int
    div_k: int
    max_m: int
    align_bytes: int
    tile: tuple
    threads: int
    lds_bytes: int
    tolerance_tier: int
    uses_workspace: bool


_lib = None


def lib_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load libvk_gemm.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    # PyTorch-ROCm ships its own HIP runtime (same SONAME, libamdhip64.so.7,
    # loaded by file name).  Importing torch first lets the dynamic linker
    # bind this library's libamdhip64.so.7 dependency to that copy; loading
    # this library first would map a second HIP runtime into the process and
    # every launch on torch-allocated memory would fail.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(hipcc --offload-arch=gfx950); there is no non-HIP fallback")
    L = ctypes.CDLL(LIB_PATH)
    sz, vp, ci = ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int
    L.vk_gemm.argtypes = [ci, ci, ci, sz, sz, sz, vp, vp, vp, vp]
    L.vk_gemm.restype = ci
    L.vk_gemm_ws.argtypes = [ci, ci, ci, sz, sz, sz, vp, vp, vp, vp, sz, vp]
    L.vk_gemm_ws.restype = ci
    L.vk_gemm_noalloc.argtypes = [ci, ci, ci, sz, sz, sz, vp, vp, vp, vp]
    L.vk_gemm_noalloc.restype = ci
    L.vk_gemm_workspace_bytes.argtypes = [ci, ci, sz, sz, sz]
    L.vk_gemm_workspace_bytes.restype = sz
    L.vk_gemm_name.argtypes = [ci, ci]
    L.vk_gemm_name.restype = ctypes.c_char_p
    L.vk_gemm_query.argtypes = [ci, ci, ctypes.POINTER(vk_caps)]
    L.vk_gemm_query.restype = ci
    L.vk_gemm_list.argtypes = [ci, ctypes.POINTER(ci), ci]
    L.vk_gemm_list.restype = ci
    L.vk_gemm_check.argtypes = [ci, ci, ci, sz, sz, sz, vp, vp, vp]
    L.vk_gemm_check.restype = ci
    L.vk_gemm_release.argtypes = []
    L.vk_gemm_release.restype = ci
    L.vk_status_string.argtypes = [ci]
    L.vk_status_string.restype = ctypes.c_char_p
    L.vk_gemm_abi_version.argtypes = []
    L.vk_gemm_abi_version.restype = ci
    _lib = L
    return L


def hip_runtimes_loaded() -> list:
    """Paths of the HIP runtime libraries mapped into this process (should be
    exactly one)."""
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64" in line:
                paths.add(line.split()[-1])
    return sorted(paths)


def status_string(status: int) -> str:
    return load().vk_status_string(status).decode()


def abi_version() -> int:
    return int(load().vk_gemm_abi_version())


# fp16 versions 71-77: version 7 with one ingredient turned off each
# (include/vk_gemm.h, VK_F16_LEAVE_ONE_OUT_FIRST/_LAST); measured, never picked.
LEAVE_ONE_OUT = range(71, 78)


def versions(in_dtype: int) -> list:
    L = load()
    n = L.vk_gemm_list(in_dtype, None, 0)
    buf = (ctypes.c_int * max(n, 1))()
    L.vk_gemm_list(in_dtype, buf, n)
    return [int(buf[i]) for i in range(n)]


def name(version: int, in_dtype: int):
    r = load().vk_gemm_name(version, in_dtype)
    return r.decode() if r is not None else None


def query(version: int, in_dtype: int) -> Caps:
    c = vk_caps()
    st = load().vk_gemm_query(version, in_dtype, ctypes.byref(c))
    if st != VK_OK:
        raise VkError(st, f"vk_gemm_query(version={version})")
    outs = tuple(d for d in (DTYPE_F16, DTYPE_F32) if c.out_dtype_mask & (1 << d))
    return Caps(c.version, c.in_dtype, outs, c.div_m, c.div_n, c.div_k, c.max_m, c.align_bytes,
                (c.tile_m, c.tile_n, c.tile_k), c.threads, c.lds_bytes, c.tolerance_tier,
                bool(c.uses_workspace))


def check(version, in_dtype, out_dtype, m, n, k, a_ptr, b_ptr, c_ptr) -> int:
    return int(load().vk_gemm_check(version, in_dtype, out_dtype, m, n, k, a_ptr, b_ptr, c_ptr))


def gemm(version, in_dtype, out_dtype, m, n, k, a_ptr, b_ptr, c_ptr, stream=None) -> int:
    return int(load().vk_gemm(version, in_dtype, out_dtype, m, n, k, a_ptr, b_ptr, c_ptr, stream))


def gemm_ws(version, in_dtype, out_dtype, m, n, k, a_ptr, b_ptr, c_ptr, ws_ptr, ws_bytes,
            stream=None) -> int:
    return int(load().vk_gemm_ws(version, in_dtype, out_dtype, m, n, k, a_ptr, b_ptr, c_ptr,
                                 ws_ptr, ws_bytes, stream))


def gemm_noalloc(version, in_dtype, out_dtype, m, n, k, a_ptr, b_ptr, c_ptr, stream=None) -> int:
    return int(load().vk_gemm_noalloc(version, in_dtype, out_dtype, m, n, k, a_ptr, b_ptr, c_ptr, stream))


def workspace_bytes(version, in_dtype, m, n, k) -> int:
    return int(load().vk_gemm_workspace_bytes(version, in_dtype, m, n, k))


def release() -> int:
    return int(load().vk_gemm_release())
