"""MI355X (gfx950) GEMM kernel suite behind the playground ``matmul`` surface.

The compute lives in libvk_gemm.so (hand-written HIP kernels + a C ABI,
include/vk_gemm.h); this package is the Python front end used by the tests
and the benchmark.
"""
from ._abi import DTYPE_F16, DTYPE_F32, VkError, abi_version, lib_path, load  # noqa: F401
from .gemm import gemm, matmul, name, pick_version, query, versions  # noqa: F401

# Default fp16 version: the fastest kernel for tile-divisible shapes (256x256 tiles,
# 64-deep k-tiles, 8 waves in two phase-shifted groups, 16x16x32 MFMAs).
DEFAULT_F16_VERSION = 7
