"""Writes the golden fixtures of this directory (run from the repository root:
``python tests/golden/make_golden.py``).

The reference holds no golden vectors for this path: its tests are run logs
of random inputs seeded from std::random_device.  These fixtures are made
here instead, from seeded inputs: for each case the inputs, the exact product
(fp64 brute force; fp16 and small-integer inputs make every product exact in
fp64 and the sums exact to well below one fp32 ulp), and the oracle's v0
results (the cblas_sgemm restatement: fp32 fmaf chain in ascending k, then
RNE to fp16 where the output is fp16).  Arrays only, stored with numpy's
savez_compressed (no pickled objects); load with allow_pickle=False.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle  # noqa: E402

# name, dtype, (m, n, k), distribution, seed
CASES = [
    ("f16_17x33x65_uniform", np.float16, (17, 33, 65), "uniform", 1701),
    ("f16_64x64x64_int", np.float16, (64, 64, 64), "int", 6464),
    ("f16_256x256x64_normal", np.float16, (256, 256, 64), "normal", 25664),
    ("f16_256x512x128_int", np.float16, (256, 512, 128), "int", 256128),
    ("f16_16x256x512_uniform", np.float16, (16, 256, 512), "uniform", 16256),
    ("f32_64x96x128_uniform", np.float32, (64, 96, 128), "uniform", 6496),
    ("f32_256x256x32_int", np.float32, (256, 256, 32), "int", 25632),
    ("f16_300x264x72_int", np.float16, (300, 264, 72), "int", 30026),
    ("f16_1x256x96_uniform", np.float16, (1, 256, 96), "uniform", 1256),
    ("f32_100x260x36_uniform", np.float32, (100, 260, 36), "uniform", 10026),
]


def inputs(dtype, m, n, k, dist, seed):
    rng = np.random.default_rng(seed)
    if dist == "uniform":
        A, B = rng.uniform(-1, 1, (m, k)), rng.uniform(-1, 1, (k, n))
    elif dist == "normal":
        A, B = rng.standard_normal((m, k)), rng.standard_normal((k, n))
    else:
        A, B = rng.integers(-2, 3, (m, k)), rng.integers(-2, 3, (k, n))
    return np.ascontiguousarray(A.astype(dtype)), np.ascontiguousarray(B.astype(dtype))


def make(name, dtype, shape, dist, seed):
    m, n, k = shape
    A, B = inputs(dtype, m, n, k, dist, seed)
    exact = A.astype(np.float64) @ B.astype(np.float64)
    out = {"A": A, "B": B, "exact_f64": exact}
    if dtype == np.float16:
        out["v0_f16"] = oracle.hgemm(A, B)
        out["v0_f32"] = oracle.hgemm(A, B, out="f32")
    else:
        out["v0_f32"] = oracle.sgemm(A, B)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **out)


if __name__ == "__main__":
    # make_golden.py [name ...]: only the named fixtures (all when none)
    for case in CASES:
        if len(sys.argv) == 1 or case[0] in sys.argv[1:]:
            make(*case)
            print("wrote", case[0])
