"""The committed golden fixtures (tests/golden/*.npz, made by
tests/golden/make_golden.py) against the CPU side: the exact products are
reproduced by an fp64 brute force, and the oracle's v0 results bit for bit.
A drift in the oracle, its build or the fixtures fails here first."""
import glob
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def test_fixtures_present():
    assert len(FIXTURES) >= 6


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p)[:-4])
def test_golden_exact_and_oracle(oracle, path):
    with np.load(path, allow_pickle=False) as z:
        A, B, exact = z["A"], z["B"], z["exact_f64"]
        # fp64 brute force in ascending k: the products are exact and the
        # sums far inside fp64, so any order agrees to a few fp64 ulps
        brute = np.einsum("ik,kj->ij", A.astype(np.float64), B.astype(np.float64))
        assert np.allclose(brute, exact, rtol=1e-12, atol=1e-12)
        if A.dtype == np.float16:
            assert np.array_equal(oracle.hgemm(A, B).view(np.uint16), z["v0_f16"].view(np.uint16))
            assert np.array_equal(oracle.hgemm(A, B, out="f32").view(np.uint32), z["v0_f32"].view(np.uint32))
        else:
            assert np.array_equal(oracle.sgemm(A, B).view(np.uint32), z["v0_f32"].view(np.uint32))
