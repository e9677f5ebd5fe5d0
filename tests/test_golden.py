"""Golden fixtures (tests/golden/gemm_golden.npz, written by
tests/golden/make_golden.py): the blocked oracle must reproduce them on the
CPU, and the HIP path (through the C ABI) on the GPU.  The last two cases are
the reference's own known answers (tests/blas/level3/test_gemm.cpp:39-88)."""
import os

import numpy as np
import pytest

import oracle

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gemm_golden.npz")


def load_cases():
    z = np.load(PATH)  # plain arrays only (allow_pickle stays False)
    n = len({k.split("_")[0] for k in z.files})
    cases = []
    for i in range(n):
        p = f"c{i:02d}_"
        meta = z[p + "meta"].tolist()
        alpha, beta = z[p + "scal"].tolist()
        cases.append((i, meta, alpha, beta, z[p + "A"], z[p + "B"], z[p + "C"], z[p + "out"]))
    return cases


CASES = load_cases()


def _tol(dtype):
    return 1e-6 if dtype == np.float32 else 1e-14


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"case{c[0]:02d}")
def test_oracle_reproduces_golden(case):
    i, (layout, ta, tb, m, n, k, lda, ldb, ldc), alpha, beta, A, B, C, out = case
    got = C.copy()
    oracle.gemm(layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, got, ldc, 1)
    assert oracle.rel_fro_err(got.reshape(1, -1), out.reshape(1, -1)) <= _tol(A.dtype.type)


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"case{c[0]:02d}")
def test_hip_reproduces_golden(cuda, case):
    from gemm_cases import TOL, run_sbx
    i, (layout, ta, tb, m, n, k, lda, ldb, ldc), alpha, beta, A, B, C, out = case
    got = run_sbx(cuda, A.dtype.type, layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C,
                  ldc)
    err = oracle.rel_fro_err(got.reshape(1, -1), out.reshape(1, -1))
    print(f"golden case {i}: err={err:.2e}")
    assert err <= TOL[A.dtype.type]
    if i >= len(CASES) - 2:  # the reference's integer known answers are exact
        np.testing.assert_array_equal(got, out)
