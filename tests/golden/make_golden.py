"""Writes tests/golden/gemm_golden.npz: small seeded GEMM cases whose expected
outputs come from the oracle's long-double triple loop (sbo_gemm_naive_ld).

Cases: fp32 and fp64 x row/column-major x the four transA/transB combinations
at (m, n, k) = (19, 13, 11), alpha/beta varied, plus one fp32 row-major case
at (70, 66, 40) that crosses 64-wide tile edges, plus the two known answers
of the reference (tests/blas/level3/test_gemm.cpp:39-88).

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402


def case(dtype, layout, ta, tb, m, n, k, alpha, beta, seed):
    sa = (k, m) if ta else (m, k)
    sb = (n, k) if tb else (k, n)
    lda = sa[1] if layout == 0 else sa[0]
    ldb = sb[1] if layout == 0 else sb[0]
    ldc = n if layout == 0 else m
    A = oracle.fill_uniform(m * k, dtype, seed, 0)
    B = oracle.fill_uniform(k * n, dtype, seed, 1)
    C = oracle.fill_uniform(m * n, dtype, seed, 2)
    out = C.copy()
    oracle.gemm_naive_ld(layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, out, ldc)
    meta = np.array([layout, ta, tb, m, n, k, lda, ldb, ldc], np.int64)
    return {"meta": meta, "scal": np.array([alpha, beta]), "A": A, "B": B, "C": C, "out": out}


def main():
    arrays = {}
    idx = 0
    for dtype in (np.float32, np.float64):
        for layout in (0, 1):
            for ta in (0, 1):
                for tb in (0, 1):
                    alpha, beta = [(1.0, 0.0), (1.5, 0.5), (-1.0, 1.0), (0.25, -2.0)][ta * 2 + tb]
                    c = case(dtype, layout, ta, tb, 19, 13, 11, alpha, beta, 4242 + idx)
                    for key, val in c.items():
                        arrays[f"c{idx:02d}_{key}"] = val
                    idx += 1
    c = case(np.float32, 0, 0, 0, 70, 66, 40, 1.0, 1.0, 4242 + idx)
    for key, val in c.items():
        arrays[f"c{idx:02d}_{key}"] = val
    idx += 1
    # the reference's own known answers
    ka = {"meta": np.array([0, 0, 0, 3, 3, 3, 3, 3, 3], np.int64), "scal": np.array([1.0, 0.0]),
          "A": np.arange(1, 10, dtype=np.float32), "B": (2 * np.eye(3, dtype=np.float32)).ravel(),
          "C": np.zeros(9, np.float32), "out": np.array([2, 4, 6, 8, 10, 12, 14, 16, 18],
                                                        np.float32)}
    kb = {"meta": np.array([1, 0, 0, 2, 2, 2, 2, 2, 2], np.int64), "scal": np.array([1.0, 0.0]),
          "A": np.array([1, 3, 2, 4], np.float32), "B": np.array([5, 7, 6, 8], np.float32),
          "C": np.zeros(4, np.float32), "out": np.array([19, 43, 22, 50], np.float32)}
    for c in (ka, kb):
        for key, val in c.items():
            arrays[f"c{idx:02d}_{key}"] = val
        idx += 1
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_golden.npz")
    np.savez(path, **arrays)
    print(f"wrote {idx} cases to {path}")


if __name__ == "__main__":
    main()
