"""Shared helpers for the GEMM parity tests: seeded inputs, the HIP run through
the C ABI, the oracle run on the same bits, and the normwise error.

Storage convention (BLAS, as the reference passes it to oneMKL at
src/ops/blas/level3/gemm.cpp:63/:76): op(A) is m x k, op(B) is k x n; the
stored A is (k x m if transA else m x k), laid out row- or column-major with
leading dimension lda.
"""
from __future__ import annotations

import numpy as np

import oracle

TOL = {np.float32: 1e-5, np.float64: 1e-12}


def stored_dims(trans: bool, rows: int, cols: int):
    return (cols, rows) if trans else (rows, cols)


def buffer_len(layout: int, sr: int, sc: int, ld: int) -> int:
    if sr == 0 or sc == 0:
        return 1
    return (sr - 1) * ld + sc if layout == 0 else (sc - 1) * ld + sr


def min_ld(layout: int, sr: int, sc: int) -> int:
    return max(1, sc if layout == 0 else sr)


def make_inputs(dtype, layout, ta, tb, m, n, k, seed, pad=(0, 0, 0), dist="uniform"):
    """Seeded host inputs (flat numpy buffers + leading dimensions)."""
    sa = stored_dims(ta, m, k)
    sb = stored_dims(tb, k, n)
    sc = (m, n)
    lda = min_ld(layout, *sa) + pad[0]
    ldb = min_ld(layout, *sb) + pad[1]
    ldc = min_ld(layout, *sc) + pad[2]
    gen = oracle.fill_uniform if dist == "uniform" else oracle.fill_normal
    A = gen(buffer_len(layout, *sa, lda), dtype, seed, 0)
    B = gen(buffer_len(layout, *sb, ldb), dtype, seed, 1)
    C = gen(buffer_len(layout, *sc, ldc), dtype, seed, 2)
    return A, lda, B, ldb, C, ldc


def c_window(layout, C, m, n, ldc):
    """The logical m x n result as a row-major 2-D array (copy)."""
    if m == 0 or n == 0:
        return np.zeros((m, n), C.dtype)
    if layout == 0:
        full = np.zeros(m * ldc, C.dtype)
        full[:C.size] = C
        return full.reshape(m, ldc)[:, :n].copy()
    full = np.zeros(n * ldc, C.dtype)
    full[:C.size] = C
    return full.reshape(n, ldc)[:, :m].T.copy()


def run_sbx(dev, dtype, layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
            algo=0, offsets=(0, 0, 0), epilogue=None, plan=None):
    """Copy host buffers to the GPU, run sbx_gemm_ex (sbx_gemm_fused when
    `epilogue` is given, sbx_gemm_ex_plan with the named plan when `plan`
    is), return the new host C.

    `offsets` shifts each device buffer by that many elements (to exercise
    pointers that are not 16-byte aligned)."""
    import torch
    import sushiblas_amd as sbx
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    dA = torch.zeros(A.size + offsets[0], dtype=tdt, device=dev)
    dB = torch.zeros(B.size + offsets[1], dtype=tdt, device=dev)
    dC = torch.zeros(C.size + offsets[2], dtype=tdt, device=dev)
    dA[offsets[0]:] = torch.from_numpy(A).to(dev)
    dB[offsets[1]:] = torch.from_numpy(B).to(dev)
    dC[offsets[2]:] = torch.from_numpy(C).to(dev)
    es = dA.element_size()
    ptrs = (dA.data_ptr() + es * offsets[0], dB.data_ptr() + es * offsets[1],
            dC.data_ptr() + es * offsets[2])
    code = sbx.F32 if dtype == np.float32 else sbx.F64
    if plan is not None:
        sbx.gemm_ex_plan(code, layout, ta, tb, m, n, k, alpha, ptrs[0], lda, 0, ptrs[1], ldb, 0,
                         beta, ptrs[2], ldc, 0, 1, plan)
    elif epilogue is None:
        sbx.gemm_ex(code, layout, ta, tb, m, n, k, alpha, ptrs[0], lda, 0, ptrs[1], ldb, 0,
                    beta, ptrs[2], ldc, 0, 1, algo)
    else:
        sbx.gemm_fused(code, layout, ta, tb, m, n, k, alpha, ptrs[0], lda, 0, ptrs[1], ldb, 0,
                       beta, ptrs[2], ldc, 0, 1, epilogue)
    torch.cuda.synchronize()
    return dC[offsets[2]:].cpu().numpy()


def run_oracle(layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, acc_mode=1):
    Cr = C.copy()
    oracle.gemm(layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, Cr, ldc, acc_mode)
    return Cr


def normwise(layout, X, Y, m, n, ldc) -> float:
    return oracle.rel_fro_err(c_window(layout, X, m, n, ldc), c_window(layout, Y, m, n, ldc))
