"""GPU parity of every plan the kernel-selection heuristics weigh
(sbx_gemm_plans), each run through sbx_gemm_ex_plan: every candidate tile
kernel, small-problem kernel and k-split of a problem gives the oracle's
result within the tolerance (normwise relative Frobenius error, accumulating
in double: 1e-5 fp32, 1e-12 fp64), single problems and strided batches, both
layouts, with beta != 0 so the epilogue and the split reduction read C."""
import numpy as np
import pytest

import oracle
from gemm_cases import TOL, make_inputs, normwise, run_oracle

pytestmark = pytest.mark.gpu

SEED = 20261230

SINGLE = [
    (np.float32, 0, 0, 0, 300, 200, 500),
    (np.float32, 1, 1, 0, 129, 257, 1000),
    (np.float32, 0, 0, 0, 1024, 64, 2048),
    (np.float32, 0, 1, 1, 48, 700, 1536),
    (np.float64, 0, 0, 1, 200, 96, 640),
    (np.float64, 1, 0, 0, 333, 65, 777),
]
BATCHED = [
    (np.float32, 0, 0, 0, 128, 128, 1024, 3),
    (np.float64, 1, 1, 0, 77, 130, 600, 4),
]


@pytest.mark.parametrize("case", SINGLE)
def test_every_plan_matches_the_oracle(cuda, case):
    import torch
    import sushiblas_amd as sbx
    dtype, layout, ta, tb, m, n, k = case
    code = sbx.F32 if dtype == np.float32 else sbx.F64
    A, lda, B, ldb, C, ldc = make_inputs(dtype, layout, ta, tb, m, n, k, SEED + m)
    want = run_oracle(layout, ta, tb, m, n, k, 0.75, A, lda, B, ldb, 0.5, C, ldc)
    dA, dB = torch.from_numpy(A).to(cuda), torch.from_numpy(B).to(cuda)
    plans = sbx.gemm_plans(code, layout, ta, tb, m, n, k, lda, ldb, ldc)
    print(f"plans {np.dtype(dtype).name} layout={layout} t{ta}{tb} {m}x{n}x{k}: {len(plans)}",
          flush=True)
    assert len(plans) >= 2
    for name, _ in plans:
        dC = torch.from_numpy(C).to(cuda)
        sbx.gemm_ex_plan(code, layout, ta, tb, m, n, k, 0.75, dA, lda, 0, dB, ldb, 0, 0.5, dC, ldc,
                         0, 1, name)
        torch.cuda.synchronize()
        err = normwise(layout, dC.cpu().numpy(), want, m, n, ldc)
        assert err <= TOL[dtype], (name, err)


@pytest.mark.parametrize("case", BATCHED)
def test_every_batched_plan_matches_the_oracle(cuda, case):
    import torch
    import sushiblas_amd as sbx
    dtype, layout, ta, tb, m, n, k, batch = case
    code = sbx.F32 if dtype == np.float32 else sbx.F64
    rows_a, cols_a = (m, k) if (layout == 0) == (not ta) else (k, m)
    rows_b, cols_b = (k, n) if (layout == 0) == (not tb) else (n, k)
    rows_c, cols_c = (m, n) if layout == 0 else (n, m)
    lda, ldb, ldc = cols_a, cols_b, cols_c
    sa, sb, sc = rows_a * lda, rows_b * ldb, rows_c * ldc
    A = oracle.fill_uniform(sa * batch, dtype, SEED + 7, 0)
    B = oracle.fill_uniform(sb * batch, dtype, SEED + 7, 1)
    C = oracle.fill_uniform(sc * batch, dtype, SEED + 7, 2)
    want = C.copy()
    oracle.gemm_strided_batched(layout, ta, tb, m, n, k, 1.25, A, lda, sa, B, ldb, sb, -0.5, want,
                                ldc, sc, batch, 1)
    dA, dB = torch.from_numpy(A).to(cuda), torch.from_numpy(B).to(cuda)
    plans = sbx.gemm_plans(code, layout, ta, tb, m, n, k, lda, ldb, ldc, batch)
    print(f"batched plans {np.dtype(dtype).name} {batch} x {m}x{n}x{k}: {len(plans)}", flush=True)
    assert any("+splitk" in p for p, _ in plans)
    for name, _ in plans:
        dC = torch.from_numpy(C).to(cuda)
        sbx.gemm_ex_plan(code, layout, ta, tb, m, n, k, 1.25, dA, lda, sa, dB, ldb, sb, -0.5, dC,
                         ldc, sc, batch, name)
        torch.cuda.synchronize()
        got = dC.cpu().numpy()
        for b in range(batch):
            g, w = got[b * sc:(b + 1) * sc], want[b * sc:(b + 1) * sc]
            assert normwise(layout, g, w, m, n, ldc) <= TOL[dtype], (name, b)


SYRK = [
    (np.float32, 0, 1, 0, 700, 900),    # 128^2 tiles (both), splits of the triangle
    (np.float32, 1, 0, 1, 513, 2000),
    (np.float32, 0, 0, 0, 4096, 256),   # enough triangle tiles for 256^2
    (np.float64, 0, 0, 1, 400, 1500),
    (np.float64, 1, 1, 0, 257, 640),
]


@pytest.mark.parametrize("case", SYRK)
def test_every_syrk_plan_matches_the_oracle(cuda, case):
    """sbx_syrk_plans through sbx_syrk_ex_plan: each plan gives the oracle's
    triangle within the tolerance and leaves the other triangle (NaN) as it
    was, bit for bit."""
    import torch
    import sushiblas_amd as sbx
    dtype, layout, upper, trans, n, k = case
    code = sbx.F32 if dtype == np.float32 else sbx.F64
    lda = (k if not trans else n) if layout == 0 else (n if not trans else k)
    A = oracle.fill_uniform(n * k, dtype, SEED + n, 0)
    C = oracle.fill_uniform(n * n, dtype, SEED + n, 1)
    i, j = np.tril_indices(n, -1) if upper else np.triu_indices(n, 1)
    other = i * n + j if layout == 0 else i + j * n
    C[other] = np.nan
    want = C.copy()
    oracle.syrk(layout, upper, trans, n, k, 0.75, A, lda, -0.5, want, n)
    fin = ~np.isnan(want)
    dA = torch.from_numpy(A).to(cuda)
    plans = sbx.syrk_plans(code, layout, upper, trans, n, k, lda, n)
    pick = sbx.syrk_select(code, layout, upper, trans, n, k, lda, n)
    print(f"syrk plans {np.dtype(dtype).name} layout={layout} upper={upper} trans={trans} "
          f"{n}x{k}: {len(plans)}", flush=True)
    assert pick in [p for p, _ in plans] and any("+splitk" in p for p, _ in plans)
    for name, _ in plans:
        dC = torch.from_numpy(C).to(cuda)
        sbx.syrk_ex_plan(code, layout, upper, trans, n, k, 0.75, dA, lda, 0, -0.5, dC, n, 0, 1,
                         name)
        torch.cuda.synchronize()
        got = dC.cpu().numpy()
        assert np.isnan(got[other]).all(), name
        d = got[fin].astype(np.float64) - want[fin]
        err = np.linalg.norm(d) / np.linalg.norm(want[fin].astype(np.float64))
        assert err <= TOL[dtype], (name, err)
