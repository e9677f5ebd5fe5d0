"""Host-side checks of the plan entry points (include/sbx.h sbx_gemm_plans,
sbx_gemm_ex_plan, sbx_syrk_plans, sbx_syrk_ex_plan): the enumeration holds
the heuristics' pick, and names that are no plan, or plans the problem cannot
use, are refused before any device call."""
import ctypes

import pytest

import sushiblas_amd as sbx

SHAPES = [
    (sbx.F32, 0, 0, 0, 8192, 8192, 8192, 1), (sbx.F32, 0, 1, 0, 4095, 3001, 2047, 1),
    (sbx.F32, 0, 0, 0, 65536, 64, 4096, 1), (sbx.F32, 0, 0, 0, 512, 512, 512, 1),
    (sbx.F64, 0, 0, 0, 8192, 8192, 8192, 1), (sbx.F64, 1, 1, 0, 300, 200, 5000, 3),
    (sbx.F32, 1, 0, 1, 1536, 1536, 1024, 1), (sbx.F32, 0, 0, 0, 128, 128, 4096, 8),
]


def _lds(layout, ta, tb, m, n, k):
    lda = (k if not ta else m) if layout == 0 else (m if not ta else k)
    ldb = (n if not tb else k) if layout == 0 else (k if not tb else n)
    ldc = n if layout == 0 else m
    return lda, ldb, ldc


@pytest.mark.parametrize("shape", SHAPES)
def test_plans_hold_the_pick(shape):
    dtype, layout, ta, tb, m, n, k, batch = shape
    lda, ldb, ldc = _lds(layout, ta, tb, m, n, k)
    plans = sbx.gemm_plans(dtype, layout, ta, tb, m, n, k, lda, ldb, ldc, batch)
    names = [p for p, _ in plans]
    assert len(names) == len(set(names)) and all(us > 0 for _, us in plans)
    pick = sbx.gemm_select(dtype, layout, ta, tb, m, n, k, lda, ldb, ldc, batch=batch)
    assert pick in names, (pick, names)
    tag = "_f32_" if dtype == sbx.F32 else "_f64_"
    assert all(tag in p for p in names)


def _plan_call(plan, dtype=sbx.F32, m=64, n=64, k=64):
    one = ctypes.c_double(1.0) if dtype == sbx.F64 else ctypes.c_float(1.0)
    return sbx.lib().sbx_gemm_ex_plan(0, dtype, 0, 0, 0, m, n, k, ctypes.byref(one), 16, k, 0,
                                      16, n, 0, ctypes.byref(one), 16, n, 0, 1,
                                      plan.encode() if plan is not None else None)


@pytest.mark.parametrize("plan", [None, "", "no_such_kernel", "mfma_f32_128x128x16_w2x2+splitk",
                                  "mfma_f32_128x128x16_w2x2+splitk1",
                                  "mfma_f32_128x128x16_w2x2+splitk33",
                                  "mfma_f32_128x128x16_w2x2+splitk3x",
                                  "mfma_f32_128x128x16_w2x2 "])
def test_names_that_are_no_plan(plan):
    assert _plan_call(plan) == 1  # SBX_INVALID_ARGUMENT


def test_plans_the_problem_cannot_use():
    # an fp64 kernel for an fp32 problem
    assert _plan_call("mfma_f64_128x128x16_w2x2") == 2
    # 64 x 64 x 64 on 128^2 tiles has 4 k tiles of 16: at most 2 k-ranges
    assert _plan_call("mfma_f32_128x128x16_w2x2+splitk3") == 2
    # an empty problem is a no-op whatever the plan
    assert _plan_call("mfma_f32_128x128x16_w2x2", m=0) == 0


SYRK_SHAPES = [(sbx.F32, 0, 0, 0, 8192, 8192), (sbx.F64, 0, 1, 1, 8192, 8192),
               (sbx.F32, 1, 1, 0, 2000, 500), (sbx.F32, 0, 0, 1, 4096, 1024),
               (sbx.F64, 1, 0, 0, 300, 5000)]


@pytest.mark.parametrize("shape", SYRK_SHAPES)
def test_syrk_plans_hold_the_pick(shape):
    dtype, layout, upper, trans, n, k = shape
    lda = (k if not trans else n) if layout == 0 else (n if not trans else k)
    plans = sbx.syrk_plans(dtype, layout, upper, trans, n, k, lda, n)
    names = [p for p, _ in plans]
    assert len(names) == len(set(names)) and all(us > 0 for _, us in plans)
    assert sbx.syrk_select(dtype, layout, upper, trans, n, k, lda, n) in names
    # only square tiles cover a triangle
    assert all(p.split("_")[2].split("x")[0] == p.split("_")[2].split("x")[1] for p in names)


def _syrk_plan_call(plan, n=64, k=64):
    one = ctypes.c_float(1.0)
    return sbx.lib().sbx_syrk_ex_plan(0, sbx.F32, 0, 0, 0, n, k, ctypes.byref(one), 16, k, 0,
                                      ctypes.byref(one), 16, max(n, 1), 0, 1, plan.encode())


def test_syrk_plans_the_triangle_cannot_use():
    assert _syrk_plan_call("no_such_kernel") == 1
    # rectangular tiles, the small-problem kernel and fp64 tiles do not cover it
    for plan in ("mfma_f32_128x64x32_w2x2", "mfma_f32_32x32_ksplit4", "mfma_f64_128x128x16_w2x2"):
        assert _syrk_plan_call(plan) == 2, plan
    assert _syrk_plan_call("mfma_f32_128x128x16_w2x2", n=0) == 0


def test_pick_cache_returns_what_the_model_picks():
    """The per-thread cache of recent picks: cycling through more problems
    than it holds (so entries are evicted and refilled), and through
    problems that differ in one key field only, gives the same picks as a
    first, cold pass, and sbx_gemm_plans (never cached) still holds each."""
    shapes = [(sbx.F32, 0, 0, 0, m, n, k, 1) for m, n, k in
              [(512, 512, 512), (513, 512, 512), (512, 513, 512), (512, 512, 513),
               (8192, 8192, 8192), (65536, 64, 4096), (4095, 3001, 2047), (1536, 1536, 1024),
               (300, 200, 5000), (1024, 1024, 1024), (2048, 2048, 2048)]]
    shapes += [(sbx.F64, 0, 0, 0, 512, 512, 512, 1), (sbx.F32, 0, 1, 0, 512, 512, 512, 1),
               (sbx.F32, 1, 0, 0, 512, 512, 512, 1), (sbx.F32, 0, 0, 0, 128, 128, 4096, 8)]
    first = {}
    for rep in range(3):
        for sh in shapes:
            dtype, layout, ta, tb, m, n, k, batch = sh
            lda, ldb, ldc = _lds(layout, ta, tb, m, n, k)
            pick = sbx.gemm_select(dtype, layout, ta, tb, m, n, k, lda, ldb, ldc, batch=batch)
            if rep == 0:
                first[sh] = pick
                plans = [p for p, _ in sbx.gemm_plans(dtype, layout, ta, tb, m, n, k, lda, ldb,
                                                      ldc, batch)]
                assert pick in plans, (sh, pick)
            assert pick == first[sh], (rep, sh, pick, first[sh])
