"""Seeded random GEMM problems at the sizes where the large tiles, the wide
splits and the three-per-CU tile run, each against the oracle.

The cases of test_random_gpu.py stay below ~700 per dimension, where the
small-problem kernel and the 128^2 and 64-wide tiles run.  Here m and n are
drawn log-uniform from 256 to 8192 and k from 64 to 16384; about one case
in six is tall-skinny (n <= 64, m from 32768 to 131072) and one in four has
m and n from 3500 to 8192 (the large-tile grids).  m*n*k is capped so the
oracle finishes each case in about a second.  Every case has a
random layout, transposes, leading-dimension padding, element offsets of
the base pointers, alpha/beta and ReLU, and runs through the model's choice
(so the 256x128, 256x64, three-per-CU 128^2 tiles, splits of up to 32 parts
and C rows without vector access all occur).  The bar and the check of the
memory outside the m x n window are those of test_random_gpu.py."""
import numpy as np
import pytest

from gemm_cases import min_ld, stored_dims
from test_random_gpu import _run_case

pytestmark = pytest.mark.gpu

SEED = 20261216
N_CASES = 48
MAX_MNK = 4e10


def _draw(rng):
    def dim(lo, hi):
        return int(np.exp(rng.uniform(np.log(lo), np.log(hi))))

    while True:
        m, n, k = dim(256, 8192), dim(256, 8192), dim(64, 16384)
        mode = rng.random()
        if mode < 0.17:
            n = int(rng.integers(1, 65))  # tall-skinny
            m = dim(32768, 131072)
        elif mode < 0.45:
            m, n = dim(3500, 8192), dim(3500, 8192)  # the large-tile grids
            k = dim(64, max(65, MAX_MNK / (m * n)))
        if m * n * k <= MAX_MNK:
            break
    return dict(
        dtype=np.float32 if rng.random() < 0.75 else np.float64,
        layout=int(rng.integers(2)), ta=int(rng.integers(2)), tb=int(rng.integers(2)),
        m=m, n=n, k=k,
        pad=tuple(int(x) for x in rng.choice([0, 0, 1, 3, 5], 3)),
        off=tuple(int(x) for x in rng.choice([0, 0, 1, 2, 3], 3)),
        alpha=float(rng.choice([1.0, -1.5, 0.25])),
        beta=float(rng.choice([0.0, 1.0, -0.5], p=[0.4, 0.3, 0.3])),
        batch=1, gap=0, algo=0, relu=bool(rng.random() < 0.2),
    )


def test_random_large_problems(cuda):
    import sushiblas_amd as sbx
    rng = np.random.default_rng(SEED)
    for i in range(N_CASES):
        c = _draw(rng)
        sa, sb_ = stored_dims(c["ta"], c["m"], c["k"]), stored_dims(c["tb"], c["k"], c["n"])
        lda = min_ld(c["layout"], *sa) + c["pad"][0]
        ldb = min_ld(c["layout"], *sb_) + c["pad"][1]
        ldc = min_ld(c["layout"], c["m"], c["n"]) + c["pad"][2]
        name = sbx.gemm_select(sbx.F32 if c["dtype"] == np.float32 else sbx.F64, c["layout"],
                               c["ta"], c["tb"], c["m"], c["n"], c["k"], lda, ldb, ldc)
        print(f"large random case {i}: {np.dtype(c['dtype']).name} layout={c['layout']} "
              f"t{c['ta']}{c['tb']} {c['m']}x{c['n']}x{c['k']} pad={c['pad']} off={c['off']} "
              f"alpha={c['alpha']} beta={c['beta']} relu={c['relu']} kernel={name}", flush=True)
        _run_case(cuda, c, SEED + i)
