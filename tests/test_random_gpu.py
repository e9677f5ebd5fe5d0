"""Seeded random GEMM problems through the C ABI, each against the oracle.

Each case draws dtype, layout, transposes, m/n/k (log-uniform up to ~700,
so the oracle stays fast), leading-dimension padding, element offsets of
the base pointers (16-byte misalignment), alpha/beta (including 0), a batch
with gaps between entries, the kernel family (model's choice, tile kernels
only, small-problem kernel only, generic) and the ReLU epilogue.  The bar is
the parity tolerance of every other GEMM test (normwise 1e-5 fp32 / 1e-12
fp64 against the double-accumulating oracle, scaled by the norm before the
ReLU when there is one) on every batch entry, and every
element of C outside the m x n windows -- padding and gaps -- is unchanged.
The case is printed before it runs."""
import numpy as np
import pytest

import oracle
from gemm_cases import TOL, buffer_len, c_window, min_ld, stored_dims

pytestmark = pytest.mark.gpu

SEED = 20261215
N_CASES = 400


def _draw(rng):
    def dim():
        return int(np.exp(rng.uniform(0, np.log(700))))

    dtype = np.float32 if rng.random() < 0.65 else np.float64
    algo = int(rng.choice([0, 0, 3, 4, 1]))
    return dict(
        dtype=dtype, layout=int(rng.integers(2)), ta=int(rng.integers(2)), tb=int(rng.integers(2)),
        m=dim(), n=dim(), k=dim(),
        pad=tuple(int(x) for x in rng.choice([0, 0, 1, 3, 5], 3)),
        off=tuple(int(x) for x in rng.choice([0, 0, 1, 2, 3], 3)),
        alpha=float(rng.choice([1.0, -1.5, 0.25, 0.0], p=[0.4, 0.25, 0.25, 0.1])),
        beta=float(rng.choice([0.0, 1.0, -0.5], p=[0.4, 0.3, 0.3])),
        batch=int(rng.choice([1, 1, 2, 3])), gap=int(rng.choice([0, 2, 7])),
        algo=algo, relu=bool(rng.random() < 0.25),
    )


def _run_case(cuda, c, seed):
    import torch
    import sushiblas_amd as sbx
    dtype, layout, ta, tb = c["dtype"], c["layout"], c["ta"], c["tb"]
    m, n, k, batch = c["m"], c["n"], c["k"], c["batch"]
    sa, sb_, sc = stored_dims(ta, m, k), stored_dims(tb, k, n), (m, n)
    lda = min_ld(layout, *sa) + c["pad"][0]
    ldb = min_ld(layout, *sb_) + c["pad"][1]
    ldc = min_ld(layout, *sc) + c["pad"][2]
    la, lb, lc = (buffer_len(layout, *sa, lda), buffer_len(layout, *sb_, ldb),
                  buffer_len(layout, *sc, ldc))
    str_a, str_b, str_c = la + c["gap"], lb + c["gap"], lc + c["gap"]
    A = oracle.fill_uniform(str_a * batch, dtype, seed, 0)
    B = oracle.fill_uniform(str_b * batch, dtype, seed, 1)
    C = oracle.fill_uniform(str_c * batch, dtype, seed, 2)
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    es = 4 if dtype == np.float32 else 8
    dev = []
    for x, o in zip((A, B, C), c["off"]):
        t = torch.zeros(x.size + o, dtype=tdt, device=cuda)
        t[o:] = torch.from_numpy(x).to(cuda)
        dev.append(t)
    ptrs = [t.data_ptr() + o * es for t, o in zip(dev, c["off"])]
    code = sbx.F32 if dtype == np.float32 else sbx.F64
    sab = (str_a, str_b, str_c) if batch > 1 else (0, 0, 0)
    if c["relu"]:
        sbx.gemm_fused(code, layout, ta, tb, m, n, k, c["alpha"], ptrs[0], lda, sab[0], ptrs[1], ldb,
                       sab[1], c["beta"], ptrs[2], ldc, sab[2], batch)
    else:
        sbx.gemm_ex(code, layout, ta, tb, m, n, k, c["alpha"], ptrs[0], lda, sab[0], ptrs[1], ldb,
                    sab[1], c["beta"], ptrs[2], ldc, sab[2], batch, algo=c["algo"])
    torch.cuda.synchronize()
    got = dev[2].cpu().numpy()[c["off"][2]:]
    want = C.copy()
    oracle.gemm_strided_batched(layout, ta, tb, m, n, k, c["alpha"], A, lda, str_a, B, ldb, str_b,
                                c["beta"], want, ldc, str_c, batch, 1)
    inside = np.zeros(C.size, bool)
    for b in range(batch):
        g = c_window(layout, got[b * str_c:b * str_c + lc], m, n, ldc)
        w = c_window(layout, want[b * str_c:b * str_c + lc], m, n, ldc)
        # ReLU is 1-Lipschitz, so the GEMM's normwise bound carries over with
        # the pre-activation norm as its scale (relative to the post-ReLU
        # norm, one surviving output near zero after cancellation would be
        # held to an absolute error far below fp32 rounding)
        scale = float(np.linalg.norm(w.astype(np.float64)))
        if c["relu"]:
            oracle.relu(w)
            assert not np.signbit(g).any()
        if scale > 0:
            err = float(np.linalg.norm(g.astype(np.float64) - w.astype(np.float64))) / scale
            assert err <= TOL[dtype], (b, err)
        else:
            assert np.array_equal(g, w), b
        idx = np.arange(lc)
        inside[b * str_c:b * str_c + lc] = (idx % ldc) < (n if layout == 0 else m)
    np.testing.assert_array_equal(got[~inside], C[~inside])


def test_random_problems(cuda):
    import sushiblas_amd as sbx
    rng = np.random.default_rng(SEED)
    for i in range(N_CASES):
        c = _draw(rng)
        # the kernel the model picks, for the log
        name = "generic" if c["algo"] == 1 else "?"
        if c["algo"] == 0 and not c["relu"]:
            sa, sb_ = stored_dims(c["ta"], c["m"], c["k"]), stored_dims(c["tb"], c["k"], c["n"])
            lda = min_ld(c["layout"], *sa) + c["pad"][0]
            ldb = min_ld(c["layout"], *sb_) + c["pad"][1]
            ldc = min_ld(c["layout"], c["m"], c["n"]) + c["pad"][2]
            name = sbx.gemm_select(sbx.F32 if c["dtype"] == np.float32 else sbx.F64, c["layout"],
                                   c["ta"], c["tb"], c["m"], c["n"], c["k"], lda, ldb, ldc)
        print(f"random case {i}: {np.dtype(c['dtype']).name} layout={c['layout']} "
              f"t{c['ta']}{c['tb']} {c['m']}x{c['n']}x{c['k']} pad={c['pad']} off={c['off']} "
              f"alpha={c['alpha']} beta={c['beta']} batch={c['batch']} gap={c['gap']} "
              f"algo={c['algo']} relu={c['relu']} kernel={name}", flush=True)
        _run_case(cuda, c, SEED + i)
