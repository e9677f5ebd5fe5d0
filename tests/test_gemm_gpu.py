"""GPU parity tests: the HIP GEMM kernels, called through the C ABI
(include/sbx.h), against the CPU oracle on identical seeded inputs.

Bar (from the task's tolerance): normwise relative Frobenius error
||C_gpu - C_oracle||_F / ||C_oracle||_F <= 1e-5 (fp32) and <= 1e-12 (fp64),
oracle accumulating in double.  Known answers are checked exactly.
"""
import math

import numpy as np
import pytest

import oracle
from gemm_cases import (TOL, c_window, make_inputs, normwise, run_oracle, run_sbx)

pytestmark = pytest.mark.gpu

SEED = 20261201


def _case(dev, dtype, layout, ta, tb, m, n, k, alpha, beta, seed, algo=0, pad=(0, 0, 0),
          offsets=(0, 0, 0), dist="uniform", plan=None):
    A, lda, B, ldb, C, ldc = make_inputs(dtype, layout, ta, tb, m, n, k, seed, pad, dist)
    got = run_sbx(dev, dtype, layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                  algo, offsets, plan=plan)
    want = run_oracle(layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
    err = normwise(layout, got, want, m, n, ldc)
    print(f"case dtype={np.dtype(dtype).name} layout={layout} tA={ta} tB={tb} "
          f"m={m} n={n} k={k} alpha={alpha} beta={beta} algo={algo} err={err:.3e}", flush=True)
    return err, got, want


# -- reference known answers (tests/blas/level3/test_gemm.cpp:39-88) --------

def test_known_answer_3x3_row_major(cuda):
    """SimpleGEMM3x3: A = [1..9], B = 2*I, beta = 0 -> C = 2*A (exact)."""
    A = np.arange(1, 10, dtype=np.float32)
    B = (2 * np.eye(3, dtype=np.float32)).ravel()
    C = np.zeros(9, np.float32)
    got = run_sbx(cuda, np.float32, 0, 0, 0, 3, 3, 3, 1.0, A, 3, B, 3, 0.0, C, 3)
    assert got.tolist() == [2, 4, 6, 8, 10, 12, 14, 16, 18]


def test_known_answer_2x2_column_major(cuda):
    """SimpleGEMMColumnMajor: memory [1,3,2,4] x [5,7,6,8] -> [19,43,22,50]."""
    A = np.array([1, 3, 2, 4], np.float32)
    B = np.array([5, 7, 6, 8], np.float32)
    C = np.zeros(4, np.float32)
    got = run_sbx(cuda, np.float32, 1, 0, 0, 2, 2, 2, 1.0, A, 2, B, 2, 0.0, C, 2)
    assert got.tolist() == [19, 43, 22, 50]


# -- BASELINE configurations ---------------------------------------------------

def test_cfg1_fp32_512(cuda):
    """fp32 512^3, row-major, alpha=1, beta=0, U[-1,1]."""
    err, got, want = _case(cuda, np.float32, 0, 0, 0, 512, 512, 512, 1.0, 0.0, SEED + 1)
    assert err <= TOL[np.float32]
    # also against the oracle accumulating in fp32, as a vendor sgemm does
    A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, 0, 0, 512, 512, 512, SEED + 1)
    native = run_oracle(0, 0, 0, 512, 512, 512, 1.0, A, lda, B, ldb, 0.0, C, ldc, acc_mode=0)
    assert normwise(0, got, native, 512, 512, ldc) <= TOL[np.float32]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_cfg3_ragged_all_transposes(cuda, ta, tb):
    """fp32 M=4095, N=3001, K=2047, alpha=beta=1, every transA/transB (masked edges)."""
    err, _, _ = _case(cuda, np.float32, 0, ta, tb, 4095, 3001, 2047, 1.0, 1.0, SEED + 3)
    assert err <= TOL[np.float32]


def test_cfg4_tall_skinny(cuda):
    """fp32 M=65536, K=4096, N=64, A ~ N(0,1), B ~ N(0,1)/sqrt(K): full oracle check."""
    import torch
    import sushiblas_amd as sbx
    m, n, k = 65536, 64, 4096
    A = oracle.fill_normal(m * k, np.float32, SEED + 4, 0)
    B = oracle.fill_normal(k * n, np.float32, SEED + 4, 1, 1.0 / math.sqrt(k))
    C = np.full(m * n, np.nan, np.float32)  # beta = 0: C must not be read
    got = run_sbx(cuda, np.float32, 0, 0, 0, m, n, k, 1.0, A, k, B, n, 0.0, C, n)
    want = run_oracle(0, 0, 0, m, n, k, 1.0, A, k, B, n, 0.0, C, n)
    assert not np.isnan(got).any()
    err = normwise(0, got, want, m, n, n)
    print(f"tall-skinny err={err:.3e} kernel="
          f"{sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n)}")
    assert err <= TOL[np.float32]
    del torch


def _sampled_rows_check(cuda, dtype, m, n, k, alpha, beta, seed, dist_c, all_rows=False, ta=0):
    """Full-size GEMM on the GPU; the oracle (accumulating in double) on a
    sample of rows -- or on every row with all_rows -- plus a Freivalds
    projection of the whole result (C_gpu x vs alpha op(A) (B x) + beta C0 x).
    ta=1: A is stored k x m (lda = m) and op(A) is its transpose."""
    import torch
    import sushiblas_amd as sbx
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    dA = torch.empty(m * k, dtype=tdt, device=cuda)
    dB = torch.empty(k * n, dtype=tdt, device=cuda)
    dC = torch.empty(m * n, dtype=tdt, device=cuda)
    sbx.fill_uniform(dA, seed, 0)
    sbx.fill_uniform(dB, seed, 1)
    if dist_c == "normal":
        sbx.fill_normal(dC, seed, 2)
    else:
        sbx.fill_uniform(dC, seed, 2)
    torch.cuda.synchronize()
    A = dA.cpu().numpy()
    B = dB.cpu().numpy()
    C0 = dC.cpu().numpy()
    sbx.gemm_ex(sbx.F32 if dtype == np.float32 else sbx.F64, 0, ta, 0, m, n, k, alpha, dA,
                m if ta else k, 0, dB, n, 0, beta, dC, n, 0)
    torch.cuda.synchronize()
    got = dC.cpu().numpy().reshape(m, n)
    opA = A.reshape(k, m).T if ta else A.reshape(m, k)
    if all_rows:
        rows = np.arange(m)
    else:
        rows = np.unique(np.concatenate([np.arange(0, 16), np.arange(m - 16, m),
                                         np.random.default_rng(seed).integers(0, m, 32)]))
    Ar = np.ascontiguousarray(opA[rows]).ravel()
    Cr = np.ascontiguousarray(C0.reshape(m, n)[rows]).ravel()
    oracle.gemm(0, 0, 0, len(rows), n, k, alpha, Ar, k, B, n, beta, Cr, n, 1)
    err_rows = oracle.rel_fro_err(np.ascontiguousarray(got[rows]), Cr.reshape(len(rows), n))
    x = np.random.default_rng(seed + 7).standard_normal(n)
    lhs = got.astype(np.float64) @ x
    rhs = alpha * (opA.astype(np.float64) @ (B.reshape(k, n).astype(np.float64) @ x))
    rhs += beta * (C0.reshape(m, n).astype(np.float64) @ x)
    err_proj = float(np.linalg.norm(lhs - rhs) / np.linalg.norm(rhs))
    print(f"{m}x{n}x{k} {np.dtype(dtype).name}: {len(rows)} rows err={err_rows:.3e} "
          f"Freivalds err={err_proj:.3e}", flush=True)
    return err_rows, err_proj


def test_cfg2_fp32_8192(cuda):
    """fp32 8192^3, alpha=1.5, beta=0.5, C ~ N(0,1): the whole matrix against
    the oracle, plus Freivalds."""
    e_rows, e_proj = _sampled_rows_check(cuda, np.float32, 8192, 8192, 8192, 1.5, 0.5,
                                         SEED + 2, "normal", all_rows=True)
    assert e_rows <= TOL[np.float32]
    assert e_proj <= TOL[np.float32]


def test_cfg5_fp64_8192(cuda):
    """fp64 8192^3, alpha=1, beta=0: the whole matrix against the oracle, plus
    Freivalds, tolerance 1e-12."""
    e_rows, e_proj = _sampled_rows_check(cuda, np.float64, 8192, 8192, 8192, 1.0, 0.0,
                                         SEED + 5, "uniform", all_rows=True)
    assert e_rows <= TOL[np.float64]
    assert e_proj <= TOL[np.float64]


def test_operand_above_2gib(cuda):
    """An A of 2.25 GiB (147456 x 4096 fp32) through the MFMA tile path: the
    buffer descriptor's record count saturates at 2^31 - 16 bytes, so tiles
    past 2 GiB must be reached through the per-tile moving base.  Sampled
    rows (including the last 16) against the oracle, plus Freivalds over the
    whole result."""
    import sushiblas_amd as sbx
    m, n, k = 147456, 64, 4096
    assert m * k * 4 > (2 << 30)
    name = sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n)
    print(f"above-2GiB case {m}x{n}x{k} -> {name}", flush=True)
    assert name.startswith("mfma_"), name
    e_rows, e_proj = _sampled_rows_check(cuda, np.float32, m, n, k, 1.0, 0.5, SEED + 6,
                                         "uniform")
    assert e_rows <= TOL[np.float32]
    assert e_proj <= TOL[np.float32]


def test_operand_above_2gib_transposed(cuda):
    """The same 2.25 GiB A stored transposed (4096 x 147456, lda = 147456):
    a tile's walk over K then spans more than 2^31 bytes from the tile's
    origin, so the k loop cannot use its fixed-descriptor section and every
    k tile goes through the moving descriptors.  Sampled rows against the
    oracle, plus Freivalds over the whole result."""
    import sushiblas_amd as sbx
    m, n, k = 147456, 64, 4096
    assert m * k * 4 > (2 << 30)
    name = sbx.gemm_select(sbx.F32, 0, 1, 0, m, n, k, m, n, n)
    print(f"above-2GiB transposed case {m}x{n}x{k} -> {name}", flush=True)
    assert name.startswith("mfma_"), name
    e_rows, e_proj = _sampled_rows_check(cuda, np.float32, m, n, k, 1.0, 0.5, SEED + 7,
                                         "uniform", ta=1)
    assert e_rows <= TOL[np.float32]
    assert e_proj <= TOL[np.float32]


# -- coverage sweeps -----------------------------------------------------------

SHAPES = [(1, 1, 1), (3, 5, 7), (64, 64, 64), (100, 37, 129), (257, 300, 45), (37, 1000, 300),
          (1000, 50, 300), (515, 301, 257)]


@pytest.mark.parametrize("algo", [0, 3, 4])  # model's choice, tile kernels only, small kernel only
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sweep_shapes_layouts_transposes(cuda, dtype, layout, ta, tb, algo):
    for i, (m, n, k) in enumerate(SHAPES):
        alpha, beta = (1.0, 0.0) if i % 2 == 0 else (-0.75, 1.25)
        err, _, _ = _case(cuda, dtype, layout, ta, tb, m, n, k, alpha, beta, SEED + 10 + i,
                          algo=algo)
        assert err <= TOL[dtype], (m, n, k)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_generic_path_matches(cuda, dtype, ta, tb):
    """The non-MFMA fallback kernel, forced through the algo override."""
    for m, n, k in [(129, 77, 65), (300, 200, 100)]:
        err, _, _ = _case(cuda, dtype, 0, ta, tb, m, n, k, 1.5, -0.5, SEED + 30, algo=1)
        assert err <= TOL[dtype]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_padded_ld_and_unaligned_pointers(cuda, dtype):
    """ld larger than the minimum and base pointers off 16-byte alignment
    (16-byte operand loads at 4/8-byte aligned addresses)."""
    for ta, tb in [(0, 0), (1, 0), (0, 1), (1, 1)]:
        err, _, _ = _case(cuda, dtype, 0, ta, tb, 260, 196, 132, 1.0, 0.5, SEED + 40,
                          pad=(3, 5, 7), offsets=(1, 3, 1))
        assert err <= TOL[dtype]
        err, _, _ = _case(cuda, dtype, 0, ta, tb, 256, 256, 128, 1.0, 0.0, SEED + 41,
                          pad=(4, 8, 4))
        assert err <= TOL[dtype]


def _poison_padding(X, layout, sr, sc, ld):
    """Set every element of a stored sr x sc matrix's buffer that lies outside
    the matrix (the ld padding) to NaN."""
    idx = np.arange(X.size)
    inner = idx % ld < (sc if layout == 0 else sr)
    X[~inner] = np.nan


@pytest.mark.parametrize("algo", [3, 4])  # tile kernels / small kernel
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_vector_loads_past_k_and_edges_ignore_padding(cuda, dtype, layout, ta, tb, algo):
    """Operands are read in 16-byte vectors at any alignment.  A vector that
    straddles K reads the ld padding (NaN here) and must zero it; one that
    straddles M or N feeds only C entries that are never stored.  Odd K,
    padded ld, bases off 16-byte alignment, every tile shape."""
    from gemm_cases import stored_dims
    shapes = [(129, 67, 37), (300, 257, 301), (1001, 63, 303), (61, 1003, 305), (130, 67, 64)]
    if dtype == np.float32 and algo == 3:
        shapes.append((4095, 3001, 97))  # three-per-CU 128x128 tile
    for i, (m, n, k) in enumerate(shapes):
        A, lda, B, ldb, C, ldc = make_inputs(dtype, layout, ta, tb, m, n, k, SEED + 45 + i,
                                             pad=(3, 1, 2))
        _poison_padding(A, layout, *stored_dims(ta, m, k), lda)
        _poison_padding(B, layout, *stored_dims(tb, k, n), ldb)
        got = run_sbx(cuda, dtype, layout, ta, tb, m, n, k, 1.0, A, lda, B, ldb, 0.5, C, ldc,
                      algo=algo, offsets=(1, 3, 1))
        want = run_oracle(layout, ta, tb, m, n, k, 1.0, A, lda, B, ldb, 0.5, C, ldc)
        gw, ww = c_window(layout, got, m, n, ldc), c_window(layout, want, m, n, ldc)
        print(f"padding-NaN case {np.dtype(dtype).name} layout={layout} t{ta}{tb} {m}x{n}x{k}",
              flush=True)
        assert np.isfinite(gw).all(), (m, n, k)
        assert oracle.rel_fro_err(gw, ww) <= TOL[dtype], (m, n, k)
        # C's own padding is never written
        cpad = np.arange(C.size) % ldc >= (n if layout == 0 else m)
        np.testing.assert_array_equal(got[cpad], C[cpad])


# -- BLAS edge semantics ------------------------------------------------------

@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_beta_zero_ignores_nan_in_c(cuda, dtype):
    A, lda, B, ldb, C, ldc = make_inputs(dtype, 0, 0, 0, 300, 300, 64, SEED + 50)
    C[:] = np.nan
    got = run_sbx(cuda, dtype, 0, 0, 0, 300, 300, 64, 1.0, A, lda, B, ldb, 0.0, C, ldc)
    assert not np.isnan(got).any()
    want = run_oracle(0, 0, 0, 300, 300, 64, 1.0, A, lda, B, ldb, 0.0, C, ldc)
    assert normwise(0, got, want, 300, 300, ldc) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_alpha_zero_and_k_zero_scale_c(cuda, dtype):
    A, lda, B, ldb, C, ldc = make_inputs(dtype, 0, 0, 0, 70, 90, 33, SEED + 51)
    A[:] = np.nan  # alpha == 0: A and B are not read
    got = run_sbx(cuda, dtype, 0, 0, 0, 70, 90, 33, 0.0, A, lda, B, ldb, 2.0, C, ldc)
    np.testing.assert_array_equal(got, (2.0 * C).astype(dtype))
    got = run_sbx(cuda, dtype, 0, 0, 0, 70, 90, 0, 1.0, A, lda, B, ldb, -0.5, C, ldc)
    np.testing.assert_array_equal(got, (-0.5 * C).astype(dtype))
    Cn = C.copy()
    Cn[:] = np.nan
    got = run_sbx(cuda, dtype, 0, 0, 0, 70, 90, 0, 1.0, A, lda, B, ldb, 0.0, Cn, ldc)
    assert (got == 0).all()


def test_empty_m_or_n_is_noop(cuda):
    A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, 0, 0, 4, 4, 4, SEED + 52)
    got = run_sbx(cuda, np.float32, 0, 0, 0, 0, 4, 4, 1.0, A, lda, B, ldb, 0.0, C, ldc)
    np.testing.assert_array_equal(got, C)
    got = run_sbx(cuda, np.float32, 0, 0, 0, 4, 0, 4, 1.0, A, lda, B, ldb, 0.0, C, ldc)
    np.testing.assert_array_equal(got, C)


# -- strided batched (gemm.cpp:55-58, :68-72) ---------------------------------

@pytest.mark.parametrize("algo", [3, 4])  # tile kernels / small kernel
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("layout", [0, 1])
def test_strided_batched(cuda, dtype, layout, algo):
    import torch
    import sushiblas_amd as sbx
    batch, m, n, k = 5, 97, 130, 71
    ta, tb = 1, 0
    sa = (k, m) if ta else (m, k)
    sb = (n, k) if tb else (k, n)
    lda = sa[1] if layout == 0 else sa[0]
    ldb = sb[1] if layout == 0 else sb[0]
    ldc = n if layout == 0 else m
    str_a, str_b, str_c = sa[0] * sa[1] + 3, sb[0] * sb[1] + 1, m * n + 2
    A = oracle.fill_uniform(batch * str_a, dtype, SEED + 60, 0)
    B = oracle.fill_uniform(batch * str_b, dtype, SEED + 60, 1)
    C = oracle.fill_uniform(batch * str_c, dtype, SEED + 60, 2)
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    dA, dB, dC = (torch.from_numpy(x).to(cuda) for x in (A, B, C))
    sbx.gemm_ex(sbx.F32 if dtype == np.float32 else sbx.F64, layout, ta, tb, m, n, k, 0.5, dA,
                lda, str_a, dB, ldb, str_b, 1.5, dC, ldc, str_c, batch, algo=algo)
    torch.cuda.synchronize()
    got = dC.cpu().numpy()
    want = C.copy()
    oracle.gemm_strided_batched(layout, ta, tb, m, n, k, 0.5, A, lda, str_a, B, ldb, str_b, 1.5,
                                want, ldc, str_c, batch, 1)
    for b in range(batch):
        g = c_window(layout, got[b * str_c:b * str_c + m * n], m, n, ldc)
        w = c_window(layout, want[b * str_c:b * str_c + m * n], m, n, ldc)
        assert oracle.rel_fro_err(g, w) <= TOL[dtype]
    # padding between batch entries is untouched
    for b in range(batch):
        np.testing.assert_array_equal(got[b * str_c + m * n:(b + 1) * str_c],
                                      C[b * str_c + m * n:(b + 1) * str_c])
    del tdt


def test_batched_broadcast_b(cuda):
    """str_b = 0: every batch entry multiplies by the same B."""
    import torch
    import sushiblas_amd as sbx
    batch, m, n, k = 4, 64, 96, 48
    A = oracle.fill_uniform(batch * m * k, np.float32, SEED + 61, 0)
    B = oracle.fill_uniform(k * n, np.float32, SEED + 61, 1)
    C = np.zeros(batch * m * n, np.float32)
    dA, dB, dC = (torch.from_numpy(x).to(cuda) for x in (A, B, C))
    sbx.gemm_ex(sbx.F32, 0, 0, 0, m, n, k, 1.0, dA, k, m * k, dB, n, 0, 0.0, dC, n, m * n, batch)
    torch.cuda.synchronize()
    got = dC.cpu().numpy()
    for b in range(batch):
        want = np.zeros(m * n, np.float32)
        oracle.gemm(0, 0, 0, m, n, k, 1.0, A[b * m * k:(b + 1) * m * k], k, B, n, 0.0, want, n, 1)
        assert oracle.rel_fro_err(got[b * m * n:(b + 1) * m * n].reshape(m, n),
                                  want.reshape(m, n)) <= 1e-5


# -- closed forms from the reference's integration tests ----------------------

def test_parallel_batched_inference_closed_form(cuda):
    """test_framework_sim.cpp:75-128: X = 1 (256x256), W = 2 (256x512) -> Y = 512,
    24 independent models (run here as one strided batch)."""
    import torch
    import sushiblas_amd as sbx
    models, m, n, k = 24, 256, 512, 256
    X = torch.ones(models, m, k, device=cuda)
    W = torch.full((models, k, n), 2.0, device=cuda)
    Y = torch.empty(models, m, n, device=cuda)
    sbx.gemm_ex(sbx.F32, 0, 0, 0, m, n, k, 1.0, X, k, m * k, W, n, k * n, 0.0, Y, n, m * n,
                models)
    torch.cuda.synchronize()
    assert bool((Y == 512.0).all())


def test_deep_forward_pass_closed_form(cuda):
    """test_framework_sim.cpp:10-73: X = 1 (512x1024), W_i = 0.01 (1024x1024),
    10 layers, ReLU between (identity on these positive values): every entry
    of layer L is (1024 * fp32(0.01))^L up to fp32 rounding -- each layer sums
    1024 products in fp32, a relative error of at most ~1024 * 2^-24 = 6e-5
    per layer in the worst case."""
    import torch
    import sushiblas_amd as sbx
    b, f = 512, 1024
    H = torch.ones(b, f, device=cuda)
    W = torch.full((f, f), 0.01, device=cuda)
    for layer in range(1, 11):
        Hn = torch.empty(b, f, device=cuda)
        sbx.sgemm(0, 0, 0, b, f, f, 1.0, H, f, W, f, 0.0, Hn, f)
        if layer < 10:
            Hn = torch.relu(Hn)
        H = Hn
        torch.cuda.synchronize()
        expect = (1024 * np.float64(np.float32(0.01))) ** layer
        rel = float((H.double() - expect).abs().max() / expect)
        assert rel < 6.2e-5 * layer, (layer, rel)


# -- three workgroups per CU --------------------------------------------------

@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_three_per_cu_tile_whole_and_split(cuda, layout, ta, tb):
    """The 128x128 fp32 tile compiled for three workgroups per CU (run by
    name, sbx_gemm_ex_plan): 768 ragged tiles in one round (scalar loads, odd
    ld) and, at 3584^2 x 512, a full round plus a tail split six ways."""
    for i, (m, n, k, beta, plan) in enumerate([
            (4095, 3001, 96, 1.0, "mfma_f32_128x128x16_w2x2_o3"),
            (3584, 3584, 512, 0.5, "mfma_f32_128x128x16_w2x2_o3+splitk6")]):
        print(f"three-per-CU case {m}x{n}x{k} -> {plan}", flush=True)
        err, _, _ = _case(cuda, np.float32, layout, ta, tb, m, n, k, 1.0, beta, SEED + 60 + i,
                          plan=plan)
        assert err <= TOL[np.float32], (m, n, k, plan)


# -- the small-problem kernel with K cut over 8 waves ---------------------------

@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_small_kernel_eight_waves(cuda, ta, tb):
    """The small-problem kernel's 8-wave form, run by name: 512^3, and a
    ragged 300 x 200 x 1001 with padded leading dimensions and misaligned
    bases (K tail, partial tiles); C outside the window untouched."""
    plan = "mfma_f32_32x32_ksplit8"
    for i, (m, n, k, pad, off) in enumerate([(512, 512, 512, (0, 0, 0), (0, 0, 0)),
                                             (300, 200, 1001, (3, 1, 5), (1, 2, 3))]):
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, ta, tb, m, n, k, SEED + 90 + i, pad)
        print(f"small-kernel case {m}x{n}x{k} t{ta}{tb} -> {plan}", flush=True)
        got = run_sbx(cuda, np.float32, 0, ta, tb, m, n, k, -1.5, A, lda, B, ldb, 0.5, C, ldc,
                      offsets=off, plan=plan)
        want = run_oracle(0, ta, tb, m, n, k, -1.5, A, lda, B, ldb, 0.5, C, ldc)
        assert normwise(0, got, want, m, n, ldc) <= TOL[np.float32], (m, n, k)
        outside = (np.arange(C.size) % ldc) >= n
        np.testing.assert_array_equal(got[outside], C[outside])


@pytest.mark.parametrize("plan", ["mfma_f32_32x32_ksplit4", "mfma_f32_32x32_ksplit8"])
def test_small_kernel_tile_order(cuda, plan):
    """Shapes with K >= 1024 whose tile count is a multiple of 8, where the
    small-problem kernel renumbers its tiles XCD by XCD in columns G tiles
    tall: 16 x 16 tiles (G = 4), 9 x 8 ragged tiles (G = 2, the last column
    group one tile tall), 2 x 128 (a group taller than the matrix), each
    with a transposed operand; 16 x 1 and 3 x 8 (G = 1), 40 x 8 (G = 4) and
    13 x 24 (G = 4, the last group one tile tall); then a strided batch of
    3 entries of 2 x 8 tiles.  Every tile of C matches the oracle and C's padding is untouched,
    so no tile is skipped or written twice."""
    import torch
    import sushiblas_amd as sbx
    for i, (m, n, k, ta, tb) in enumerate([(512, 512, 1031, 0, 0), (283, 253, 1100, 0, 1),
                                           (283, 253, 1100, 1, 0), (64, 4096, 1024, 0, 0),
                                           (64, 4096, 1024, 1, 1), (512, 32, 1024, 0, 0),
                                           (96, 256, 1030, 1, 1), (1280, 256, 1024, 0, 1),
                                           (416, 768, 1024, 1, 0)]):
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, ta, tb, m, n, k, SEED + 95 + i,
                                             pad=(1, 2, 3))
        print(f"tile-order case {m}x{n}x{k} t{ta}{tb} -> {plan}", flush=True)
        got = run_sbx(cuda, np.float32, 0, ta, tb, m, n, k, 0.75, A, lda, B, ldb, -0.5, C, ldc,
                      plan=plan)
        want = run_oracle(0, ta, tb, m, n, k, 0.75, A, lda, B, ldb, -0.5, C, ldc)
        assert normwise(0, got, want, m, n, ldc) <= TOL[np.float32], (m, n, k, ta, tb)
        outside = (np.arange(C.size) % ldc) >= n
        np.testing.assert_array_equal(got[outside], C[outside])
    batch, m, n, k = 3, 64, 256, 1024
    str_a, str_b, str_c = m * k + 5, k * n + 3, m * n + 7
    A = oracle.fill_uniform(batch * str_a, np.float32, SEED + 99, 0)
    B = oracle.fill_uniform(batch * str_b, np.float32, SEED + 99, 1)
    C = oracle.fill_uniform(batch * str_c, np.float32, SEED + 99, 2)
    dA, dB, dC = (torch.from_numpy(x).to(cuda) for x in (A, B, C))
    print(f"tile-order case batch {batch} x {m}x{n}x{k} -> {plan}", flush=True)
    sbx.gemm_ex_plan(sbx.F32, 0, 0, 0, m, n, k, 1.25, dA, k, str_a, dB, n, str_b, 0.5, dC, n,
                     str_c, batch, plan)
    torch.cuda.synchronize()
    got = dC.cpu().numpy()
    want = C.copy()
    oracle.gemm_strided_batched(0, 0, 0, m, n, k, 1.25, A, k, str_a, B, n, str_b, 0.5, want, n,
                                str_c, batch, 1)
    for b in range(batch):
        g = c_window(0, got[b * str_c:b * str_c + m * n], m, n, n)
        w = c_window(0, want[b * str_c:b * str_c + m * n], m, n, n)
        assert oracle.rel_fro_err(g, w) <= TOL[np.float32], b
        np.testing.assert_array_equal(got[b * str_c + m * n:(b + 1) * str_c],
                                      C[b * str_c + m * n:(b + 1) * str_c])


# -- the 256x64 tile computing 48 columns (32 < n <= 48) -----------------------

@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_tile_256x48(cuda, layout, ta, tb):
    """The 256x64 tile that computes only its first 48 columns, run by name
    where C is 33-48 wide (column-major: 33-48 rows): ragged rows, a K tail,
    padded leading dimensions, beta != 0, unsplit and split in four; C's
    padding untouched."""
    for i, (m, n, k, plan) in enumerate([(4097, 48, 515, "mfma_f32_256x48x32_w8x1"),
                                         (1000, 33, 2049, "mfma_f32_256x48x32_w8x1+splitk4"),
                                         (300, 45, 64, "mfma_f32_256x48x32_w8x1")]):
        if layout == 1:
            m, n = n, m  # the narrow side is m of a column-major C
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, layout, ta, tb, m, n, k, SEED + 110 + i,
                                             pad=(2, 3, 5))
        print(f"256x48 case layout={layout} {m}x{n}x{k} t{ta}{tb} -> {plan}", flush=True)
        got = run_sbx(cuda, np.float32, layout, ta, tb, m, n, k, 1.25, A, lda, B, ldb, 0.5, C,
                      ldc, plan=plan)
        want = run_oracle(layout, ta, tb, m, n, k, 1.25, A, lda, B, ldb, 0.5, C, ldc)
        assert normwise(layout, got, want, m, n, ldc) <= TOL[np.float32], (m, n, k, plan)
        inner = n if layout == 0 else m
        outside = (np.arange(C.size) % ldc) >= inner
        np.testing.assert_array_equal(got[outside], C[outside])


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_tile_48x256(cuda, layout, ta, tb):
    """The mirror: the 64x256 tile computing only its first 48 rows, run by
    name where C has 33-48 rows (column-major: 33-48 columns), with the
    same ragged edges, K tail, padding, beta != 0 and split."""
    for i, (m, n, k, plan) in enumerate([(48, 4097, 515, "mfma_f32_48x256x32_w1x8"),
                                         (33, 1000, 2049, "mfma_f32_48x256x32_w1x8+splitk4"),
                                         (45, 300, 64, "mfma_f32_48x256x32_w1x8")]):
        if layout == 1:
            m, n = n, m
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, layout, ta, tb, m, n, k, SEED + 120 + i,
                                             pad=(2, 3, 5))
        print(f"48x256 case layout={layout} {m}x{n}x{k} t{ta}{tb} -> {plan}", flush=True)
        got = run_sbx(cuda, np.float32, layout, ta, tb, m, n, k, 1.25, A, lda, B, ldb, 0.5, C,
                      ldc, plan=plan)
        want = run_oracle(layout, ta, tb, m, n, k, 1.25, A, lda, B, ldb, 0.5, C, ldc)
        assert normwise(layout, got, want, m, n, ldc) <= TOL[np.float32], (m, n, k, plan)
        inner = n if layout == 0 else m
        outside = (np.arange(C.size) % ldc) >= inner
        np.testing.assert_array_equal(got[outside], C[outside])


# -- the large fp32 tiles on ragged edges --------------------------------------

@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_large_tiles_ragged_edges(cuda, ta, tb):
    """The 256x128 tile (two per CU) with partial tiles on both edges, a K
    tail (257 = 16*16 + 1) and padded leading dimensions.  With ldc = n + 5
    no C row allows vector access, and the same shape runs the three-per-CU
    128^2 tile, whose interior tiles then load and store C one element at a
    time.  4097 x 8191 x 515 runs the 128x128 tile with a split tail.  Each
    runs by name; the ldc padding of C stays untouched."""
    for i, (m, n, k, c_pad, want_name) in enumerate([
            (8191, 8190, 257, 6, "mfma_f32_256x128x16_w4x1"),
            (8191, 8190, 257, 5, "mfma_f32_128x128x16_w2x2_o3"),
            (4097, 8191, 515, 5, "mfma_f32_128x128x16_w2x2+splitk4")]):
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, ta, tb, m, n, k, SEED + 80 + i,
                                             pad=(3, 1, c_pad))
        print(f"large-tile case {m}x{n}x{k} t{ta}{tb} -> {want_name}", flush=True)
        got = run_sbx(cuda, np.float32, 0, ta, tb, m, n, k, 1.25, A, lda, B, ldb, 0.5, C, ldc,
                      plan=want_name)
        want = run_oracle(0, ta, tb, m, n, k, 1.25, A, lda, B, ldb, 0.5, C, ldc)
        assert normwise(0, got, want, m, n, ldc) <= TOL[np.float32], (m, n, k)
        outside = (np.arange(C.size) % ldc) >= n
        np.testing.assert_array_equal(got[outside], C[outside])


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_tall_skinny_eight_wave_tile(cuda, ta, tb):
    """The 8-wave 256x64 tile (n <= 64 with a full round of 256-row tiles):
    a ragged last row tile, n = 63, a K tail (515 = 16*32 + 3) and padded
    leading dimensions; 65536 x 64 x 1000 is a whole round with a K tail.  Run
    by name; the ldc padding of C stays untouched."""
    plan = "mfma_f32_256x64x32_w8x1"
    for i, (m, n, k) in enumerate([(65535, 63, 515), (65536, 64, 1000)]):
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, ta, tb, m, n, k, SEED + 90 + i,
                                             pad=(3, 1, 5))
        print(f"tall-skinny case {m}x{n}x{k} t{ta}{tb} -> {plan}", flush=True)
        got = run_sbx(cuda, np.float32, 0, ta, tb, m, n, k, 1.25, A, lda, B, ldb, 0.5, C, ldc,
                      plan=plan)
        want = run_oracle(0, ta, tb, m, n, k, 1.25, A, lda, B, ldb, 0.5, C, ldc)
        assert normwise(0, got, want, m, n, ldc) <= TOL[np.float32], (m, n, k)
        outside = (np.arange(C.size) % ldc) >= n
        np.testing.assert_array_equal(got[outside], C[outside])


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_wide_eight_wave_tile(cuda, ta, tb):
    """The 8-wave 64x256 tile, the tall tile's mirror (m <= 64 with a full
    round of 256-column tiles): a ragged last column tile, m = 63 and a K
    tail (515); 64 x 65536 x 1100, whose B (288 MB) is loaded
    non-temporal; m = 48.  Run by name; padded leading dimensions; the ldc
    padding of C stays untouched."""
    plan = "mfma_f32_64x256x32_w1x8"
    for i, (m, n, k) in enumerate([(63, 65535, 515), (64, 65536, 1100), (48, 65536, 2048)]):
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, ta, tb, m, n, k, SEED + 84 + i,
                                             pad=(3, 1, 5))
        print(f"wide case {m}x{n}x{k} t{ta}{tb} -> {plan}", flush=True)
        got = run_sbx(cuda, np.float32, 0, ta, tb, m, n, k, 1.25, A, lda, B, ldb, 0.5, C, ldc,
                      plan=plan)
        want = run_oracle(0, ta, tb, m, n, k, 1.25, A, lda, B, ldb, 0.5, C, ldc)
        assert normwise(0, got, want, m, n, ldc) <= TOL[np.float32], (m, n, k)
        outside = (np.arange(C.size) % ldc) >= n
        np.testing.assert_array_equal(got[outside], C[outside])


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_narrow_tiles(cuda, ta, tb):
    """The 32-wide tiles (128x32 for n <= 32, its 32x128 mirror for m <= 32):
    ragged last tiles with a K tail (515); a split tail (40000 x 32 x 2048,
    3 parts); an operand above 256 MiB loaded non-temporal (1100 deep);
    n = 1.  Run by name; padded leading dimensions; the ldc padding of C
    stays untouched."""
    cases = [(65535, 31, 515, "mfma_f32_128x32x32_w4x1"),
             (40000, 32, 2048, "mfma_f32_128x32x32_w4x1+splitk3"),
             (65536, 32, 1100, "mfma_f32_128x32x32_w4x1"),
             (4096, 1, 4096, "mfma_f32_128x32x32_w4x1+splitk8"),
             (31, 65535, 515, "mfma_f32_32x128x32_w1x4"),
             (32, 65536, 1100, "mfma_f32_32x128x32_w1x4")]
    for i, (m, n, k, want_name) in enumerate(cases):
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, ta, tb, m, n, k, SEED + 100 + i,
                                             pad=(3, 1, 5))
        print(f"narrow case {m}x{n}x{k} t{ta}{tb} -> {want_name}", flush=True)
        got = run_sbx(cuda, np.float32, 0, ta, tb, m, n, k, -0.5, A, lda, B, ldb, 1.5, C, ldc,
                      plan=want_name)
        want = run_oracle(0, ta, tb, m, n, k, -0.5, A, lda, B, ldb, 1.5, C, ldc)
        assert normwise(0, got, want, m, n, ldc) <= TOL[np.float32], (m, n, k)
        outside = (np.arange(C.size) % ldc) >= n
        np.testing.assert_array_equal(got[outside], C[outside])


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_fp32_64x64_tile(cuda, ta, tb):
    """The fp32 64x64 tile (four waves of 32x32 on 32x32x2 MFMAs): ragged
    edges with K = 1023 (a k-contiguous vector straddles K) and with
    misaligned bases; a split tail (1536 x 1536 x 1024, 4 parts).  Run by
    name; padded leading dimensions; the ldc padding of C stays untouched."""
    for i, (m, n, k, off, want_name) in enumerate([
            (1000, 1100, 1023, (0, 0, 0), "mfma_f32_64x64x32_w2x2"),
            (999, 1001, 1025, (1, 2, 3), "mfma_f32_64x64x32_w2x2"),
            (1536, 1536, 1024, (0, 0, 0), "mfma_f32_64x64x32_w2x2+splitk4")]):
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, ta, tb, m, n, k, SEED + 115 + i,
                                             pad=(3, 1, 5))
        print(f"fp32 64x64 case {m}x{n}x{k} t{ta}{tb} -> {want_name}", flush=True)
        got = run_sbx(cuda, np.float32, 0, ta, tb, m, n, k, 1.5, A, lda, B, ldb, 0.25, C, ldc,
                      offsets=off, plan=want_name)
        want = run_oracle(0, ta, tb, m, n, k, 1.5, A, lda, B, ldb, 0.25, C, ldc)
        assert normwise(0, got, want, m, n, ldc) <= TOL[np.float32], (m, n, k)
        outside = (np.arange(C.size) % ldc) >= n
        np.testing.assert_array_equal(got[outside], C[outside])


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_fp64_64x64_tile(cuda, ta, tb):
    """The fp64 64x64 tile (four waves of 32x32, 16x16x4 fp64 MFMAs): ragged
    edges with an odd K (a k-contiguous vector straddles K); a split tail
    (1536^3, 4 parts); one tile cut 31 ways along a long K, whole and ragged
    (m, n <= 64).  Run by name; padded leading dimensions; the ldc padding
    of C stays untouched.  Bar 1e-12."""
    for i, (m, n, k, want_name) in enumerate([(1500, 1300, 1023, "mfma_f64_64x64x16_w2x2"),
                                              (1536, 1536, 1536, "mfma_f64_64x64x16_w2x2+splitk4"),
                                              (64, 64, 8192, "mfma_f64_64x64x16_w2x2+splitk31"),
                                              (40, 17, 4099, "mfma_f64_64x64x16_w2x2+splitk31")]):
        A, lda, B, ldb, C, ldc = make_inputs(np.float64, 0, ta, tb, m, n, k, SEED + 110 + i,
                                             pad=(3, 1, 5))
        print(f"fp64 64x64 case {m}x{n}x{k} t{ta}{tb} -> {want_name}", flush=True)
        got = run_sbx(cuda, np.float64, 0, ta, tb, m, n, k, 0.75, A, lda, B, ldb, -1.25, C, ldc,
                      plan=want_name)
        want = run_oracle(0, ta, tb, m, n, k, 0.75, A, lda, B, ldb, -1.25, C, ldc)
        assert normwise(0, got, want, m, n, ldc) <= TOL[np.float64], (m, n, k)
        outside = (np.arange(C.size) % ldc) >= n
        np.testing.assert_array_equal(got[outside], C[outside])


@pytest.mark.parametrize("m,n,k", [(64, 64, 64), (40, 17, 70)])
def test_fp64_batch_of_tiny_problems(cuda, m, n, k):
    """A strided batch of 384 fp64 problems with m, n <= 64, where the model
    offers the 64x64 tile beside the small-problem kernel (one tile per
    problem, the batch entry on the grid's z axis), against the oracle
    entry by entry.  Bar 1e-12."""
    import torch
    import sushiblas_amd as sbx
    batch = 384
    str_a, str_b, str_c = m * k + 2, k * n + 1, m * n + 3
    A = oracle.fill_uniform(batch * str_a, np.float64, SEED + 120, 0)
    B = oracle.fill_uniform(batch * str_b, np.float64, SEED + 120, 1)
    C = oracle.fill_uniform(batch * str_c, np.float64, SEED + 120, 2)
    print(f"fp64 tiny batch {batch} x {m}x{n}x{k}", flush=True)
    dA, dB, dC = (torch.from_numpy(x).to(cuda) for x in (A, B, C))
    sbx.gemm_ex(sbx.F64, 0, 0, 0, m, n, k, -0.5, dA, k, str_a, dB, n, str_b, 1.25, dC, n, str_c,
                batch)
    torch.cuda.synchronize()
    got = dC.cpu().numpy()
    want = C.copy()
    oracle.gemm_strided_batched(0, 0, 0, m, n, k, -0.5, A, k, str_a, B, n, str_b, 1.25, want, n,
                                str_c, batch, 1)
    for b in range(batch):
        g = got[b * str_c:b * str_c + m * n].reshape(m, n)
        w = want[b * str_c:b * str_c + m * n].reshape(m, n)
        assert oracle.rel_fro_err(g, w) <= TOL[np.float64], b
        np.testing.assert_array_equal(got[b * str_c + m * n:(b + 1) * str_c],
                                      C[b * str_c + m * n:(b + 1) * str_c])


@pytest.mark.parametrize("dtype,layout,ta,tb,batch,m,n,k,want", [
    (np.float32, 0, 0, 0, 3, 300, 200, 5000, "mfma_f32_64x128x32_w2x2+splitk17"),
    (np.float64, 0, 0, 0, 3, 300, 200, 5000, "mfma_f64_64x64x16_w2x2+splitk8"),
    (np.float32, 1, 1, 0, 5, 130, 257, 3001, "mfma_f32_64x64x32_w2x2+splitk3"),
    (np.float64, 0, 1, 1, 2, 77, 500, 6000, "mfma_f64_64x64x16_w2x2+splitk8"),
])
def test_split_k_strided_batch(cuda, dtype, layout, ta, tb, batch, m, n, k, want):
    """A batch whose grid fills less than one round cuts K: every entry's
    tiles are split, entry z's partials after entry z-1's in the workspace,
    and the reduction finishes each entry's C (alpha, beta) in part order.
    Run by name.  Each entry against the oracle, and the padding between
    entries of C untouched.  Bars 1e-5 / 1e-12."""
    import torch
    import sushiblas_amd as sbx
    code = sbx.F32 if dtype == np.float32 else sbx.F64
    sa = (k, m) if ta else (m, k)
    sb = (n, k) if tb else (k, n)
    lda = sa[1] if layout == 0 else sa[0]
    ldb = sb[1] if layout == 0 else sb[0]
    ldc = n if layout == 0 else m
    str_a, str_b, str_c = sa[0] * sa[1], sb[0] * sb[1], m * n + 4
    A = oracle.fill_uniform(batch * str_a, dtype, SEED + 130, 0)
    B = oracle.fill_uniform(batch * str_b, dtype, SEED + 130, 1)
    C = oracle.fill_uniform(batch * str_c, dtype, SEED + 130, 2)
    print(f"split batch {batch} x {m}x{n}x{k} layout={layout} t{ta}{tb} -> {want}", flush=True)
    dA, dB, dC = (torch.from_numpy(x).to(cuda) for x in (A, B, C))
    sbx.gemm_ex_plan(code, layout, ta, tb, m, n, k, 0.75, dA, lda, str_a, dB, ldb, str_b, -0.5,
                     dC, ldc, str_c, batch, want)
    torch.cuda.synchronize()
    got = dC.cpu().numpy()
    want_c = C.copy()
    oracle.gemm_strided_batched(layout, ta, tb, m, n, k, 0.75, A, lda, str_a, B, ldb, str_b, -0.5,
                                want_c, ldc, str_c, batch, 1)
    for b in range(batch):
        g = c_window(layout, got[b * str_c:b * str_c + m * n], m, n, ldc)
        w = c_window(layout, want_c[b * str_c:b * str_c + m * n], m, n, ldc)
        assert oracle.rel_fro_err(g, w) <= TOL[dtype], b
        np.testing.assert_array_equal(got[b * str_c + m * n:(b + 1) * str_c],
                                      C[b * str_c + m * n:(b + 1) * str_c])


def test_column_major_tall_skinny(cuda):
    """cfg4's shape (65536 x 64 x 4096) in column-major storage: C^T = B^T A^T
    makes it the wide row-major problem 64 x 65536 x 4096, run on the 64x256
    tile (its pick) with the long operand loaded non-temporal."""
    m, n, k = 65536, 64, 4096
    err, _, _ = _case(cuda, np.float32, 1, 0, 0, m, n, k, 1.0, 0.0, SEED + 87,
                      plan="mfma_f32_64x256x32_w1x8")
    assert err <= TOL[np.float32]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_tall_skinny_eight_wave_split_and_rounds(cuda, ta, tb):
    """The 8-wave 256x64 tile where its grid is not one whole round:
    80000 x 64 x 2048 runs 256 whole tiles plus a 57-tile tail cut 4 ways
    (its split partials fill 16384-element workspace slots and the reduction
    walks 64 chunks of each), and 131000 x 63 x 515 runs two whole rounds
    of 256 tiles (a ragged last row tile, n = 63 and a K tail); 100000 x 63
    x 515 on the 128x64 tile, unsplit with a partial last round.  Run by
    name; padded leading dimensions; the ldc padding of C stays untouched."""
    for i, (m, n, k, want_name) in enumerate([
            (80000, 64, 2048, "mfma_f32_256x64x32_w8x1+splitk4"),
            (131000, 63, 515, "mfma_f32_256x64x32_w8x1"),
            (100000, 63, 515, "mfma_f32_128x64x32_w2x2")]):
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, ta, tb, m, n, k, SEED + 96 + i,
                                             pad=(3, 1, 5))
        print(f"tall-skinny case {m}x{n}x{k} t{ta}{tb} -> {want_name}", flush=True)
        got = run_sbx(cuda, np.float32, 0, ta, tb, m, n, k, -0.75, A, lda, B, ldb, 1.5, C, ldc,
                      plan=want_name)
        want = run_oracle(0, ta, tb, m, n, k, -0.75, A, lda, B, ldb, 1.5, C, ldc)
        assert normwise(0, got, want, m, n, ldc) <= TOL[np.float32], (m, n, k)
        outside = (np.arange(C.size) % ldc) >= n
        np.testing.assert_array_equal(got[outside], C[outside])


@pytest.mark.parametrize("dtype,m,n,k,ta,tb,kernel", [
    (np.float32, 48, 70000, 1024, 0, 0, "mfma_f32_64x128x32_w2x2+splitk6"),  # B 287 MB
    (np.float32, 48, 70000, 1024, 1, 1, "mfma_f32_64x128x32_w2x2+splitk6"),
    (np.float32, 64, 65536, 1024, 0, 1, "mfma_f32_64x256x32_w1x8"),         # B 268 MB
    (np.float64, 65536, 64, 1024, 0, 0, "mfma_f64_128x64x16_w2x2"),         # A 537 MB
    (np.float64, 65536, 40, 1024, 1, 0, "mfma_f64_128x64x16_w2x2"),
    (np.float32, 70000, 64, 4096, 1, 0, "mfma_f32_256x64x32_w8x1+splitk11"),  # A 1.15 GB
])
def test_streamed_operand_above_last_level_cache(cuda, dtype, m, n, k, ta, tb, kernel):
    """A grid one tile wide reads its long operand once; above 256 MiB that
    operand's loads are non-temporal (a kernel variant with the nt cache
    policy, unsplit and with a split tail), whichever plan runs; each runs by
    name.  Every output against the oracle."""
    err, _, _ = _case(cuda, dtype, 0, ta, tb, m, n, k, 1.0, 0.5, SEED + 83, plan=kernel)
    assert err <= TOL[dtype]


# -- split-K of under-filled grids ---------------------------------------------

@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_split_k_is_deterministic(cuda, dtype):
    """The reduction kernel sums a split tile's partials in fixed part order:
    two runs give identical bits, and they match the oracle."""
    import sushiblas_amd as sbx
    m, n, k = 384, 320, 3000
    name = sbx.gemm_select(sbx.F32 if dtype == np.float32 else sbx.F64, 0, 0, 0, m, n, k, k, n, n)
    assert "+splitk" in name, name
    A, lda, B, ldb, C, ldc = make_inputs(dtype, 0, 0, 0, m, n, k, SEED + 70)
    g1 = run_sbx(cuda, dtype, 0, 0, 0, m, n, k, 1.25, A, lda, B, ldb, -0.5, C, ldc)
    g2 = run_sbx(cuda, dtype, 0, 0, 0, m, n, k, 1.25, A, lda, B, ldb, -0.5, C, ldc)
    np.testing.assert_array_equal(g1.view(np.uint8), g2.view(np.uint8))
    want = run_oracle(0, 0, 0, m, n, k, 1.25, A, lda, B, ldb, -0.5, C, ldc)
    assert normwise(0, g1, want, m, n, ldc) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_long_k_wide_splits(cuda, dtype):
    """Small outputs over a long K, run by name: the tail is cut into up to
    32 k-ranges (256 x 256 x 65536: 16 64^2 tiles, 32 parts each; 325 x 351
    x 12266: 36 tiles, 14 parts), and the reduction sums up to 32 partials
    per element in part order.  Ragged edges, padded leading dimensions and
    a K tail on the second shape; whole results against the oracle, the ldc
    padding untouched, two runs bit-identical."""
    tile = "mfma_f32_64x64x32_w2x2" if dtype == np.float32 else "mfma_f64_64x64x16_w2x2"
    for i, (m, n, k, parts) in enumerate([(256, 256, 65536, 32), (325, 351, 12266, 14)]):
        A, lda, B, ldb, C, ldc = make_inputs(dtype, 0, 0, 0, m, n, k, SEED + 74 + i,
                                             pad=(3, 1, 5))
        plan = f"{tile}+splitk{parts}"
        print(f"long-K case {m}x{n}x{k} {np.dtype(dtype).name} -> {plan}", flush=True)
        g1 = run_sbx(cuda, dtype, 0, 0, 0, m, n, k, 0.75, A, lda, B, ldb, 0.5, C, ldc, plan=plan)
        g2 = run_sbx(cuda, dtype, 0, 0, 0, m, n, k, 0.75, A, lda, B, ldb, 0.5, C, ldc, plan=plan)
        np.testing.assert_array_equal(g1.view(np.uint8), g2.view(np.uint8))
        want = run_oracle(0, 0, 0, m, n, k, 0.75, A, lda, B, ldb, 0.5, C, ldc)
        assert normwise(0, g1, want, m, n, ldc) <= TOL[dtype], (m, n, k)
        outside = (np.arange(C.size) % ldc) >= n
        np.testing.assert_array_equal(g1[outside], C[outside])


def test_workspace_growth_under_concurrent_host_threads(cuda):
    """Host threads share one (fresh) stream and mix a small split-K shape
    (workspace within the initial size) with a 128x128-tile shape whose split
    tail needs a larger workspace, so the cache grows while other threads may
    hold the old address.  Every result must match the oracle."""
    import threading
    import torch
    import sushiblas_amd as sbx
    shapes = [(512, 512, 512), (3072, 3456, 2048)]
    # 24 x 27 = 648 tiles of 128x128: a round of 512 and a 136-tile tail cut
    # into >= 4 parts of 64 KiB: > 32 MiB of partials
    name = sbx.gemm_select(sbx.F32, 0, 0, 0, 3072, 3456, 2048, 2048, 3456, 3456)
    assert name.startswith("mfma_f32_128x128x16_w2x2+") and int(name.split("splitk")[1]) >= 4, name
    data = []
    for i, (m, n, k) in enumerate(shapes):
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, 0, 0, m, n, k, SEED + 72 + i)
        want = run_oracle(0, 0, 0, m, n, k, 1.0, A, lda, B, ldb, 0.0, C, ldc)
        data.append((m, n, k, torch.from_numpy(A).to(cuda), lda, torch.from_numpy(B).to(cuda),
                     ldb, ldc, want))
    stream = torch.cuda.Stream()
    outs = [[torch.zeros(d[0] * d[1], device=cuda) for _ in range(3)] for d in data]
    torch.cuda.synchronize()
    errors = []

    def worker(t):
        try:
            for rep in range(3):
                for j in ((t + rep) % 2, (t + rep + 1) % 2):
                    m, n, k, dA, lda, dB, ldb, ldc, _ = data[j]
                    sbx.sgemm(0, 0, 0, m, n, k, 1.0, dA, lda, dB, ldb, 0.0, outs[j][t % 3], ldc,
                              stream=stream)
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(6)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    stream.synchronize()
    assert not errors, errors
    for (m, n, k, _, _, _, _, ldc, want), group in zip(data, outs):
        for o in group:
            assert normwise(0, o.cpu().numpy(), want, m, n, ldc) <= TOL[np.float32]


HIP_STREAM_PER_THREAD = 2  # hipStreamPerThread: a different stream in every host thread


@pytest.mark.skip(reason="run six times in one process against per-thread workspaces that "
                  "the exiting thread synchronized and pooled, this test aborted with "
                  "'free(): invalid pointer' on its third run, cause not found; "
                  "hipStreamPerThread now gets no workspace (its calls run unsplit), "
                  "which test_per_thread_stream_runs_unsplit covers from one thread")
def test_split_k_per_thread_streams(cuda):
    """hipStreamPerThread names one stream per host thread, so two threads
    issuing split-K GEMMs through it run concurrently on different streams:
    each thread must get its own workspace.  A third and fourth thread start
    as soon as the first two have exited, without any synchronization of
    their own: they take the pooled workspaces, which the exiting threads
    left idle by waiting for their per-thread streams.  After a device-wide
    synchronization a fifth and sixth thread take pooled workspaces again
    (without allocating).  Threads of the later waves synchronize before
    they exit, so that their per-thread streams have finished when the
    results are read.  Every result must match the oracle, and every call
    must succeed (a pooled workspace once carried an event recorded on the
    exited thread's destroyed stream, whose query failed and left an error
    that the next launch check reported)."""
    import threading
    import torch
    import sushiblas_amd as sbx
    shapes = [(1536, 1536, 1024), (384, 320, 3000)]
    data = []
    for i, (m, n, k) in enumerate(shapes):
        name = sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n)
        assert "+splitk" in name, name
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, 0, 0, m, n, k, SEED + 73 + i)
        want = run_oracle(0, 0, 0, m, n, k, 1.0, A, lda, B, ldb, 0.0, C, ldc)
        data.append((m, n, k, torch.from_numpy(A).to(cuda), lda, torch.from_numpy(B).to(cuda),
                     ldb, ldc, want))
    outs = {t: [[torch.zeros(d[0] * d[1], device=cuda) for _ in range(4)] for d in data]
            for t in range(6)}
    torch.cuda.synchronize()
    errors = []

    def worker(t, sync_at_exit):
        try:
            for rep in range(4):
                for j in ((t + rep) % 2, (t + rep + 1) % 2):
                    m, n, k, dA, lda, dB, ldb, ldc, _ = data[j]
                    sbx.sgemm(0, 0, 0, m, n, k, 1.0, dA, lda, dB, ldb, 0.0, outs[t][j][rep], ldc,
                              stream=HIP_STREAM_PER_THREAD)
            if sync_at_exit:
                torch.cuda.synchronize()  # from this thread: covers its per-thread stream
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    free_before_last = None
    for wave, sync_at_exit in (((0, 1), False), ((2, 3), True), ((4, 5), True)):
        if wave[0] == 4:
            torch.cuda.synchronize()
            free_before_last = torch.cuda.mem_get_info()[0]
        threads = [threading.Thread(target=worker, args=(t, sync_at_exit)) for t in wave]
        for th in threads:
            th.start()
        for th in threads:
            th.join()
    torch.cuda.synchronize()
    assert not errors, errors
    # the last wave reused idle pooled workspaces (>= 32 MiB each if new); the
    # runtime's own set-up of two new per-thread streams takes a few MiB
    grown = free_before_last - torch.cuda.mem_get_info()[0]
    assert grown < (32 << 20), grown
    for t in range(6):
        for (m, n, k, _, _, _, _, ldc, want), group in zip(data, outs[t]):
            for o in group:
                assert normwise(0, o.cpu().numpy(), want, m, n, ldc) <= TOL[np.float32], (t, m)


def test_per_thread_stream_runs_unsplit(cuda):
    """hipStreamPerThread gets no workspace: a GEMM that splits on an
    explicit stream and a column-chunked GEMV run unsplit on it, from the
    calling thread, match the oracle and allocate nothing."""
    import torch
    import sushiblas_amd as sbx
    m, n, k = 1536, 1536, 1024
    assert "+splitk" in sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n)
    A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, 0, 0, m, n, k, SEED + 81)
    want = run_oracle(0, 0, 0, m, n, k, 1.0, A, lda, B, ldb, 0.0, C, ldc)
    gm, gn = 64, 262144  # row-dot GEMV whose columns are cut into chunks elsewhere
    gA = oracle.fill_uniform(gm * gn, np.float32, SEED + 82, 0)
    gx = oracle.fill_uniform(gn, np.float32, SEED + 82, 1)
    gwant = np.zeros(gm, np.float32)
    oracle.gemv(0, 0, gm, gn, 1.0, gA, gn, gx, 1, 0.0, gwant, 1)
    dA, dB = torch.from_numpy(A).to(cuda), torch.from_numpy(B).to(cuda)
    dgA, dgx = torch.from_numpy(gA).to(cuda), torch.from_numpy(gx).to(cuda)
    out = torch.zeros(m * n, device=cuda)
    gy = torch.zeros(gm, device=cuda)
    # the runtime's set-up of this thread's per-thread stream comes first
    sbx.sgemm(0, 0, 0, 64, 64, 64, 1.0, dA, lda, dB, ldb, 0.0, out, 64,
              stream=HIP_STREAM_PER_THREAD)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(2):
        sbx.sgemm(0, 0, 0, m, n, k, 1.0, dA, lda, dB, ldb, 0.0, out, ldc,
                  stream=HIP_STREAM_PER_THREAD)
        sbx.gemv(sbx.F32, 0, 0, gm, gn, 1.0, dgA.data_ptr(), gn, dgx.data_ptr(), 1, 0.0,
                 gy.data_ptr(), 1, stream=HIP_STREAM_PER_THREAD)
    torch.cuda.synchronize()  # device-wide: covers the per-thread stream
    grown = free0 - torch.cuda.mem_get_info()[0]
    assert grown < (32 << 20), grown  # a workspace is at least 32 MiB
    assert normwise(0, out.cpu().numpy(), want, m, n, ldc) <= TOL[np.float32]
    got = gy.cpu().numpy().astype(np.float64)
    err = np.linalg.norm(got - gwant) / np.linalg.norm(gwant.astype(np.float64))
    assert err <= TOL[np.float32], err


def test_split_k_when_the_workspace_cannot_be_allocated(cuda):
    """With less device memory free than the smallest workspace (32 MiB), a
    split GEMM and a column-chunked GEMV on a new stream (no workspace yet)
    run without splitting and succeed: the failed hipMalloc leaves its error
    as the thread's last error, which the library consumes, since a launch
    check that reported it would fail the call.  With the memory free again,
    the next calls allocate and split.  All kernels the test launches are
    loaded and the stream's queue made beforehand, so that nothing else
    needs device memory while it is exhausted."""
    import ctypes
    import os
    import torch
    import sushiblas_amd as sbx
    # the runtime torch loaded (loading another would start a second one)
    hip = ctypes.CDLL(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so"))
    m, n, k = 1536, 1536, 1024
    assert "+splitk" in sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n)
    A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, 0, 0, m, n, k, SEED + 79)
    want = run_oracle(0, 0, 0, m, n, k, 1.0, A, lda, B, ldb, 0.0, C, ldc)
    gm, gn = 64, 262144  # row-dot GEMV whose columns are cut into chunks
    gA = oracle.fill_uniform(gm * gn, np.float32, SEED + 80, 0)
    gx = oracle.fill_uniform(gn, np.float32, SEED + 80, 1)
    gwant = np.zeros(gm, np.float32)
    oracle.gemv(0, 0, gm, gn, 1.0, gA, gn, gx, 1, 0.0, gwant, 1)
    dA, dB = torch.from_numpy(A).to(cuda), torch.from_numpy(B).to(cuda)
    dgA, dgx = torch.from_numpy(gA).to(cuda), torch.from_numpy(gx).to(cuda)
    outs = [torch.zeros(m * n, device=cuda) for _ in range(3)]
    gys = [torch.zeros(gm, device=cuda) for _ in range(3)]
    raw = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(raw)) == 0
    s = raw.value

    def calls(i, stream):
        sbx.sgemm(0, 0, 0, m, n, k, 1.0, dA, lda, dB, ldb, 0.0, outs[i], ldc, stream=stream)
        sbx.gemv(sbx.F32, 0, 0, gm, gn, 1.0, dgA.data_ptr(), gn, dgx.data_ptr(), 1, 0.0,
                 gys[i].data_ptr(), 1, stream=stream)

    hog = []
    try:
        calls(0, None)  # loads the kernels, split and unsplit alike
        # an unsplit call on the new stream makes its queue, no workspace
        sbx.sgemm(0, 0, 0, 64, 64, 64, 1.0, dA, lda, dB, ldb, 0.0, outs[1], 64, stream=s)
        assert hip.hipStreamSynchronize(ctypes.c_void_p(s)) == 0
        torch.cuda.synchronize()
        # torch's cached blocks count as used until they are released
        torch.cuda.empty_cache()
        for _ in range(3):
            left = torch.cuda.mem_get_info()[0]
            if left < (32 << 20):
                break
            hog.append(torch.empty(left - (24 << 20), dtype=torch.uint8, device=cuda))
            print(f"hog of {(left >> 20) - 24} MiB", flush=True)
        left = torch.cuda.mem_get_info()[0]
        print(f"free with the hog {left >> 20} MiB", flush=True)
        assert left < (32 << 20), left
        calls(1, s)  # no memory for a workspace: unsplit, and no error
        assert hip.hipStreamSynchronize(ctypes.c_void_p(s)) == 0
        hog.clear()
        torch.cuda.empty_cache()
        calls(2, s)  # allocates the stream's workspace and splits
        assert hip.hipStreamSynchronize(ctypes.c_void_p(s)) == 0
    finally:
        hog.clear()
        torch.cuda.empty_cache()
        torch.cuda.synchronize()
        assert hip.hipStreamDestroy(ctypes.c_void_p(s)) == 0
    for i in range(3):
        assert normwise(0, outs[i].cpu().numpy(), want, m, n, ldc) <= TOL[np.float32], i
        got = gys[i].cpu().numpy().astype(np.float64)
        err = np.linalg.norm(got - gwant) / np.linalg.norm(gwant.astype(np.float64))
        assert err <= TOL[np.float32], (i, err)


def test_split_k_on_two_streams(cuda):
    """Each stream has its own split-K workspace: concurrent calls on two
    streams do not corrupt each other."""
    import torch
    import sushiblas_amd as sbx
    m, n, k = 1536, 1536, 1024
    assert "+splitk" in sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n)
    A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, 0, 0, m, n, k, SEED + 71)
    want = run_oracle(0, 0, 0, m, n, k, 1.0, A, lda, B, ldb, 0.0, C, ldc)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    dA = torch.from_numpy(A).to(cuda)
    dB = torch.from_numpy(B).to(cuda)
    outs = [torch.zeros(m * n, device=cuda) for _ in range(4)]
    torch.cuda.synchronize()
    for rep in range(3):
        for i, o in enumerate(outs):
            st = s1 if i % 2 == 0 else s2
            with torch.cuda.stream(st):
                sbx.sgemm(0, 0, 0, m, n, k, 1.0, dA, lda, dB, ldb, 0.0, o, ldc, stream=st)
    torch.cuda.synchronize()
    for o in outs:
        assert normwise(0, o.cpu().numpy(), want, m, n, ldc) <= TOL[np.float32]


def test_default_stream_is_torch_current_stream(cuda):
    """A call without an explicit stream goes to torch's current stream,
    including inside a `torch.cuda.stream` context (the raw-handle query
    must agree with torch.cuda.current_stream())."""
    import torch
    import sushiblas_amd as sbx
    assert sbx._stream(None) == torch.cuda.current_stream().cuda_stream
    s = torch.cuda.Stream()
    m, n, k = 512, 512, 512
    A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, 0, 0, m, n, k, SEED + 81)
    want = run_oracle(0, 0, 0, m, n, k, 1.0, A, lda, B, ldb, 0.0, C, ldc)
    dA = torch.from_numpy(A).to(cuda)
    dB = torch.from_numpy(B).to(cuda)
    out = torch.zeros(m * n, device=cuda)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        assert sbx._stream(None) == s.cuda_stream
        sbx.gemm_ex(sbx.F32, 0, 0, 0, m, n, k, 1.0, dA, lda, 0, dB, ldb, 0, 0.0, out, ldc, 0)
    s.synchronize()
    assert normwise(0, out.cpu().numpy(), want, m, n, ldc) <= TOL[np.float32]
