"""Pins the CPU oracle (oracle/sbo.c) before anything is checked against it.

Each check is independent of the oracle's own formula:
  * published known answers: Random123's Philox4x32-10 KAT vectors; the
    reference's GEMM known answers (tests/blas/level3/test_gemm.cpp:39-88);
  * closed forms from the reference's integration inputs
    (tests/runtime/test_framework_sim.cpp);
  * a plain long-double triple loop (no packing/blocking) on small inputs;
  * independent host BLAS: numpy/OpenBLAS and torch/MKL;
  * invariants that a dropped term, wrong sign/index or transposed operand
    breaks: explicit-transpose copies, column-major == swapped row-major,
    batched == loop, quick returns;
  * planted mistakes: feeding the oracle a wrong flag must fail the checks.
"""
import numpy as np
import pytest

import oracle


# -- Philox4x32-10 known-answer vectors (Random123 kat_vectors, 10 rounds) ----

@pytest.mark.parametrize("ctr,key,expect", [
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
])
def test_philox_known_answers(ctr, key, expect):
    assert oracle.philox4x32_10(ctr, key).tolist() == expect


def test_uniform_stream_layout():
    """f32 element e = (word e%4 of block e/4 >> 8) * 2^-23 - 1, exact in float."""
    u = oracle.fill_uniform(10, np.float32, 1234, 5)
    for e in range(10):
        w = oracle.philox4x32_10([e // 4, 0, 5, 0], [1234, 0])[e % 4]
        assert u[e] == np.float32((int(w) >> 8) * 2.0 ** -23 - 1.0)
    d = oracle.fill_uniform(6, np.float64, 99, 1)
    for e in range(6):
        w = oracle.philox4x32_10([e // 2, 0, 1, 0], [99, 0])
        a, b = int(w[2 * (e % 2)]), int(w[2 * (e % 2) + 1])
        assert d[e] == ((a >> 5) * 2.0 ** 26 + (b >> 6)) * 2.0 ** -52 - 1.0


def test_generator_ranges_and_statistics():
    u = oracle.fill_uniform(1 << 20, np.float32, 7, 0)
    assert u.min() >= -1.0 and u.max() < 1.0
    assert np.all((u.astype(np.float64) + 1.0) * 2 ** 23 == np.round((u + 1.0) * 2 ** 23))
    assert abs(u.mean()) < 3e-3 and abs(u.var() - 1 / 3) < 3e-3
    d = oracle.fill_uniform(1 << 20, np.float64, 7, 0)
    assert d.min() >= -1.0 and d.max() < 1.0 and abs(d.mean()) < 3e-3
    z = oracle.fill_normal(1 << 20, np.float64, 7, 0)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1) < 5e-3
    assert abs(np.mean(z ** 4) - 3) < 0.05  # Gaussian kurtosis
    # distinct streams / seeds give distinct numbers
    assert not np.array_equal(oracle.fill_uniform(64, np.float32, 7, 0),
                              oracle.fill_uniform(64, np.float32, 7, 1))
    assert not np.array_equal(oracle.fill_uniform(64, np.float32, 7, 0),
                              oracle.fill_uniform(64, np.float32, 8, 0))


# -- reference known answers ----------------------------------------------------

def test_reference_known_answer_3x3():
    """test_gemm.cpp:39-63 (row-major, beta = 0)."""
    A = np.arange(1, 10, dtype=np.float32)
    B = (2 * np.eye(3, dtype=np.float32)).ravel()
    for mode in (0, 1):
        C = np.full(9, np.nan, np.float32)
        oracle.gemm(0, 0, 0, 3, 3, 3, 1.0, A, 3, B, 3, 0.0, C, 3, mode)
        assert C.tolist() == [2, 4, 6, 8, 10, 12, 14, 16, 18]


def test_reference_known_answer_column_major():
    """test_gemm.cpp:65-88 (column-major engine)."""
    for dtype in (np.float32, np.float64):
        A = np.array([1, 3, 2, 4], dtype)
        B = np.array([5, 7, 6, 8], dtype)
        C = np.zeros(4, dtype)
        oracle.gemm(1, 0, 0, 2, 2, 2, 1.0, A, 2, B, 2, 0.0, C, 2)
        assert C.tolist() == [19, 43, 22, 50]


def test_framework_sim_closed_forms():
    """test_framework_sim.cpp:75-128: X = 1, W = 2, K = 256 -> Y = 512 exactly;
    :10-73: X = 1, W = 0.01, K = 1024 -> 1024 * fp32(0.01) up to fp32 rounding."""
    X = np.ones(256 * 256, np.float32)
    W = np.full(256 * 512, 2.0, np.float32)
    Y = np.empty(256 * 512, np.float32)
    oracle.gemm(0, 0, 0, 256, 512, 256, 1.0, X, 256, W, 512, 0.0, Y, 512, 0)
    assert (Y == 512.0).all()
    X = np.ones(64 * 1024, np.float32)
    W = np.full(1024 * 1024, 0.01, np.float32)
    H = np.empty(64 * 1024, np.float32)
    oracle.gemm(0, 0, 0, 64, 1024, 1024, 1.0, X, 1024, W, 1024, 0.0, H, 1024, 1)
    assert np.allclose(H, 1024 * np.float64(np.float32(0.01)), rtol=1e-7)


# -- brute force ---------------------------------------------------------------

def _inputs(dtype, layout, ta, tb, m, n, k, seed, pad=0):
    sa = (k, m) if ta else (m, k)
    sb = (n, k) if tb else (k, n)
    lda = (sa[1] if layout == 0 else sa[0]) + pad
    ldb = (sb[1] if layout == 0 else sb[0]) + pad
    ldc = (n if layout == 0 else m) + pad
    na = (sa[0] - 1) * lda + sa[1] if layout == 0 else (sa[1] - 1) * lda + sa[0]
    nb = (sb[0] - 1) * ldb + sb[1] if layout == 0 else (sb[1] - 1) * ldb + sb[0]
    nc = (m - 1) * ldc + n if layout == 0 else (n - 1) * ldc + m
    A = oracle.fill_uniform(max(na, 1), dtype, seed, 0)
    B = oracle.fill_uniform(max(nb, 1), dtype, seed, 1)
    C = oracle.fill_uniform(max(nc, 1), dtype, seed, 2)
    return A, lda, B, ldb, C, ldc


def _op(layout, trans, X, rows, cols, ld):
    """op(X) as a dense rows x cols float64 array (independent index path)."""
    sr, sc = (cols, rows) if trans else (rows, cols)
    full = np.zeros((sr if layout == 0 else sc) * ld, np.float64)
    full[:X.size] = X
    M = full.reshape(sr, ld)[:, :sc] if layout == 0 else full.reshape(sc, ld)[:, :sr].T
    return M.T if trans else M


SHAPES = [(1, 1, 1), (5, 3, 7), (65, 257, 31), (64, 256, 256), (70, 300, 513), (130, 9, 260)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_blocked_matches_long_double_brute_force(dtype, layout, ta, tb):
    tol = 2e-7 if dtype == np.float32 else 1e-15
    for i, (m, n, k) in enumerate(SHAPES):
        alpha, beta = [(1.0, 0.0), (-0.75, 1.25), (1.5, 0.5)][i % 3]
        A, lda, B, ldb, C, ldc = _inputs(dtype, layout, ta, tb, m, n, k, 300 + i, pad=i % 2)
        C1, C2 = C.copy(), C.copy()
        oracle.gemm(layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C1, ldc, 1)
        oracle.gemm_naive_ld(layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C2, ldc)
        assert oracle.rel_fro_err(C1.reshape(1, -1), C2.reshape(1, -1)) <= tol, (m, n, k)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_against_numpy_blas(dtype, ta, tb):
    """Independent library: numpy matmul (OpenBLAS) in float64 on op(A), op(B)."""
    m, n, k = 300, 257, 411
    for layout in (0, 1):
        A, lda, B, ldb, C, ldc = _inputs(dtype, layout, ta, tb, m, n, k, 11)
        want = 1.5 * _op(layout, ta, A, m, k, lda) @ _op(layout, tb, B, k, n, ldb) \
            - 0.5 * _op(layout, 0, C, m, n, ldc)
        got = C.copy()
        oracle.gemm(layout, ta, tb, m, n, k, 1.5, A, lda, B, ldb, -0.5, got, ldc, 1)
        g = _op(layout, 0, got, m, n, ldc)
        err = np.linalg.norm(g - want) / np.linalg.norm(want)
        assert err <= (1e-7 if dtype == np.float32 else 1e-15)


def test_against_torch_mkl():
    """Independent library: torch.mm on CPU (MKL, the vendor family of the
    reference's oneMKL CPU path), fp32 in fp32."""
    torch = pytest.importorskip("torch")
    m, n, k = 512, 512, 512
    A = oracle.fill_uniform(m * k, np.float32, 20261202, 0)
    B = oracle.fill_uniform(k * n, np.float32, 20261202, 1)
    C = np.zeros(m * n, np.float32)
    oracle.gemm(0, 0, 0, m, n, k, 1.0, A, k, B, n, 0.0, C, n, 0)
    ref = torch.mm(torch.from_numpy(A).view(m, k), torch.from_numpy(B).view(k, n)).numpy()
    assert oracle.rel_fro_err(C.reshape(m, n), ref) <= 1e-6


# -- invariants ------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_transposed_copies_give_identical_results(dtype):
    m, n, k = 67, 45, 130
    A = oracle.fill_uniform(m * k, dtype, 5, 0).reshape(m, k)
    B = oracle.fill_uniform(k * n, dtype, 5, 1).reshape(k, n)
    ref = None
    for ta in (0, 1):
        for tb in (0, 1):
            Ast = np.ascontiguousarray(A.T if ta else A).ravel()
            Bst = np.ascontiguousarray(B.T if tb else B).ravel()
            C = np.zeros(m * n, dtype)
            oracle.gemm(0, ta, tb, m, n, k, 1.0, Ast, m if ta else k, Bst, k if tb else n, 0.0,
                        C, n, 1)
            if ref is None:
                ref = C
            np.testing.assert_array_equal(C, ref)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_column_major_equals_swapped_row_major(dtype):
    """col-major C = op(A) op(B) is row-major C^T = op(B)^T op(A)^T."""
    m, n, k = 33, 70, 90
    for ta in (0, 1):
        for tb in (0, 1):
            A, lda, B, ldb, C, ldc = _inputs(dtype, 1, ta, tb, m, n, k, 17)
            C1, C2 = C.copy(), C.copy()
            oracle.gemm(1, ta, tb, m, n, k, 0.5, A, lda, B, ldb, 2.0, C1, ldc, 1)
            oracle.gemm(0, tb, ta, n, m, k, 0.5, B, ldb, A, lda, 2.0, C2, ldc, 1)
            np.testing.assert_array_equal(C1, C2)


def test_batched_equals_loop():
    batch, m, n, k = 3, 20, 30, 40
    A = oracle.fill_uniform(batch * m * k + 5, np.float32, 3, 0)
    B = oracle.fill_uniform(k * n, np.float32, 3, 1)
    C = oracle.fill_uniform(batch * (m * n + 2), np.float32, 3, 2)
    got = C.copy()
    oracle.gemm_strided_batched(0, 0, 0, m, n, k, 1.0, A, k, m * k, B, n, 0, 1.0, got, n,
                                m * n + 2, batch, 1)
    for b in range(batch):
        want = C[b * (m * n + 2):b * (m * n + 2) + m * n].copy()
        oracle.gemm(0, 0, 0, m, n, k, 1.0, A[b * m * k:(b + 1) * m * k].copy(), k, B, n, 1.0,
                    want, n, 1)
        np.testing.assert_array_equal(got[b * (m * n + 2):b * (m * n + 2) + m * n], want)
        assert got[b * (m * n + 2) + m * n] == C[b * (m * n + 2) + m * n]


def test_quick_returns():
    A = np.full(12, np.nan, np.float32)
    B = np.full(12, np.nan, np.float32)
    C = np.arange(12, dtype=np.float32)
    got = C.copy()
    oracle.gemm(0, 0, 0, 3, 4, 4, 0.0, A, 4, B, 4, 2.0, got, 4)   # alpha = 0: C = beta C
    np.testing.assert_array_equal(got, 2 * C)
    got = C.copy()
    oracle.gemm(0, 0, 0, 3, 4, 0, 1.0, A, 1, B, 4, -1.0, got, 4)  # k = 0
    np.testing.assert_array_equal(got, -C)
    got = np.full(12, np.nan, np.float32)
    oracle.gemm(0, 0, 0, 3, 4, 0, 1.0, A, 1, B, 4, 0.0, got, 4)   # beta = 0 never reads C
    assert (got == 0).all()
    got = C.copy()
    oracle.gemm(0, 0, 0, 0, 4, 4, 1.0, A, 4, B, 4, 0.0, got, 4)   # m = 0: no-op
    np.testing.assert_array_equal(got, C)
    Af = oracle.fill_uniform(12, np.float32, 1, 0)
    Bf = oracle.fill_uniform(16, np.float32, 1, 1)
    got = np.full(12, np.nan, np.float32)
    oracle.gemm(0, 0, 0, 3, 4, 4, 1.0, Af, 4, Bf, 4, 0.0, got, 4)
    assert not np.isnan(got).any()


def test_rejects_bad_arguments():
    A = np.zeros(16, np.float32)
    with pytest.raises(ValueError):
        oracle.gemm(0, 0, 0, 4, 4, 4, 1.0, A, 3, A, 4, 0.0, A.copy(), 4)  # lda < k
    with pytest.raises(ValueError):
        oracle.gemm(2, 0, 0, 4, 4, 4, 1.0, A, 4, A, 4, 0.0, A.copy(), 4)  # bad layout


def test_rel_fro_err_closed_forms():
    Y = oracle.fill_uniform(1000, np.float64, 1, 0).reshape(10, 100)
    assert oracle.rel_fro_err(Y, Y) == 0.0
    assert abs(oracle.rel_fro_err(Y * (1 + 1e-3), Y) - 1e-3) < 1e-12
    assert abs(oracle.rel_fro_err(-Y, Y) - 2.0) < 1e-12
    assert oracle.rel_fro_err(np.zeros((2, 2)), np.zeros((2, 2))) == 0.0
    assert oracle.rel_fro_err(np.ones((2, 2)), np.zeros((2, 2))) == float("inf")


# -- planted mistakes: the checks above must be able to fail -----------------

def test_checks_catch_a_transposed_operand():
    m = n = k = 48
    A, lda, B, ldb, C, ldc = _inputs(np.float32, 0, 0, 0, m, n, k, 77)
    good, bad = C.copy(), C.copy()
    oracle.gemm_naive_ld(0, 0, 0, m, n, k, 1.0, A, lda, B, ldb, 0.0, good, ldc)
    oracle.gemm(0, 1, 0, m, n, k, 1.0, A, lda, B, ldb, 0.0, bad, ldc, 1)  # planted: transA
    assert oracle.rel_fro_err(bad.reshape(m, n), good.reshape(m, n)) > 0.1


def test_checks_catch_a_dropped_beta_term():
    m = n = k = 32
    A, lda, B, ldb, C, ldc = _inputs(np.float64, 0, 0, 0, m, n, k, 78)
    good, bad = C.copy(), C.copy()
    oracle.gemm_naive_ld(0, 0, 0, m, n, k, 1.0, A, lda, B, ldb, 0.25, good, ldc)
    oracle.gemm(0, 0, 0, m, n, k, 1.0, A, lda, B, ldb, 0.0, bad, ldc, 1)  # planted: beta lost
    assert oracle.rel_fro_err(bad.reshape(m, n), good.reshape(m, n)) > 1e-3


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_relu_special_values(dtype):
    """relu.cpp:38-41: greater_than_zero(x) ? x : 0 -- NaN, -0 and -inf map to +0."""
    x = np.array([1.5, -2.0, 0.0, -0.0, np.inf, -np.inf, np.nan, 1e-300, -1e-300, 3.0], dtype)
    oracle.relu(x)
    want = np.array([1.5, 0, 0, 0, np.inf, 0, 0, 1e-300, 0, 3.0], dtype)
    np.testing.assert_array_equal(x, want)
    assert not np.signbit(x).any()  # no -0 survives
