"""Pins the GEMV and SYRK routines of the CPU oracle (oracle/sbo.c) before the
GPU kernels are checked against them.

Checks independent of the oracle's own loops:
  * the reference's known answers: tests/blas/level2/test_gemv.cpp
    (SimpleGEMV) and tests/blas/level3/test_syrk.cpp (SimpleSYRK,
    SimpleSYRKColumnMajor);
  * a dense long-double evaluation through numpy on small random inputs;
  * numpy/OpenBLAS in float64;
  * exact invariants on integer-valued inputs (every partial sum exact in
    double, so any correct evaluation order gives the same bits): SYRK equals
    the GEMM oracle's A*A^T on the triangle, GEMV equals the GEMM oracle with
    one column, column-major equals row-major with flipped flags, batched
    equals a loop, strided vectors equal packed copies;
  * netlib quick returns and the untouched triangle, bit for bit;
  * planted mistakes (wrong triangle, wrong transpose, ignored increment,
    dropped beta) that the checks must catch.
"""
import numpy as np
import pytest

import oracle


def _dense(layout, X, rows, cols, ld):
    """The rows x cols matrix stored in X (layout, ld) as float64 (own index path)."""
    full = np.zeros(max(rows if layout == 0 else cols, 1) * ld, np.float64)
    full[:X.size] = X[:full.size]
    if layout == 0:
        return full.reshape(-1, ld)[:rows, :cols]
    return full.reshape(-1, ld)[:cols, :rows].T


def _len(layout, rows, cols, ld):
    if rows == 0 or cols == 0:
        return 1
    return (rows - 1) * ld + cols if layout == 0 else (cols - 1) * ld + rows


# -- reference known answers ------------------------------------------------------

def test_known_answer_simple_gemv():
    """test_gemv.cpp SimpleGEMV: [[1,2,3],[4,5,6]] x [1,1,1] = [6, 15]."""
    A = np.arange(1, 7, dtype=np.float32)
    x = np.ones(3, np.float32)
    y = np.zeros(2, np.float32)
    oracle.gemv(0, 0, 2, 3, 1.0, A, 3, x, 1, 0.0, y, 1)
    assert y.tolist() == [6, 15]


def test_known_answer_simple_syrk():
    """test_syrk.cpp SimpleSYRK: lower of A A^T, A = [[1,2],[3,4],[5,6]]."""
    A = np.arange(1, 7, dtype=np.float32)
    C = np.zeros(9, np.float32)
    oracle.syrk(0, 0, 0, 3, 2, 1.0, A, 2, 0.0, C, 3)
    assert C.tolist() == [5, 0, 0, 11, 25, 0, 17, 39, 61]


def test_known_answer_simple_syrk_column_major():
    """test_syrk.cpp SimpleSYRKColumnMajor: lower of A^T A, A (3x2) column-major."""
    A = np.arange(1, 7, dtype=np.float32)
    C = np.zeros(4, np.float32)
    oracle.syrk(1, 0, 1, 2, 3, 1.0, A, 3, 0.0, C, 2)
    assert C.tolist() == [14, 32, 0, 77]


# -- long-double brute force ----------------------------------------------------

GEMV_SHAPES = [(1, 1), (5, 3), (65, 257), (300, 7), (7, 300)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("incx,incy", [(1, 1), (3, 2)])
def test_gemv_matches_long_double(dtype, layout, trans, incx, incy):
    for idx, (m, n) in enumerate(GEMV_SHAPES):
        lda = (n if layout == 0 else m) + 2
        A = oracle.fill_uniform(_len(layout, m, n, lda), dtype, 500 + idx, 0)
        xlen, ylen = (m, n) if trans else (n, m)
        x = oracle.fill_uniform((xlen - 1) * incx + 1, dtype, 500 + idx, 1)
        y = oracle.fill_uniform((ylen - 1) * incy + 1, dtype, 500 + idx, 2)
        alpha, beta = 1.25, -0.5
        op = _dense(layout, A, m, n, lda).astype(np.longdouble)
        if trans:
            op = op.T
        xv = x[::incx].astype(np.longdouble)
        want = np.longdouble(alpha) * (op @ xv) + np.longdouble(beta) * y[::incy].astype(np.longdouble)
        got = y.copy()
        oracle.gemv(layout, trans, m, n, alpha, A, lda, x, incx, beta, got, incy)
        err = np.linalg.norm((got[::incy] - want.astype(dtype)).astype(np.float64)) / \
            max(np.linalg.norm(want.astype(np.float64)), 1e-300)
        assert err <= (1e-7 if dtype == np.float32 else 1e-15), (m, n, err)
        # elements between the strided y entries are untouched
        mask = np.ones(got.size, bool)
        mask[::incy] = False
        assert np.array_equal(got[mask], y[mask])


SYRK_SHAPES = [(1, 1), (3, 2), (65, 31), (130, 257), (64, 0)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("upper", [0, 1])
@pytest.mark.parametrize("trans", [0, 1])
def test_syrk_matches_long_double(dtype, layout, upper, trans):
    for idx, (n, k) in enumerate(SYRK_SHAPES):
        ar, ac = (k, n) if trans else (n, k)
        lda = max((ac if layout == 0 else ar), 1) + 1
        ldc = n + 3
        A = oracle.fill_uniform(_len(layout, ar, ac, lda), dtype, 600 + idx, 0)
        C = oracle.fill_uniform(_len(layout, n, n, ldc), dtype, 600 + idx, 1)
        alpha, beta = -0.75, 1.5
        op = _dense(layout, A, ar, ac, lda).astype(np.longdouble)
        if trans:
            op = op.T
        Cd = _dense(layout, C, n, n, ldc).astype(np.longdouble)
        full = np.longdouble(alpha) * (op @ op.T) + np.longdouble(beta) * Cd
        got = C.copy()
        oracle.syrk(layout, upper, trans, n, k, alpha, A, lda, beta, got, ldc)
        G = _dense(layout, got, n, n, ldc)
        C0 = _dense(layout, C, n, n, ldc)
        tri = np.triu(np.ones((n, n), bool)) if upper else np.tril(np.ones((n, n), bool))
        want = full.astype(dtype).astype(np.float64)
        err = np.linalg.norm((G - want)[tri]) / max(np.linalg.norm(want[tri]), 1e-300)
        assert err <= (1e-7 if dtype == np.float32 else 1e-15), (n, k, err)
        # the other triangle and the ldc padding are bit-for-bit untouched
        assert np.array_equal(G[~tri], C0[~tri])
        inside = np.zeros(got.size, bool)
        for i in range(n):
            for j in range(n):
                inside[i * ldc + j if layout == 0 else i + j * ldc] = True
        assert np.array_equal(got[~inside], C[~inside])


# -- independent host BLAS ---------------------------------------------------------

def test_against_numpy_blas():
    m, n, k = 257, 193, 129
    A = oracle.fill_uniform(m * n, np.float64, 700, 0)
    x = oracle.fill_uniform(n, np.float64, 700, 1)
    y = np.zeros(m)
    oracle.gemv(0, 0, m, n, 1.0, A, n, x, 1, 0.0, y, 1)
    want = A.reshape(m, n) @ x
    assert np.linalg.norm(y - want) / np.linalg.norm(want) < 1e-14
    S = oracle.fill_uniform(n * k, np.float64, 701, 0)
    C = np.zeros(n * n)
    oracle.syrk(0, 1, 0, n, k, 1.0, S, k, 0.0, C, n)
    full = S.reshape(n, k) @ S.reshape(n, k).T
    tri = np.triu(np.ones((n, n), bool))
    assert np.linalg.norm(C.reshape(n, n)[tri] - full[tri]) / np.linalg.norm(full[tri]) < 1e-14


# -- exact invariants on integer-valued inputs --------------------------------

def _ints(size, seed, lo=-8, hi=9, dtype=np.float64):
    return np.random.default_rng(seed).integers(lo, hi, size).astype(dtype)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("trans", [0, 1])
def test_syrk_equals_gemm_on_the_triangle(dtype, trans):
    n, k = 77, 45
    A = _ints(n * k, 1, dtype=dtype)
    C = _ints(n * n, 2, dtype=dtype)
    lda = n if trans else k
    ref = C.copy()
    # GEMM with B = A: op(A) op(A)^T
    oracle.gemm(0, trans, 1 - trans, n, n, k, 2.0, A, lda, A, lda, -1.0, ref, n)
    for upper in (0, 1):
        got = C.copy()
        oracle.syrk(0, upper, trans, n, k, 2.0, A, lda, -1.0, got, n)
        tri = np.triu(np.ones((n, n), bool)) if upper else np.tril(np.ones((n, n), bool))
        G, R, C0 = got.reshape(n, n), ref.reshape(n, n), C.reshape(n, n)
        assert np.array_equal(G[tri], R[tri])
        assert np.array_equal(G[~tri], C0[~tri])


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_syrk_column_major_is_row_major_with_flipped_flags(dtype):
    n, k = 40, 23
    for trans in (0, 1):
        for upper in (0, 1):
            A = _ints(n * k, 3, dtype=dtype)
            C = _ints(n * n, 4, dtype=dtype)
            lda = k if trans else n  # column-major: A n x k has ld n; k x n has ld k
            a, b = C.copy(), C.copy()
            oracle.syrk(1, upper, trans, n, k, 1.5, A, lda, 0.5, a, n)
            oracle.syrk(0, 1 - upper, 1 - trans, n, k, 1.5, A, lda, 0.5, b, n)
            assert np.array_equal(a, b)


def test_gemv_equals_gemm_with_one_column():
    m, n = 61, 37
    A = _ints(m * n, 5)
    x = _ints(n, 6)
    y = _ints(m, 7)
    got, ref = y.copy(), y.copy()
    oracle.gemv(0, 0, m, n, 3.0, A, n, x, 1, 2.0, got, 1)
    oracle.gemm(0, 0, 0, m, 1, n, 3.0, A, n, x, 1, 2.0, ref, 1)
    assert np.array_equal(got, ref)
    # transposed: y (n) = A^T x (m), against GEMM with transA
    x2 = _ints(m, 8)
    y2 = _ints(n, 9)
    got, ref = y2.copy(), y2.copy()
    oracle.gemv(0, 1, m, n, 3.0, A, n, x2, 1, 2.0, got, 1)
    oracle.gemm(0, 1, 0, n, 1, m, 3.0, A, n, x2, 1, 2.0, ref, 1)
    assert np.array_equal(got, ref)


def test_gemv_column_major_is_transposed_row_major():
    m, n = 29, 53
    A = _ints(m * n, 10)  # column-major m x n, ld m == row-major n x m
    for trans in (0, 1):
        xlen, ylen = (m, n) if trans else (n, m)
        x = _ints(xlen, 11)
        y = _ints(ylen, 12)
        a, b = y.copy(), y.copy()
        oracle.gemv(1, trans, m, n, 1.0, A, m, x, 1, 1.0, a, 1)
        oracle.gemv(0, 1 - trans, n, m, 1.0, A, m, x, 1, 1.0, b, 1)
        assert np.array_equal(a, b)


def test_strided_vectors_equal_packed_copies():
    m, n = 33, 70
    A = _ints(m * n, 13)
    x = _ints(n * 4, 14)
    y = _ints(m * 3, 15)
    got = y.copy()
    oracle.gemv(0, 0, m, n, 1.0, A, n, x, 4, -1.0, got, 3)
    packed = y[::3].copy()
    oracle.gemv(0, 0, m, n, 1.0, A, n, x[::4].copy(), 1, -1.0, packed, 1)
    assert np.array_equal(got[::3], packed)


def test_syrk_batched_equals_loop():
    n, k, batch = 19, 11, 4
    sa, sc = n * k + 5, n * n + 3
    A = _ints(sa * batch, 16)
    C = _ints(sc * batch, 17)
    got = C.copy()
    oracle.syrk_strided_batched(0, 0, 0, n, k, 1.0, A, k, sa, 1.0, got, n, sc, batch)
    for b in range(batch):
        one = C[b * sc:b * sc + n * n].copy()
        oracle.syrk(0, 0, 0, n, k, 1.0, A[b * sa:b * sa + n * k].copy(), k, 1.0, one, n)
        assert np.array_equal(got[b * sc:b * sc + n * n], one)
        assert np.array_equal(got[b * sc + n * n:(b + 1) * sc], C[b * sc + n * n:(b + 1) * sc])


# -- quick returns ----------------------------------------------------------------

def test_gemv_quick_returns():
    A = _ints(12, 18)
    x = _ints(4, 19)
    y = np.array([1.0, np.nan, -2.0])
    got = y.copy()
    oracle.gemv(0, 0, 3, 0, 1.0, A, 1, x, 1, 0.5, got, 1)        # n == 0: y untouched
    assert np.array_equal(got, y, equal_nan=True)
    got = y.copy()
    oracle.gemv(0, 0, 3, 4, 0.0, A, 4, x, 1, 0.5, got, 1)        # alpha == 0: beta*y
    assert np.array_equal(got, 0.5 * y, equal_nan=True)
    got = y.copy()
    oracle.gemv(0, 0, 3, 4, 0.0, A, 4, x, 1, 0.0, got, 1)        # beta == 0: y not read
    assert got.tolist() == [0.0, 0.0, 0.0]
    got = y.copy()
    oracle.gemv(0, 0, 3, 4, 1.0, A, 4, x, 1, 0.0, got, 1)        # NaN in y ignored
    assert not np.isnan(got).any()


def test_syrk_quick_returns():
    n = 5
    C = _ints(n * n, 20)
    C[7] = np.nan  # row 1, col 2: in the upper triangle
    A = _ints(n * 3, 21)
    lower = np.tril(np.ones((n, n), bool)).ravel()
    got = C.copy()
    oracle.syrk(0, 0, 0, n, 0, 1.0, A, 1, 0.5, got, n)           # k == 0: beta*C on the triangle
    assert np.array_equal(got[lower], 0.5 * C[lower])
    assert np.array_equal(got[~lower], C[~lower], equal_nan=True)
    got = C.copy()
    oracle.syrk(0, 1, 0, n, 3, 0.0, A, 3, 0.0, got, n)           # alpha == beta == 0: zeros
    assert np.array_equal(got[~lower | np.eye(n, dtype=bool).ravel()],
                          np.zeros(int((~lower | np.eye(n, dtype=bool).ravel()).sum())))


def test_rejects_bad_arguments():
    A = np.zeros(16)
    y = np.zeros(4)
    with pytest.raises(ValueError):
        oracle.gemv(0, 0, 4, 4, 1.0, A, 3, A, 1, 0.0, y, 1)      # lda < n
    with pytest.raises(ValueError):
        oracle.gemv(0, 0, 4, 4, 1.0, A, 4, A, 0, 0.0, y, 1)      # incx == 0
    with pytest.raises(ValueError):
        oracle.syrk(0, 0, 0, 4, 4, 1.0, A, 4, 0.0, A.copy(), 3)  # ldc < n
    with pytest.raises(ValueError):
        oracle.syrk(2, 0, 0, 4, 4, 1.0, A, 4, 0.0, A.copy(), 4)  # bad layout


# -- planted mistakes -----------------------------------------------------------------

def _syrk_truth(n, k, seed):
    A = oracle.fill_uniform(n * k, np.float64, seed, 0)
    full = A.reshape(n, k) @ A.reshape(n, k).T
    return A, full


def test_checks_catch_the_wrong_triangle():
    n, k = 24, 16
    A, full = _syrk_truth(n, k, 800)
    C = np.full(n * n, -3.0)
    oracle.syrk(0, 1, 0, n, k, 1.0, A, k, 0.0, C, n)  # planted: upper instead of lower
    lower = np.tril(np.ones((n, n), bool), -1)
    assert np.abs(C.reshape(n, n)[lower] - full[lower]).max() > 0.1


def test_checks_catch_a_wrong_transpose():
    m, n = 40, 40
    A = oracle.fill_uniform(m * n, np.float64, 801, 0)
    x = oracle.fill_uniform(n, np.float64, 801, 1)
    y = np.zeros(m)
    oracle.gemv(0, 1, m, n, 1.0, A, n, x, 1, 0.0, y, 1)  # planted: transposed
    want = A.reshape(m, n) @ x
    assert np.linalg.norm(y - want) / np.linalg.norm(want) > 0.1


def test_checks_catch_an_ignored_increment():
    m, n = 30, 20
    A = oracle.fill_uniform(m * n, np.float64, 802, 0)
    x = oracle.fill_uniform(2 * n, np.float64, 802, 1)
    y = np.zeros(m)
    oracle.gemv(0, 0, m, n, 1.0, A, n, x, 1, 0.0, y, 1)  # planted: incx 1 instead of 2
    want = A.reshape(m, n) @ x[::2]
    assert np.linalg.norm(y - want) / np.linalg.norm(want) > 0.1


def test_checks_catch_a_dropped_beta_term():
    n, k = 20, 10
    A, full = _syrk_truth(n, k, 803)
    C0 = oracle.fill_uniform(n * n, np.float64, 803, 1)
    C = C0.copy()
    oracle.syrk(0, 0, 0, n, k, 1.0, A, k, 0.0, C, n)  # planted: beta lost
    want = full + 0.5 * C0.reshape(n, n)
    lower = np.tril(np.ones((n, n), bool))
    got = C.reshape(n, n)
    assert np.linalg.norm(got[lower] - want[lower]) / np.linalg.norm(want[lower]) > 1e-3
