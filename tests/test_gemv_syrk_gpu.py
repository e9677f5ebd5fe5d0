"""GPU parity tests of GEMV (sbx_sgemv / sbx_dgemv) and SYRK
(sbx_{s,d}syrk_strided_batched) through the C ABI, against the CPU oracle on
identical seeded inputs.

Bars: normwise relative error <= 1e-5 (fp32) / 1e-12 (fp64) against the
oracle (sums in double); the reference's known answers exactly
(tests/blas/level2/test_gemv.cpp, tests/blas/level3/test_syrk.cpp); quick
returns bit for bit; SYRK's other triangle and every element outside the
logical window (ld padding, batch gaps, vector strides) bit for bit untouched;
repeated runs bit-identical (the chunked reductions are ordered).
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

TOL = {np.float32: 1e-5, np.float64: 1e-12}
SEED = 20261207


def _dev(x, cuda, offset=0):
    """Device copy of x starting `offset` elements into a fresh buffer."""
    import torch
    t = torch.zeros(x.size + offset, dtype=torch.float32 if x.dtype == np.float32
                    else torch.float64, device=cuda)
    t[offset:] = torch.from_numpy(x).to(cuda)
    return t, t.data_ptr() + offset * t.element_size()


def _code(dtype):
    import sushiblas_amd as sbx
    return sbx.F32 if dtype == np.float32 else sbx.F64


def _alen(layout, rows, cols, ld):
    if rows == 0 or cols == 0:
        return 1
    return (rows - 1) * ld + cols if layout == 0 else (cols - 1) * ld + rows


def _err(got, want):
    g = got.astype(np.float64)
    w = want.astype(np.float64)
    den = np.linalg.norm(w)
    return float(np.linalg.norm(g - w) / den) if den > 0 else float(np.linalg.norm(g))


# -- GEMV -------------------------------------------------------------------------

def run_gemv(cuda, dtype, layout, trans, m, n, alpha, beta, seed, incx=1, incy=1, pad=0,
             offsets=(0, 0, 0), y_init=None, nan_pad=False):
    import torch
    import sushiblas_amd as sbx
    lda = max(n if layout == 0 else m, 1) + pad
    A = oracle.fill_uniform(_alen(layout, m, n, lda), dtype, seed, 0)
    if nan_pad:  # the ld padding must never be read
        A[np.arange(A.size) % lda >= (n if layout == 0 else m)] = np.nan
    xlen, ylen = (m, n) if trans else (n, m)
    x = oracle.fill_uniform(max((xlen - 1) * incx + 1, 1), dtype, seed, 1)
    y = y_init.copy() if y_init is not None else \
        oracle.fill_uniform(max((ylen - 1) * incy + 1, 1), dtype, seed, 2)
    dA, pA = _dev(A, cuda, offsets[0])
    dx, px = _dev(x, cuda, offsets[1])
    dy, py = _dev(y, cuda, offsets[2])
    sbx.gemv(_code(dtype), layout, trans, m, n, alpha, pA, lda, px, incx, beta, py, incy)
    torch.cuda.synchronize()
    got = dy[offsets[2]:].cpu().numpy()
    want = y.copy()
    oracle.gemv(layout, trans, m, n, alpha, A, lda, x, incx, beta, want, incy)
    print(f"gemv {np.dtype(dtype).name} layout={layout} trans={trans} m={m} n={n} "
          f"inc=({incx},{incy}) pad={pad} off={offsets}", flush=True)
    return got, want, y


def test_gemv_known_answer(cuda):
    """test_gemv.cpp SimpleGEMV: [[1,2,3],[4,5,6]] x [1,1,1] -> [6, 15]."""
    import sushiblas_amd as sbx
    A = np.arange(1, 7, dtype=np.float32)
    x = np.ones(3, np.float32)
    y = np.zeros(2, np.float32)
    dA, pA = _dev(A, cuda)
    dx, px = _dev(x, cuda)
    dy, py = _dev(y, cuda)
    sbx.gemv(sbx.F32, 0, 0, 2, 3, 1.0, pA, 3, px, 1, 0.0, py, 1)
    assert dy.cpu().tolist() == [6, 15]


# Shapes chosen to reach each kernel form: row-dot with 64/16/4 lanes per row,
# with and without column chunks; column-axpy with 256..1 column threads, with
# and without row chunks.
GEMV_CASES = [
    (4096, 4096), (257, 1023), (1, 100000), (100000, 1), (8192, 64), (64, 8192),
    (64, 262144), (131072, 16), (3, 5), (1000, 300), (2048, 2048),
]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("trans", [0, 1])
def test_gemv_matches_oracle(cuda, dtype, layout, trans):
    for i, (m, n) in enumerate(GEMV_CASES):
        got, want, y0 = run_gemv(cuda, dtype, layout, trans, m, n, 1.5, -0.5, SEED + i)
        err = _err(got, want)
        assert err <= TOL[dtype], (m, n, err)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("trans", [0, 1])
def test_gemv_strided_padded_unaligned(cuda, dtype, trans):
    """incx/incy > 1 (the row-dot form then reads x and A element by element),
    lda padding and base pointers off 16-byte alignment; entries between
    strided y elements untouched."""
    for m, n in ((300, 517), (5000, 70), (33, 20000)):
        for incx, incy, pad, off in ((2, 3, 3, (1, 1, 1)), (1, 1, 1, (0, 0, 0)),
                                     (1, 1, 0, (1, 0, 0)), (3, 1, 4, (0, 1, 0))):
            got, want, y0 = run_gemv(cuda, dtype, 0, trans, m, n, 0.75, 1.25, SEED + 50,
                                     incx, incy, pad, off)
            assert _err(got[::incy], want[::incy]) <= TOL[dtype]
            mask = np.ones(got.size, bool)
            mask[::incy] = False
            assert np.array_equal(got[mask], y0[mask])


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("trans", [0, 1])
def test_gemv_odd_ld_vector_loads(cuda, dtype, layout, trans):
    """Odd leading dimensions and misaligned bases: A is still read in
    16-byte vectors (at 4/8-byte aligned addresses); NaN in the ld padding
    must not reach y."""
    for m, n, pad in ((4095, 3001, 0), (1001, 777, 3), (33, 20001, 1), (20001, 33, 5), (7, 5, 1)):
        got, want, _ = run_gemv(cuda, dtype, layout, trans, m, n, 0.5, 1.5, SEED + 70, pad=pad,
                                offsets=(1, 0, 1), nan_pad=True)
        assert np.isfinite(got).all(), (m, n)
        assert _err(got, want) <= TOL[dtype], (m, n)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_gemv_quick_returns(cuda, dtype):
    """m == 0 or n == 0: y untouched (even with beta != 1); alpha == 0:
    y = beta*y; beta == 0: y is not read (NaN does not propagate)."""
    y = np.array([1.0, np.nan, -2.0, 4.0], dtype)
    got, _, _ = run_gemv(cuda, dtype, 0, 0, 4, 0, 1.0, 0.5, SEED, y_init=y)
    assert np.array_equal(got, y, equal_nan=True)
    got, _, _ = run_gemv(cuda, dtype, 0, 1, 0, 4, 1.0, 0.5, SEED, y_init=y)
    assert np.array_equal(got, y, equal_nan=True)
    got, want, _ = run_gemv(cuda, dtype, 0, 0, 4, 7, 0.0, 0.5, SEED, y_init=y)
    assert np.array_equal(got, (dtype(0.5) * y).astype(dtype), equal_nan=True)
    got, _, _ = run_gemv(cuda, dtype, 0, 0, 4, 7, 0.0, 0.0, SEED, y_init=y)
    assert got.tolist() == [0, 0, 0, 0]
    got, want, _ = run_gemv(cuda, dtype, 0, 1, 7, 4, 1.0, 0.0, SEED, y_init=y)
    assert not np.isnan(got).any() and _err(got, want) <= TOL[dtype]


def test_gemv_deterministic(cuda):
    """The chunked reductions are ordered: two runs give the same bits."""
    for trans, (m, n) in ((0, (64, 262144)), (1, (131072, 16)), (1, (4096, 4096))):
        a, _, _ = run_gemv(cuda, np.float32, 0, trans, m, n, 1.0, 0.0, SEED + 9)
        b, _, _ = run_gemv(cuda, np.float32, 0, trans, m, n, 1.0, 0.0, SEED + 9)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_gemv_full_size(cuda):
    """16384 x 16384 fp32 (1 GiB of A), both transposes, against the oracle."""
    for trans in (0, 1):
        got, want, _ = run_gemv(cuda, np.float32, 0, trans, 16384, 16384, 1.0, 0.5, SEED + 11)
        assert _err(got, want) <= TOL[np.float32]


# -- SYRK -------------------------------------------------------------------------

def run_syrk(cuda, dtype, layout, upper, trans, n, k, alpha, beta, seed, pad=(0, 0),
             offsets=(0, 0), batch=1, gaps=(0, 0), sentinel=True):
    import torch
    import sushiblas_amd as sbx
    ar, ac = (k, n) if trans else (n, k)
    lda = max(ac if layout == 0 else ar, 1) + pad[0]
    ldc = max(n, 1) + pad[1]
    na = _alen(layout, ar, ac, lda)
    nc = _alen(layout, n, n, ldc)
    sa, sc = na + gaps[0], nc + gaps[1]
    A = oracle.fill_uniform(sa * batch if batch > 1 else na, dtype, seed, 0)
    C = oracle.fill_uniform(sc * batch if batch > 1 else nc, dtype, seed, 1)
    if sentinel and n > 0:
        # NaN in the other triangle: it must be neither read nor written
        i, j = np.tril_indices(n, -1) if upper else np.triu_indices(n, 1)
        idx = i * ldc + j if layout == 0 else i + j * ldc
        for b in range(batch):
            C[b * sc + idx] = np.nan
    dA, pA = _dev(A, cuda, offsets[0])
    dC, pC = _dev(C, cuda, offsets[1])
    sbx.syrk(_code(dtype), layout, upper, trans, n, k, alpha, pA, lda, sa if batch > 1 else 0,
             beta, pC, ldc, sc if batch > 1 else 0, batch)
    torch.cuda.synchronize()
    got = dC[offsets[1]:].cpu().numpy()
    want = C.copy()
    oracle.syrk_strided_batched(layout, upper, trans, n, k, alpha, A, lda,
                                sa if batch > 1 else 0, beta, want, ldc,
                                sc if batch > 1 else 0, batch)
    print(f"syrk {np.dtype(dtype).name} layout={layout} upper={upper} trans={trans} n={n} "
          f"k={k} batch={batch} pad={pad} off={offsets}", flush=True)
    return got, want, C


def _check_syrk(got, want, C0, dtype):
    nanmask = np.isnan(C0)
    # untouched: the sentinel triangle, ld padding and batch gaps (bit for bit)
    same = np.isnan(want) == np.isnan(got)
    assert same.all()
    fin = ~np.isnan(want)
    assert np.array_equal(got[nanmask], C0[nanmask], equal_nan=True)
    assert _err(got[fin], want[fin]) <= TOL[dtype]


def test_syrk_known_answers(cuda):
    import sushiblas_amd as sbx
    A = np.arange(1, 7, dtype=np.float32)
    C = np.zeros(9, np.float32)
    dA, pA = _dev(A, cuda)
    dC, pC = _dev(C, cuda)
    sbx.syrk(sbx.F32, 0, 0, 0, 3, 2, 1.0, pA, 2, 0, 0.0, pC, 3, 0)  # SimpleSYRK
    assert dC.cpu().tolist() == [5, 0, 0, 11, 25, 0, 17, 39, 61]
    C = np.zeros(4, np.float32)
    dC, pC = _dev(C, cuda)
    sbx.syrk(sbx.F32, 1, 0, 1, 2, 3, 1.0, pA, 3, 0, 0.0, pC, 2, 0)  # SimpleSYRKColumnMajor
    assert dC.cpu().tolist() == [14, 32, 0, 77]


# (n, k): 128x128 tiles with split-K tails, the three-per-CU 128x128 tile
# whole (4416) and with a split tail (4928), 256x256 tiles (7680; fp32
# only), ragged edges, tiny sizes
SYRK_CASES = [(1, 1), (3, 2), (130, 257), (1000, 300), (2048, 512), (4100, 64), (4416, 256),
              (4928, 256), (7680, 32)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("upper", [0, 1])
@pytest.mark.parametrize("trans", [0, 1])
def test_syrk_matches_oracle(cuda, dtype, layout, upper, trans):
    import sushiblas_amd as sbx
    for i, (n, k) in enumerate(SYRK_CASES):
        if dtype == np.float64 and n > 4100:
            continue
        lda = (n if trans else k) if layout == 0 else (k if trans else n)
        sdt = sbx.F32 if dtype == np.float32 else sbx.F64
        print(f"syrk case {n}x{k}: {sbx.syrk_select(sdt, layout, upper, trans, n, k, lda, n)}",
              flush=True)
        got, want, C0 = run_syrk(cuda, dtype, layout, upper, trans, n, k, 0.5, 1.5, SEED + i,
                                 sentinel=n <= 1000)
        if n <= 1000:
            _check_syrk(got, want, C0, dtype)
        else:
            assert _err(got, want) <= TOL[dtype], (n, k)


@pytest.mark.parametrize("layout,upper,trans", [(0, 0, 0), (0, 1, 1), (1, 0, 1), (1, 1, 0)])
def test_syrk_largest_tile_ragged(cuda, layout, upper, trans):
    """The 256x256 tile (8 waves, one per CU), which only SYRK uses: n = 7553
    leaves a partial tile on both edges of the triangle, k = 257 a K tail
    (8*32 + 1), and lda is padded."""
    import sushiblas_amd as sbx
    n, k = 7553, 257
    lda = (n if trans else k) if layout == 0 else (k if trans else n)
    name = sbx.syrk_select(sbx.F32, layout, upper, trans, n, k, lda + 3, n + 1)
    print(f"syrk largest-tile case {n}x{k}: {name}", flush=True)
    assert name == "mfma_f32_256x256x32_w4x2", name
    got, want, C0 = run_syrk(cuda, np.float32, layout, upper, trans, n, k, 0.5, 1.5, SEED + 60,
                             pad=(3, 1), sentinel=False)
    assert _err(got, want) <= TOL[np.float32]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_syrk_padded_unaligned_batched(cuda, dtype):
    for upper in (0, 1):
        got, want, C0 = run_syrk(cuda, dtype, 0, upper, 0, 300, 129, 1.0, 0.5, SEED + 20,
                                 pad=(3, 5), offsets=(1, 1))
        _check_syrk(got, want, C0, dtype)
        got, want, C0 = run_syrk(cuda, dtype, 1, upper, 1, 97, 200, -1.0, 1.0, SEED + 21,
                                 batch=4, gaps=(7, 9))
        _check_syrk(got, want, C0, dtype)
        # a batch of few triangle tiles and a long K: every entry's tiles split
        got, want, C0 = run_syrk(cuda, dtype, 0, upper, 0, 200, 3000, 0.5, -1.0, SEED + 22,
                                 batch=3, gaps=(5, 3))
        _check_syrk(got, want, C0, dtype)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_syrk_quick_returns(cuda, dtype):
    """alpha == 0 or k == 0: C = beta*C on the triangle only; beta == 0 there
    writes zeros without reading (the triangle's own NaN does not survive)."""
    for alpha, k, beta in ((0.0, 16, 0.5), (1.0, 0, 2.0), (0.0, 16, 0.0)):
        got, want, C0 = run_syrk(cuda, dtype, 0, 0, 0, 70, k, alpha, beta, SEED + 30)
        assert np.array_equal(got, want, equal_nan=True)


def test_syrk_generic_fallback(cuda):
    """lda too large for 32-bit tile offsets: the generic kernel, triangle-masked."""
    got, want, C0 = run_syrk(cuda, np.float32, 0, 0, 0, 64, 64, 1.0, 1.0, SEED + 40,
                             pad=((1 << 22) - 64, 0))
    _check_syrk(got, want, C0, np.float32)


def test_syrk_deterministic(cuda):
    a, _, _ = run_syrk(cuda, np.float32, 0, 0, 0, 1000, 300, 1.0, 0.0, SEED + 50,
                       sentinel=False)
    b, _, _ = run_syrk(cuda, np.float32, 0, 0, 0, 1000, 300, 1.0, 0.0, SEED + 50,
                       sentinel=False)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
