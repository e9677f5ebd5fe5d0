"""GPU parity tests of the fused GEMM+ReLU epilogue (sbx_gemm_fused) and the
stand-alone ReLU (sbx_relu), through the C ABI.

The caller pattern is the reference's integration tests: Level3::gemm then
NonLinearOps::relu on C (tests/runtime/test_framework_sim.cpp:51-57,109-110);
ReLU is x > 0 ? x : 0 (src/ops/math/nonlinear/relu.cpp:38-41).  Bars:
- fused result vs oracle.gemm followed by oracle.relu: normwise relative
  Frobenius error <= 1e-5 (fp32) / 1e-12 (fp64), no negative, NaN or -0;
- fused result vs the same GEMM followed by sbx_relu: bit-identical (the
  dispatcher picks the same kernel, and the epilogue rectifies the very value
  the unfused GEMM would have stored);
- sbx_relu vs oracle.relu: bit-identical, special values included.
"""
import numpy as np
import pytest

import oracle
from gemm_cases import TOL, c_window, make_inputs, normwise, run_oracle, run_sbx

pytestmark = pytest.mark.gpu

SEED = 20261205


def _fused_case(dev, dtype, layout, ta, tb, m, n, k, alpha, beta, seed, pad=(0, 0, 0),
                offsets=(0, 0, 0)):
    import sushiblas_amd as sbx
    A, lda, B, ldb, C, ldc = make_inputs(dtype, layout, ta, tb, m, n, k, seed, pad)
    fused = run_sbx(dev, dtype, layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                    offsets=offsets, epilogue=sbx.EPILOGUE_RELU)
    plain = run_sbx(dev, dtype, layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                    offsets=offsets)
    want = run_oracle(layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
    want_win = c_window(layout, want, m, n, ldc)
    oracle.relu(want_win)
    got_win = c_window(layout, fused, m, n, ldc)
    err = oracle.rel_fro_err(got_win, want_win) if want_win.size else 0.0
    print(f"fused dtype={np.dtype(dtype).name} layout={layout} tA={ta} tB={tb} m={m} n={n} "
          f"k={k} alpha={alpha} beta={beta} err={err:.3e}", flush=True)
    assert err <= TOL[dtype]
    assert not np.isnan(got_win).any()
    assert not np.signbit(got_win).any()          # no negatives, no -0
    # the unfused pair, rectified on the host: identical bits
    plain_win = c_window(layout, plain, m, n, ldc)
    oracle.relu(plain_win)
    assert np.array_equal(got_win.view(np.uint8), plain_win.view(np.uint8))
    # elements outside the m x n window (padding of ldc) are untouched
    if pad[2]:
        mask = np.ones(C.size, bool)
        idx = np.arange(C.size)
        inner = (idx % ldc) < (n if layout == 0 else m)
        mask[inner] = False
        assert np.array_equal(fused[mask], C[mask])
    return err


@pytest.mark.parametrize("dtype,layout,ta,tb,m,n,k,alpha,beta", [
    (np.float32, 0, 0, 0, 4096, 4096, 64, 1.0, 0.0),      # 256x128 tiles
    (np.float32, 0, 0, 1, 1000, 777, 300, 1.5, 0.5),       # 128x128 + split-K
    (np.float32, 0, 1, 0, 512, 512, 512, 1.0, 1.0),        # split-K 8
    (np.float32, 0, 0, 0, 8192, 64, 1024, 1.0, -1.0),      # 128x64 tall-skinny
    (np.float32, 1, 1, 1, 37, 1000, 300, -2.0, 0.25),      # 64x128 + split-K, column-major
    (np.float64, 0, 0, 0, 1024, 1024, 256, 1.0, 0.5),      # f64 128x128
    (np.float64, 1, 0, 1, 4096, 64, 512, 0.5, 0.0),        # f64 128x64
    (np.float64, 0, 1, 1, 33, 700, 129, 1.0, 1.0),         # f64 64x128
])
def test_fused_relu_matches_oracle(cuda, dtype, layout, ta, tb, m, n, k, alpha, beta):
    _fused_case(cuda, dtype, layout, ta, tb, m, n, k, alpha, beta, SEED)


def test_fused_relu_padded_and_unaligned(cuda):
    """Leading-dimension padding and pointers off 16-byte alignment (scalar loads)."""
    _fused_case(cuda, np.float32, 0, 0, 0, 300, 257, 129, 1.25, 0.5, SEED + 1, pad=(3, 5, 7),
                offsets=(1, 3, 1))
    _fused_case(cuda, np.float64, 0, 1, 0, 129, 65, 47, 1.0, 1.0, SEED + 2, pad=(1, 0, 3),
                offsets=(1, 1, 1))


def test_fused_relu_generic_kernel(cuda):
    """A leading dimension too large for 32-bit buffer offsets in any MFMA tile
    (32 rows x 2^24 floats spans 2 GiB): generic kernel + ReLU.  Three rows
    keep the buffer small."""
    import sushiblas_amd as sbx
    assert sbx.gemm_select(0, 0, 0, 0, 3, 64, 64, 1 << 24, 64, 64) == "generic_64x64x16"
    import torch
    m, n, k = 3, 64, 64
    lda = 1 << 24
    dA = torch.zeros((m - 1) * lda + k, dtype=torch.float32, device=cuda)
    A = oracle.fill_uniform(m * k, np.float32, SEED + 3, 0).reshape(m, k)
    dA.view(-1)[: (m - 1) * lda + k].as_strided((m, k), (lda, 1)).copy_(torch.from_numpy(A))
    B = oracle.fill_uniform(k * n, np.float32, SEED + 3, 1)
    C = oracle.fill_uniform(m * n, np.float32, SEED + 3, 2)
    dB = torch.from_numpy(B).to(cuda)
    dC = torch.from_numpy(C).to(cuda)
    sbx.gemm_fused(sbx.F32, 0, 0, 0, m, n, k, 1.0, dA, lda, 0, dB, n, 0, 0.5, dC, n, 0)
    torch.cuda.synchronize()
    want = C.copy()
    oracle.gemm(0, 0, 0, m, n, k, 1.0, np.ascontiguousarray(A).ravel(), k, B, n, 0.5, want, n)
    oracle.relu(want)
    got = dC.cpu().numpy()
    assert oracle.rel_fro_err(got.reshape(m, n), want.reshape(m, n)) <= TOL[np.float32]
    assert not np.signbit(got).any()


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_fused_relu_quick_returns(cuda, dtype):
    """alpha == 0 and k == 0 reduce to C = relu(beta*C) (the scaling kernel);
    beta == 0 there writes zeros without reading C (NaN in C is not read)."""
    import torch
    import sushiblas_amd as sbx
    code = sbx.F32 if dtype == np.float32 else sbx.F64
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    m, n = 130, 70
    C = oracle.fill_uniform(m * n, dtype, SEED + 4, 2)
    for alpha, k, beta in ((0.0, 16, -1.5), (1.0, 0, 2.0), (0.0, 16, 0.0)):
        src = C.copy() if beta != 0 else np.full(m * n, np.nan, dtype)
        dC = torch.from_numpy(src).to(cuda)
        dA = torch.ones(max(1, m * k), dtype=tdt, device=cuda)
        dB = torch.ones(max(1, k * n), dtype=tdt, device=cuda)
        sbx.gemm_fused(code, 0, 0, 0, m, n, k, alpha, dA, max(1, k), 0, dB, n, 0, beta, dC, n, 0)
        torch.cuda.synchronize()
        want = (dtype(beta) * C) if beta != 0 else np.zeros(m * n, dtype)
        want = want.astype(dtype)
        oracle.relu(want)
        got = dC.cpu().numpy()
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), (alpha, k, beta)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_fused_relu_strided_batched(cuda, dtype):
    """Batch of 5 with padded batch strides; every batch rectified, gaps untouched."""
    import torch
    import sushiblas_amd as sbx
    code = sbx.F32 if dtype == np.float32 else sbx.F64
    m, n, k, batch = 96, 80, 72, 5
    sa, sb_, sc = m * k + 8, k * n + 4, m * n + 12
    A = oracle.fill_uniform(sa * batch, dtype, SEED + 5, 0)
    B = oracle.fill_uniform(sb_ * batch, dtype, SEED + 5, 1)
    C = oracle.fill_uniform(sc * batch, dtype, SEED + 5, 2)
    dA, dB, dC = (torch.from_numpy(x).to(cuda) for x in (A, B, C))
    sbx.gemm_fused(code, 0, 0, 0, m, n, k, 1.0, dA, k, sa, dB, n, sb_, 0.75, dC, n, sc, batch)
    torch.cuda.synchronize()
    got = dC.cpu().numpy()
    want = C.copy()
    oracle.gemm_strided_batched(0, 0, 0, m, n, k, 1.0, A, k, sa, B, n, sb_, 0.75, want, n, sc,
                                batch)
    for b in range(batch):
        blk = slice(b * sc, b * sc + m * n)
        w = want[blk].copy()
        oracle.relu(w)
        assert oracle.rel_fro_err(got[blk].reshape(m, n), w.reshape(m, n)) <= TOL[dtype]
        assert not np.signbit(got[blk]).any()
        gap = slice(b * sc + m * n, (b + 1) * sc)
        assert np.array_equal(got[gap], C[gap])


# -- stand-alone ReLU ----------------------------------------------------------

def _special(dtype):
    f = np.finfo(dtype)
    return np.array([-1.5, 0.0, -0.0, 2.25, np.nan, -np.nan, np.inf, -np.inf, f.tiny,
                     -f.tiny, f.smallest_subnormal, -f.smallest_subnormal, f.max, -f.max],
                    dtype=dtype)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("n,offset", [(0, 0), (1, 0), (3, 1), (5, 0), (14, 0), (1023, 3),
                                      (4099, 1), (1 << 20, 0), ((1 << 20) + 7, 2)])
def test_relu_bit_exact(cuda, dtype, n, offset):
    """sbx_relu vs oracle.relu, bit for bit, at ragged lengths and misaligned starts."""
    import torch
    import sushiblas_amd as sbx
    if n <= 64:
        x = np.resize(_special(dtype), n) * (1 + (np.arange(n) % 3)).astype(dtype)
    else:
        x = oracle.fill_uniform(n, dtype, SEED + 6, n % 97)
        x[:14] = _special(dtype)
    guard = np.full(offset + n + 5, 7.0, dtype) * -1
    guard[offset:offset + n] = x
    d = torch.from_numpy(guard).to(cuda)
    sbx.relu(d.data_ptr() + offset * d.element_size(), n,
             sbx.F32 if dtype == np.float32 else sbx.F64)
    torch.cuda.synchronize()
    got = d.cpu().numpy()
    want = x.copy()
    oracle.relu(want)
    assert np.array_equal(got[offset:offset + n].view(np.uint8), want.view(np.uint8))
    # the guards before and after are untouched
    assert np.all(got[:offset] == -7.0) and np.all(got[offset + n:] == -7.0)
