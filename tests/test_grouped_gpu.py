"""GPU parity of the grouped launch (sbx_gemm_grouped): `count` problems of one
shape whose operands sit anywhere in device memory, named by a device table
of (A, B, C) pointers, in one launch.  Every problem is checked against the
oracle (normwise <= 1e-5 fp32 / 1e-12 fp64), with the buffers around each C
untouched.  Covers both layouts, all transposes, the ReLU epilogue, the
alpha == 0 quick return and pointers off 16-byte alignment."""
import ctypes

import numpy as np
import pytest

import oracle
from gemm_cases import TOL, c_window, make_inputs, run_oracle

pytestmark = pytest.mark.gpu

SEED = 20261209


def _grouped(cuda, dtype, layout, ta, tb, m, n, k, alpha, beta, count, epilogue=0, misalign=False,
             pad=(0, 0, 0)):
    import torch
    import sushiblas_amd as sbx
    L = sbx.lib()
    vp = ctypes.c_void_p
    L.sbx_gemm_grouped.restype = ctypes.c_int
    L.sbx_gemm_grouped.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, vp,
                                   ctypes.c_int64, ctypes.c_int64, vp, ctypes.c_int64, vp,
                                   ctypes.c_int64, ctypes.c_int, ctypes.c_int]
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    es = 4 if dtype == np.float32 else 8
    off = 1 if misalign else 0
    problems, bufs, ptrs = [], [], []
    for i in range(count):
        A, lda, B, ldb, C, ldc = make_inputs(dtype, layout, ta, tb, m, n, k, SEED + i, pad=pad)
        # each operand in its own allocation, with guard elements before and after
        dev = []
        for x in (A, B, C):
            t = torch.full((x.size + 2 * off + 8,), -3.0, dtype=tdt, device=cuda)
            t[off:off + x.size] = torch.from_numpy(x).to(cuda)
            dev.append(t)
        bufs.append(dev)
        ptrs += [d.data_ptr() + off * es for d in dev]
        problems.append((A, lda, B, ldb, C, ldc))
    table = torch.tensor(ptrs, dtype=torch.int64, device=cuda)
    real = ctypes.c_float if dtype == np.float32 else ctypes.c_double
    a, b = real(alpha), real(beta)
    lda, ldb, ldc = problems[0][1], problems[0][3], problems[0][5]
    stream = torch.cuda.current_stream().cuda_stream
    st = L.sbx_gemm_grouped(stream, sbx.F32 if dtype == np.float32 else sbx.F64, layout, ta, tb,
                            m, n, k, ctypes.byref(a), lda, ldb, ctypes.byref(b), ldc,
                            table.data_ptr(), count, 0 if misalign else 1, epilogue)
    assert st == 0, st
    torch.cuda.synchronize()
    print(f"grouped {np.dtype(dtype).name} layout={layout} t{ta}{tb} {m}x{n}x{k} x{count} "
          f"alpha={alpha} beta={beta} epi={epilogue} misalign={misalign}", flush=True)
    for (A, lda, B, ldb, C, ldc), dev in zip(problems, bufs):
        want = run_oracle(layout, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
        got_full = dev[2].cpu().numpy()
        got = got_full[off:off + C.size]
        gw, ww = c_window(layout, got, m, n, ldc), c_window(layout, want, m, n, ldc)
        if epilogue:
            oracle.relu(ww)
            assert not np.signbit(gw).any()
        if np.linalg.norm(ww) > 0:
            assert oracle.rel_fro_err(gw, ww) <= TOL[dtype]
        else:
            assert np.array_equal(gw, ww)
        # guards around C untouched, and C's elements outside the m x n window
        # (the ld padding) keep their input bits
        assert np.all(got_full[:off] == -3.0) and np.all(got_full[off + C.size:] == -3.0)
        outside = np.ones(C.size, bool)
        idx = np.arange(C.size)
        if layout == 0:
            outside[(idx // ldc < m) & (idx % ldc < n)] = False
        else:
            outside[(idx // ldc < n) & (idx % ldc < m)] = False
        assert np.array_equal(got[outside].view(np.uint8), C[outside].view(np.uint8))
        # A and B untouched too
        for x, d in ((A, dev[0]), (B, dev[1])):
            assert np.array_equal(d.cpu().numpy()[off:off + x.size], x)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_grouped_matches_oracle(cuda, dtype, layout, ta, tb):
    _grouped(cuda, dtype, layout, ta, tb, 96, 80, 72, 1.25, -0.5, 7)


def test_grouped_shapes_epilogue_quick_and_misaligned(cuda):
    _grouped(cuda, np.float32, 0, 0, 0, 256, 512, 256, 1.0, 0.0, 24, epilogue=1)  # framework sim
    _grouped(cuda, np.float32, 0, 0, 0, 8, 8, 8, 1.0, 1.0, 300)                   # many tiny
    _grouped(cuda, np.float32, 0, 1, 0, 300, 257, 129, 0.75, 0.25, 3, misalign=True)
    _grouped(cuda, np.float64, 1, 0, 1, 65, 33, 17, 0.0, 2.0, 4)                  # alpha == 0
    _grouped(cuda, np.float32, 0, 0, 0, 1000, 64, 512, 1.0, 0.0, 2)              # tall tiles


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("layout", [0, 1])
def test_grouped_split_k(cuda, dtype, layout):
    """Grouped launches whose grid fills less than one round split K: entry
    z's partials follow entry z-1's in the workspace and the reduction finds
    each entry's C through the table (swapped operands in column-major).
    Run plain, with C off 16-byte alignment, and with the ReLU epilogue, with
    ld padding around each window."""
    import sushiblas_amd as sbx
    code = sbx.F32 if dtype == np.float32 else sbx.F64
    for m, n, k, count in ((128, 128, 4096, 8), (300, 200, 5000, 3)):
        lda, ldb, ldc = (k, n, n) if layout == 0 else (m, k, m)
        name = sbx.gemm_select(code, layout, 0, 0, m, n, k, lda, ldb, ldc, batch=count)
        print(f"grouped split case {np.dtype(dtype).name} layout={layout} {m}x{n}x{k} "
              f"x{count} -> {name}", flush=True)
        assert "+splitk" in name, name
        _grouped(cuda, dtype, layout, 0, 0, m, n, k, 1.0, 0.5, count, pad=(3, 5, 7))
        _grouped(cuda, dtype, layout, 1, 1, m, n, k, -0.75, 0.0, count, misalign=True,
                 pad=(1, 2, 3))
        _grouped(cuda, dtype, layout, 0, 1, m, n, k, 1.5, -1.0, count, epilogue=1, pad=(0, 0, 4))
