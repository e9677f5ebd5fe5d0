"""GPU tests of the allocation-free entry point sbx_gemm_ex_noalloc
(include/sbx.h): split-K partials in the fixed per-device scratch array
instead of the stream workspace.  It has no counterpart in the reference; it
must give sbx_gemm_ex's results (bit for bit where both plan the same split,
within the fp32/fp64 tolerance where the scratch bounds the split) and must
not allocate device memory.

Bar: normwise relative Frobenius error against the oracle accumulating in
double <= 1e-5 (fp32) / 1e-12 (fp64), as for every GEMM test.
"""
import numpy as np
import pytest

from gemm_cases import TOL, make_inputs, normwise, run_oracle

pytestmark = pytest.mark.gpu

SEED = 20261277
SCRATCH = 32 << 20  # SBX_NOALLOC_SCRATCH_BYTES


def _run_both(cuda, dtype, m, n, k, alpha, beta, seed, stream):
    """The same problem through sbx_gemm_ex and sbx_gemm_ex_noalloc (same
    input bits, separate outputs) plus the oracle; host results."""
    import torch
    import sushiblas_amd as sbx
    A, lda, B, ldb, C, ldc = make_inputs(dtype, 0, 0, 0, m, n, k, seed)
    code = sbx.F32 if dtype == np.float32 else sbx.F64
    dA = torch.from_numpy(A).to(cuda)
    dB = torch.from_numpy(B).to(cuda)
    c_ref = torch.from_numpy(C).to(cuda)
    c_na = torch.from_numpy(C).to(cuda)
    torch.cuda.synchronize()
    sbx.gemm_ex(code, 0, 0, 0, m, n, k, alpha, dA, lda, 0, dB, ldb, 0, beta, c_ref, ldc, 0,
                stream=stream)
    sbx.gemm_ex_noalloc(code, 0, 0, 0, m, n, k, alpha, dA, lda, 0, dB, ldb, 0, beta, c_na, ldc,
                        0, stream=stream)
    torch.cuda.synchronize()
    want = run_oracle(0, 0, 0, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
    return c_ref.cpu().numpy(), c_na.cpu().numpy(), want, ldc


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_noalloc_matches_gemm_ex_two_calls(cuda, dtype):
    """Two calls in a row on one stream, the second on a smaller problem:
    both split K, both fit the scratch, so the plans and the bits match
    sbx_gemm_ex's; both are within tolerance of the oracle."""
    import torch
    import sushiblas_amd as sbx
    code = sbx.F32 if dtype == np.float32 else sbx.F64
    stream = torch.cuda.Stream()
    shapes = ([(1536, 1536, 1024), (384, 320, 3000)] if dtype == np.float32
              else [(512, 384, 2048), (384, 320, 3000)])
    for i, (m, n, k) in enumerate(shapes):
        name = sbx.gemm_select(code, 0, 0, 0, m, n, k, k, n, n)
        print(f"noalloc case {np.dtype(dtype).name} {m}x{n}x{k} -> {name}", flush=True)
        assert "+splitk" in name, name
        ref, got, want, ldc = _run_both(cuda, dtype, m, n, k, 1.25, -0.5, SEED + i, stream)
        np.testing.assert_array_equal(got.view(np.uint8), ref.view(np.uint8))
        assert normwise(0, got, want, m, n, ldc) <= TOL[dtype]


def test_noalloc_bounds_the_split_to_the_scratch(cuda):
    """A problem whose preferred split needs more than the scratch (648
    tiles of 128x128: a round of 512 and a 136-tile tail cut 4-5 ways, 34-42
    MiB of partials) runs with a split that fits; the result stays within
    tolerance of the oracle and of sbx_gemm_ex.  A second, smaller call
    follows."""
    import torch
    import sushiblas_amd as sbx
    stream = torch.cuda.Stream()
    m, n, k = 3072, 3456, 2048
    name = sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n)
    parts = int(name.split("splitk")[1])
    tail = (m // 128) * (n // 128) % 512  # 24 x 27 tiles, two per CU
    assert name.startswith("mfma_f32_128x128x16_w2x2+") and tail * parts * 128 * 128 * 4 > SCRATCH, name
    for i, (mm, nn, kk) in enumerate([(m, n, k), (640, 640, 4096)]):
        ref, got, want, ldc = _run_both(cuda, np.float32, mm, nn, kk, 1.0, 0.5, SEED + 10 + i,
                                        stream)
        err = normwise(0, got, want, mm, nn, ldc)
        print(f"noalloc bounded case {mm}x{nn}x{kk} err={err:.3e}", flush=True)
        assert err <= TOL[np.float32]
        assert normwise(0, got, ref, mm, nn, ldc) <= TOL[np.float32]


def test_noalloc_allocates_nothing(cuda):
    """On a stream it has never seen, a split-K call of sbx_gemm_ex_noalloc
    takes no device memory (sbx_gemm_ex would allocate that stream's
    workspace, at least 32 MiB)."""
    import torch
    import sushiblas_amd as sbx
    m, n, k = 1536, 1536, 1024
    assert "+splitk" in sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n)
    A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, 0, 0, m, n, k, SEED + 20)
    dA = torch.from_numpy(A).to(cuda)
    dB = torch.from_numpy(B).to(cuda)
    dC = torch.from_numpy(C).to(cuda)
    # First use on this device resolves the scratch address; the first
    # launches on a new stream let the HIP runtime set that stream up (its own
    # lazy allocations, a few MiB).  Neither is measured: a 64^3 problem runs
    # unsplit, so it touches no scratch either way.
    fresh = torch.cuda.Stream()
    for _ in range(2):
        sbx.gemm_ex_noalloc(sbx.F32, 0, 0, 0, 64, 64, 64, 1.0, dA, lda, 0, dB, ldb, 0, 0.0, dC,
                            ldc, 0, stream=fresh)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        sbx.gemm_ex_noalloc(sbx.F32, 0, 0, 0, m, n, k, 1.0, dA, lda, 0, dB, ldb, 0, 0.0, dC,
                            ldc, 0, stream=fresh)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free0 - free1 < (1 << 20), (free0, free1)


def test_noalloc_split_batch_two_calls(cuda):
    """Strided batches that cut K (their grids fill less than one round):
    every entry's partials sit in the scratch after the previous entry's.
    Two calls in a row on one stream, the second with a smaller batch and a
    different tile, both fit the scratch, so the bits match sbx_gemm_ex's;
    each entry within tolerance of the oracle."""
    import torch
    import oracle
    import sushiblas_amd as sbx
    stream = torch.cuda.Stream()
    for i, (batch, m, n, k) in enumerate([(8, 128, 128, 4096), (3, 300, 200, 5000)]):
        name = sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n, batch=batch)
        print(f"noalloc split batch {batch} x {m}x{n}x{k} -> {name}", flush=True)
        assert "+splitk" in name, name
        str_a, str_b, str_c = m * k, k * n, m * n
        A = oracle.fill_uniform(batch * str_a, np.float32, SEED + 20 + i, 0)
        B = oracle.fill_uniform(batch * str_b, np.float32, SEED + 20 + i, 1)
        C = oracle.fill_uniform(batch * str_c, np.float32, SEED + 20 + i, 2)
        dA, dB = torch.from_numpy(A).to(cuda), torch.from_numpy(B).to(cuda)
        c_ref, c_na = torch.from_numpy(C).to(cuda), torch.from_numpy(C).to(cuda)
        torch.cuda.synchronize()
        sbx.gemm_ex(sbx.F32, 0, 0, 0, m, n, k, 0.5, dA, k, str_a, dB, n, str_b, 1.5, c_ref, n,
                    str_c, batch, stream=stream)
        sbx.gemm_ex_noalloc(sbx.F32, 0, 0, 0, m, n, k, 0.5, dA, k, str_a, dB, n, str_b, 1.5, c_na,
                            n, str_c, batch, stream=stream)
        torch.cuda.synchronize()
        ref, got = c_ref.cpu().numpy(), c_na.cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint8), ref.view(np.uint8))
        want = C.copy()
        oracle.gemm_strided_batched(0, 0, 0, m, n, k, 0.5, A, k, str_a, B, n, str_b, 1.5, want, n,
                                    str_c, batch, 1)
        for b in range(batch):
            w = want[b * str_c:(b + 1) * str_c].reshape(m, n)
            g = got[b * str_c:(b + 1) * str_c].reshape(m, n)
            assert oracle.rel_fro_err(g, w) <= TOL[np.float32], b


def test_noalloc_concurrent_host_threads_one_stream(cuda):
    """Six host threads share one stream and call sbx_gemm_ex_noalloc on two
    split shapes in alternation.  Each call's partial kernel and reduction
    must be enqueued back to back (the per-GPU scratch lock): were another
    thread's partial kernel to land between them, the reduction would sum
    that call's partials and return wrong values.  Every result is checked
    against the oracle."""
    import threading
    import torch
    import sushiblas_amd as sbx
    shapes = [(1536, 1536, 1024), (384, 320, 3000)]
    data = []
    for i, (m, n, k) in enumerate(shapes):
        name = sbx.gemm_select(sbx.F32, 0, 0, 0, m, n, k, k, n, n)
        print(f"noalloc threads case {m}x{n}x{k} -> {name}", flush=True)
        assert "+splitk" in name, name
        A, lda, B, ldb, C, ldc = make_inputs(np.float32, 0, 0, 0, m, n, k, SEED + 30 + i)
        want = run_oracle(0, 0, 0, m, n, k, 1.0, A, lda, B, ldb, 0.0, C, ldc)
        data.append((m, n, k, torch.from_numpy(A).to(cuda), lda, torch.from_numpy(B).to(cuda),
                     ldb, ldc, want))
    nthreads = 6
    outs = [[torch.full((d[0] * d[1],), float("nan"), device=cuda) for _ in range(nthreads)]
            for d in data]
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    errors = []

    def worker(t):
        try:
            for rep in range(4):
                for j in ((t + rep) % 2, (t + rep + 1) % 2):
                    m, n, k, dA, lda, dB, ldb, ldc, _ = data[j]
                    sbx.gemm_ex_noalloc(sbx.F32, 0, 0, 0, m, n, k, 1.0, dA, lda, 0, dB, ldb, 0,
                                        0.0, outs[j][t], ldc, 0, stream=stream)
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(nthreads)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    stream.synchronize()
    assert not errors, errors
    for (m, n, k, _, _, _, _, ldc, want), group in zip(data, outs):
        for t, o in enumerate(group):
            err = normwise(0, o.cpu().numpy(), want, m, n, ldc)
            assert err <= TOL[np.float32], (m, n, k, t, err)
