"""Device Philox generators (sbx_fill_*) against the host restatement in the
oracle: uniform streams are exact in their type, so they must match bit for
bit; normals go through log/sqrt/sincos and must match to rounding."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("n", [1, 3, 4, 5, 1023, 100003])
def test_uniform_bit_exact(cuda, dtype, n):
    import torch
    import sushiblas_amd as sbx
    t = torch.empty(n, dtype=torch.float32 if dtype == np.float32 else torch.float64,
                    device=cuda)
    sbx.fill_uniform(t, 20261203, 1)
    torch.cuda.synchronize()
    got = t.cpu().numpy()
    want = oracle.fill_uniform(n, dtype, 20261203, 1)
    np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_normal_matches_host(cuda, dtype):
    import torch
    import sushiblas_amd as sbx
    n = 200001
    t = torch.empty(n, dtype=torch.float32 if dtype == np.float32 else torch.float64,
                    device=cuda)
    sbx.fill_normal(t, 7, 2, 0.5)
    torch.cuda.synchronize()
    got = t.cpu().numpy().astype(np.float64)
    want = oracle.fill_normal(n, dtype, 7, 2, 0.5).astype(np.float64)
    tol = 4e-7 if dtype == np.float32 else 1e-14
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-3)) < tol
    assert abs(got.mean()) < 0.01 and abs(got.std() - 0.5) < 0.01
