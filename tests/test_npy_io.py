"""The product's .npy IO (IO::save_npy / load_npy, src/io.cpp:136-235 of the
reference) against NumPy, which defines the format.

* host: the preamble IO::npy_header builds is byte-identical to the one
  np.save writes, for every dtype the engine has and several shapes / orders;
* GPU: the golden GEMM vectors (tests/golden/gemm_golden.npz) are written as
  .npy files by NumPy, loaded through IO::load_npy, multiplied by
  Level3::gemm, and the result is written back with IO::save_npy and read by
  NumPy (np.load, no pickle) -- a round trip through the product's own IO.
"""
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "sushiblas_amd", "lib", "sushiblas_engine_tests")
GOLDEN = os.path.join(ROOT, "tests", "golden", "gemm_golden.npz")

# Core::DataType values (HALF, FLOAT32, FLOAT64, COMPLEX32, COMPLEX64)
DTYPES = {np.float16: 0, np.float32: 1, np.float64: 2, np.complex64: 3, np.complex128: 4}


def _run_case(case, env_dir, timeout):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built: run __graft_entry__.build()")
    env = dict(os.environ, SBX_NPY_DIR=str(env_dir))
    res = subprocess.run([BIN, case], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                         timeout=timeout, env=env)
    print(res.stdout)
    assert res.returncode == 0, res.stdout[-2000:]
    assert re.search(rf"^\[  OK  \] {case}$", res.stdout, flags=re.M), res.stdout[-2000:]


def test_npy_headers_match_numpy(tmp_path):
    lines = []
    shapes = [(2, 3), (5,), (1, 1), (7, 1, 3), (100000,), (3, 4, 5, 6), (65, 257)]
    i = 0
    for dt, code in DTYPES.items():
        for shape in shapes:
            arr = np.zeros(shape, dt)
            name = f"h{i}.npy"
            np.save(tmp_path / name, arr)
            lines.append(f"{name} {code} 0 {len(shape)} " + " ".join(map(str, shape)))
            i += 1
        # column-major: numpy writes fortran_order True for F-contiguous arrays
        for shape in [(4, 6), (3, 5, 2)]:
            arr = np.asfortranarray(np.zeros(shape, dt))
            name = f"h{i}.npy"
            np.save(tmp_path / name, arr)
            lines.append(f"{name} {code} 1 {len(shape)} " + " ".join(map(str, shape)))
            i += 1
    (tmp_path / "headers.txt").write_text("\n".join(lines) + "\n")
    _run_case("NpyHeadersMatchNumpy", tmp_path, 120)


def _stored(flat, layout, rows, cols):
    """A flat BLAS buffer (minimal ld) as the rows x cols array it stores."""
    if layout == 0:
        return flat.reshape(rows, cols)
    return flat.reshape(cols, rows).T  # F-ordered view: np.save writes fortran_order True


@pytest.mark.gpu
def test_golden_gemm_through_npy(cuda, tmp_path):
    g = np.load(GOLDEN)
    ids = sorted({k.split("_")[0] for k in g.files})
    lines = []
    for cid in ids:
        layout, ta, tb, m, n, k = (int(v) for v in g[f"{cid}_meta"][:6])
        alpha, beta = (float(v) for v in g[f"{cid}_scal"])
        A, B, C, out = (g[f"{cid}_{x}"] for x in ("A", "B", "C", "out"))
        sa = (k, m) if ta else (m, k)
        sb = (n, k) if tb else (k, n)
        np.save(tmp_path / f"{cid}_A.npy", _stored(A, layout, *sa))
        np.save(tmp_path / f"{cid}_B.npy", _stored(B, layout, *sb))
        np.save(tmp_path / f"{cid}_C.npy", _stored(C, layout, m, n))
        np.save(tmp_path / f"{cid}_out.npy", _stored(out, layout, m, n))
        lines.append(f"{cid} {DTYPES[A.dtype.type]} {layout} {ta} {tb} {m} {n} {k} "
                     f"{alpha!r} {beta!r}")
    (tmp_path / "cases.txt").write_text("\n".join(lines) + "\n")
    _run_case("GoldenGemmThroughNpy", tmp_path, 300)
    # NumPy reads what save_npy wrote: same shape, order and values
    for cid in ids:
        layout = int(g[f"{cid}_meta"][0])
        m, n = (int(v) for v in g[f"{cid}_meta"][3:5])
        got = np.load(tmp_path / f"{cid}_got.npy")
        want = _stored(g[f"{cid}_out"], layout, m, n)
        assert got.shape == (m, n) and got.dtype == want.dtype
        assert got.flags.f_contiguous if (layout == 1 and min(m, n) > 1) else got.flags.c_contiguous
        tol = 1e-5 if got.dtype == np.float32 else 1e-12
        err = np.linalg.norm((got - want).astype(np.float64)) / np.linalg.norm(want.astype(np.float64))
        assert err <= tol, (cid, err)
