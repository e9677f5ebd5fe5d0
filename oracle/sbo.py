"""ctypes front end of the CPU oracle (test infrastructure only).

Every routine works on numpy buffers and mirrors the C entry point of the
same name in ``oracle/sbo.c``.  Matrices are passed as flat (or any
C-contiguous) numpy arrays plus BLAS leading dimensions, exactly as the
reference hands raw pointers + ld to oneMKL (src/ops/blas/level3/gemm.cpp:63).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
lib_path = os.path.join(_HERE, "lib", "libsbo.so")
_lib = None

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


def build(force: bool = False) -> None:
    """Compile oracle/sbo.c with the Makefile beside it."""
    args = ["make", "-C", _HERE] + (["-B"] if force else [])
    subprocess.run(args, check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(lib_path):
        build()
    lib = ctypes.CDLL(lib_path)
    for name, real in (("sbo_sgemm_strided_batched", ctypes.c_float),
                       ("sbo_dgemm_strided_batched", ctypes.c_double)):
        f = getattr(lib, name)
        f.restype = ctypes.c_int
        f.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _i64, _i64, _i64, real,
                      _vp, _i64, _i64, _vp, _i64, _i64, real, _vp, _i64, _i64, _i64,
                      ctypes.c_int]
    lib.sbo_gemm_naive_ld.restype = ctypes.c_int
    lib.sbo_gemm_naive_ld.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      _i64, _i64, _i64, ctypes.c_double, _vp, _i64, _vp, _i64,
                                      ctypes.c_double, _vp, _i64]
    for name in ("sbo_rel_fro_err_f32", "sbo_rel_fro_err_f64"):
        f = getattr(lib, name)
        f.restype = ctypes.c_double
        f.argtypes = [_i64, _i64, _vp, _i64, _vp, _i64]
    lib.sbo_philox4x32_10.restype = None
    lib.sbo_philox4x32_10.argtypes = [_vp, _vp, _vp]
    for name in ("sbo_fill_uniform_f32", "sbo_fill_uniform_f64"):
        f = getattr(lib, name)
        f.restype = None
        f.argtypes = [_vp, _i64, ctypes.c_uint64, ctypes.c_uint32]
    for name in ("sbo_fill_normal_f32", "sbo_fill_normal_f64"):
        f = getattr(lib, name)
        f.restype = None
        f.argtypes = [_vp, _i64, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_double]
    for name in ("sbo_relu_f32", "sbo_relu_f64"):
        f = getattr(lib, name)
        f.restype = None
        f.argtypes = [_vp, _i64]
    for name, real in (("sbo_sgemv", ctypes.c_float), ("sbo_dgemv", ctypes.c_double)):
        f = getattr(lib, name)
        f.restype = ctypes.c_int
        f.argtypes = [ctypes.c_int, ctypes.c_int, _i64, _i64, real, _vp, _i64, _vp, _i64, real,
                      _vp, _i64]
    for name, real in (("sbo_ssyrk_strided_batched", ctypes.c_float),
                       ("sbo_dsyrk_strided_batched", ctypes.c_double)):
        f = getattr(lib, name)
        f.restype = ctypes.c_int
        f.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _i64, _i64, real, _vp, _i64, _i64,
                      real, _vp, _i64, _i64, _i64]
    lib.sbo_num_threads.restype = ctypes.c_int
    lib.sbo_num_threads.argtypes = []
    _lib = lib
    return lib


def _ptr(a: np.ndarray) -> int:
    if not a.flags.c_contiguous:
        raise ValueError("oracle buffers must be C-contiguous numpy arrays")
    return a.ctypes.data


def gemm_strided_batched(layout, transA, transB, m, n, k, alpha, A, lda, str_a, B, ldb, str_b,
                         beta, C, ldc, str_c, batch, acc_mode=1):
    """C <- alpha*op(A)*op(B) + beta*C for `batch` strided problems (in place on C)."""
    lib = _load()
    if not (A.dtype == B.dtype == C.dtype):
        raise TypeError("dtype mismatch")
    if A.dtype == np.float32:
        f = lib.sbo_sgemm_strided_batched
    elif A.dtype == np.float64:
        f = lib.sbo_dgemm_strided_batched
    else:
        raise TypeError(f"unsupported dtype {A.dtype}")
    rc = f(int(layout), int(bool(transA)), int(bool(transB)), m, n, k, float(alpha), _ptr(A),
           lda, str_a, _ptr(B), ldb, str_b, float(beta), _ptr(C), ldc, str_c, batch,
           int(acc_mode))
    if rc != 0:
        raise ValueError(f"oracle gemm rejected its arguments (status {rc})")
    return C


def gemm(layout, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, acc_mode=1):
    return gemm_strided_batched(layout, transA, transB, m, n, k, alpha, A, lda, 0, B, ldb, 0,
                                beta, C, ldc, 0, 1, acc_mode)


def gemm_naive_ld(layout, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc):
    lib = _load()
    elem = A.dtype.itemsize
    rc = lib.sbo_gemm_naive_ld(elem, int(layout), int(bool(transA)), int(bool(transB)), m, n, k,
                               float(alpha), _ptr(A), lda, _ptr(B), ldb, float(beta), _ptr(C),
                               ldc)
    if rc != 0:
        raise ValueError(f"naive gemm rejected its arguments (status {rc})")
    return C


def rel_fro_err(X: np.ndarray, Y: np.ndarray) -> float:
    """||X - Y||_F / ||Y||_F for two 2-D C-contiguous arrays of one dtype."""
    lib = _load()
    X = np.ascontiguousarray(X)
    Y = np.ascontiguousarray(Y)
    if X.shape != Y.shape or X.dtype != Y.dtype:
        raise ValueError("shape/dtype mismatch")
    rows, cols = (X.shape[0], int(np.prod(X.shape[1:]))) if X.ndim >= 2 else (1, X.size)
    f = lib.sbo_rel_fro_err_f32 if X.dtype == np.float32 else lib.sbo_rel_fro_err_f64
    return float(f(rows, cols, _ptr(X), cols, _ptr(Y), cols))


def philox4x32_10(ctr, key):
    lib = _load()
    c = np.asarray(ctr, dtype=np.uint32)
    k = np.asarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib.sbo_philox4x32_10(_ptr(c), _ptr(k), _ptr(out))
    return out


def fill_uniform(n: int, dtype, seed: int, stream: int) -> np.ndarray:
    lib = _load()
    out = np.empty(int(n), dtype=dtype)
    f = lib.sbo_fill_uniform_f32 if out.dtype == np.float32 else lib.sbo_fill_uniform_f64
    f(_ptr(out), out.size, seed, stream)
    return out


def fill_normal(n: int, dtype, seed: int, stream: int, scale: float = 1.0) -> np.ndarray:
    lib = _load()
    out = np.empty(int(n), dtype=dtype)
    f = lib.sbo_fill_normal_f32 if out.dtype == np.float32 else lib.sbo_fill_normal_f64
    f(_ptr(out), out.size, seed, stream, float(scale))
    return out


def relu(x: np.ndarray) -> np.ndarray:
    """In-place ReLU as the reference defines it: x > 0 ? x : 0."""
    lib = _load()
    f = lib.sbo_relu_f32 if x.dtype == np.float32 else lib.sbo_relu_f64
    f(_ptr(x), x.size)
    return x


def gemv(layout, trans, m, n, alpha, A, lda, x, incx, beta, y, incy):
    """y <- alpha*op(A)*x + beta*y in place (netlib quick returns)."""
    lib = _load()
    if not (A.dtype == x.dtype == y.dtype):
        raise TypeError("dtype mismatch")
    f = lib.sbo_sgemv if A.dtype == np.float32 else lib.sbo_dgemv
    rc = f(int(layout), int(bool(trans)), m, n, float(alpha), _ptr(A), lda, _ptr(x), incx,
           float(beta), _ptr(y), incy)
    if rc != 0:
        raise ValueError(f"oracle gemv rejected its arguments (status {rc})")
    return y


def syrk_strided_batched(layout, upper, trans, n, k, alpha, A, lda, str_a, beta, C, ldc, str_c,
                         batch):
    """One triangle of C <- alpha*op(A)*op(A)^T + beta*C, in place."""
    lib = _load()
    if A.dtype != C.dtype:
        raise TypeError("dtype mismatch")
    f = (lib.sbo_ssyrk_strided_batched if A.dtype == np.float32
         else lib.sbo_dsyrk_strided_batched)
    rc = f(int(layout), int(bool(upper)), int(bool(trans)), n, k, float(alpha), _ptr(A), lda,
           str_a, float(beta), _ptr(C), ldc, str_c, batch)
    if rc != 0:
        raise ValueError(f"oracle syrk rejected its arguments (status {rc})")
    return C


def syrk(layout, upper, trans, n, k, alpha, A, lda, beta, C, ldc):
    return syrk_strided_batched(layout, upper, trans, n, k, alpha, A, lda, 0, beta, C, ldc, 0, 1)


def num_threads() -> int:
    return int(_load().sbo_num_threads())
