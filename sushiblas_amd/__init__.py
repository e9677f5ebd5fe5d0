"""sushiblas_amd -- MI355X (gfx950) GEMM hot path of SushiBLAS.

The product is the HIP library ``lib/libsbx.so`` behind the C ABI declared in
``include/sbx.h``, plus the C++ Engine/Tensor/Storage layer in ``cpp/`` that
mirrors the reference's API (``Level3::gemm``, src/ops/blas/level3/gemm.cpp:82).
This module is a thin ctypes binding of the C ABI for Python callers (tests,
benchmarks): device buffers are passed as raw pointers (ints) or torch tensors
(their ``data_ptr()``), and the stream defaults to torch's current stream.

There is no CPU fallback: if the HIP library is missing, every call raises.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libsbx.so")
# The probe build of the same sources (csrc/sbx_probe.h): per-workgroup clock
# stamps for measurements; use_probe_library() selects it before first use.
PROBE_LIB_PATH = os.path.join(_HERE, "lib", "libsbx_probe.so")

F32, F64 = 0, 1
ALGO_AUTO, ALGO_GENERIC, ALGO_MFMA, ALGO_MFMA_TILE, ALGO_MFMA_SMALL = 0, 1, 2, 3, 4
EPILOGUE_NONE, EPILOGUE_RELU = 0, 1
STATUS = {0: "SBX_OK", 1: "SBX_INVALID_ARGUMENT", 2: "SBX_UNSUPPORTED", 3: "SBX_HIP_ERROR"}

_lib = None


class SbxError(RuntimeError):
    """Raised when an sbx_* entry point returns a non-zero status."""

    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where} failed: {STATUS.get(status, status)} ({_status_text(status)})")


def build(force: bool = True, jobs: int = 8) -> None:
    """Compile the HIP library in-tree (hipcc --offload-arch=gfx950)."""
    args = ["make", "-C", _HERE, f"-j{jobs}"] + (["-B"] if force else [])
    res = subprocess.run(args, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError("building libsbx.so failed:\n" + res.stdout[-4000:])


def use_probe_library() -> None:
    """Load lib/libsbx_probe.so instead of lib/libsbx.so: the same kernels
    plus per-workgroup clock stamps (probe_set, probe_dispatches).  Must be
    called before the first lib() call."""
    global LIB_PATH
    if _lib is not None and LIB_PATH != PROBE_LIB_PATH:
        raise RuntimeError("use_probe_library() after the product library was loaded")
    LIB_PATH = PROBE_LIB_PATH


def lib() -> ctypes.CDLL:
    """Load libsbx.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() "
                           "(or `make -C sushiblas_amd`) first")
    # torch ships its own HIP runtime.  Loading it first makes libsbx.so bind to
    # that same runtime (one soname, one instance); loading libsbx.so first
    # would bring up the system runtime beside torch's, and launches from the
    # second one to initialise fail with "invalid device function".
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = ctypes.CDLL(LIB_PATH)
    i64, vp, i32 = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
    L.sbx_gemm_ex.restype = i32
    L.sbx_gemm_ex.argtypes = [vp, i32, i32, i32, i32, i64, i64, i64, vp, vp, i64, i64, vp, i64,
                              i64, vp, vp, i64, i64, i64, i32]
    for name, real in (("sbx_sgemm", ctypes.c_float), ("sbx_dgemm", ctypes.c_double)):
        f = getattr(L, name)
        f.restype = i32
        f.argtypes = [vp, i32, i32, i32, i64, i64, i64, real, vp, i64, vp, i64, real, vp, i64]
    for name, real in (("sbx_sgemm_strided_batched", ctypes.c_float),
                       ("sbx_dgemm_strided_batched", ctypes.c_double)):
        f = getattr(L, name)
        f.restype = i32
        f.argtypes = [vp, i32, i32, i32, i64, i64, i64, real, vp, i64, i64, vp, i64, i64, real,
                      vp, i64, i64, i64]
    L.sbx_gemm_ex_noalloc.restype = i32
    L.sbx_gemm_ex_noalloc.argtypes = L.sbx_gemm_ex.argtypes
    L.sbx_gemm_fused.restype = i32
    L.sbx_gemm_fused.argtypes = [vp, i32, i32, i32, i32, i64, i64, i64, vp, vp, i64, i64, vp,
                                 i64, i64, vp, vp, i64, i64, i64, i32]
    L.sbx_relu.restype = i32
    L.sbx_relu.argtypes = [vp, i32, vp, i64]
    for name, real in (("sbx_sgemv", ctypes.c_float), ("sbx_dgemv", ctypes.c_double)):
        f = getattr(L, name)
        f.restype = i32
        f.argtypes = [vp, i32, i32, i64, i64, real, vp, i64, vp, i64, real, vp, i64]
    for name, real in (("sbx_ssyrk_strided_batched", ctypes.c_float),
                       ("sbx_dsyrk_strided_batched", ctypes.c_double)):
        f = getattr(L, name)
        f.restype = i32
        f.argtypes = [vp, i32, i32, i32, i64, i64, real, vp, i64, i64, real, vp, i64, i64, i64]
    for name, real in (("sbx_ssyrk", ctypes.c_float), ("sbx_dsyrk", ctypes.c_double)):
        f = getattr(L, name)
        f.restype = i32
        f.argtypes = [vp, i32, i32, i32, i64, i64, real, vp, i64, real, vp, i64]
    L.sbx_gemm_select.restype = i32
    L.sbx_gemm_select.argtypes = [i32, i32, i32, i32, i64, i64, i64, i64, i64, i64,
                                  ctypes.c_char_p, ctypes.c_size_t]
    L.sbx_gemm_select_batched.restype = i32
    L.sbx_gemm_select_batched.argtypes = [i32, i32, i32, i32, i64, i64, i64, i64, i64, i64, i64,
                                          ctypes.c_char_p, ctypes.c_size_t]
    L.sbx_gemm_plans.restype = i32
    L.sbx_gemm_plans.argtypes = [i32, i32, i32, i32, i64, i64, i64, i64, i64, i64, i64,
                                 ctypes.c_char_p, ctypes.c_size_t]
    L.sbx_gemm_ex_plan.restype = i32
    L.sbx_gemm_ex_plan.argtypes = L.sbx_gemm_ex.argtypes[:-1] + [ctypes.c_char_p]
    L.sbx_syrk_select.restype = i32
    L.sbx_syrk_select.argtypes = [i32, i32, i32, i32, i64, i64, i64, i64, ctypes.c_char_p,
                                  ctypes.c_size_t]
    L.sbx_syrk_plans.restype = i32
    L.sbx_syrk_plans.argtypes = L.sbx_syrk_select.argtypes
    L.sbx_syrk_ex_plan.restype = i32
    L.sbx_syrk_ex_plan.argtypes = [vp, i32, i32, i32, i32, i64, i64, vp, vp, i64, i64, vp, vp,
                                   i64, i64, i64, ctypes.c_char_p]
    L.sbx_status_string.restype = ctypes.c_char_p
    L.sbx_status_string.argtypes = [i32]
    L.sbx_fill_uniform.restype = i32
    L.sbx_fill_uniform.argtypes = [vp, i32, vp, i64, ctypes.c_uint64, ctypes.c_uint32]
    L.sbx_fill_normal.restype = i32
    L.sbx_fill_normal.argtypes = [vp, i32, vp, i64, ctypes.c_uint64, ctypes.c_uint32,
                                  ctypes.c_double]
    L.sbx_version.restype = ctypes.c_char_p
    L.sbx_version.argtypes = []
    if LIB_PATH == PROBE_LIB_PATH:
        L.sbx_probe_set.restype = i32
        L.sbx_probe_set.argtypes = [vp, i64, i64]
        L.sbx_probe_dispatches.restype = i64
        L.sbx_probe_dispatches.argtypes = []
        L.sbx_probe_wall_clock_khz.restype = i64
        L.sbx_probe_wall_clock_khz.argtypes = []
    _lib = L
    return L


PROBE_POINTS = 4  # SBX_PROBE_POINTS


def probe_set(buf, blocks: int, ring: int) -> None:
    """Start recording stamps into `buf` (a uint64/int64 device tensor of
    ring * blocks * PROBE_POINTS * 2 elements; None stops).  Probe build only."""
    _check(lib().sbx_probe_set(_ptr(buf), blocks if buf is not None else 0,
                               ring if buf is not None else 0), "sbx_probe_set")


def probe_dispatches() -> int:
    return int(lib().sbx_probe_dispatches())


def probe_wall_clock_khz() -> int:
    return int(lib().sbx_probe_wall_clock_khz())


def _status_text(status: int) -> str:
    try:
        return lib().sbx_status_string(status).decode()
    except Exception:  # pragma: no cover - only when the library itself is absent
        return "?"


def _ptr(x) -> int:
    if x is None:
        return 0
    if isinstance(x, int):
        return x
    return int(x.data_ptr())


_raw_stream = None  # torch's current-stream query without building a Stream object


def _current_stream() -> int:
    """torch's current stream on the current device, as a raw handle.
    torch.cuda.current_stream() builds a Python Stream object on every call
    (about 2.5 us of host time, a third of a 512^3 GEMM call); the raw query
    that torch's own generated code uses returns the same handle without it."""
    global _raw_stream
    import torch
    if _raw_stream is None:
        C = torch._C
        if hasattr(C, "_cuda_getCurrentRawStream") and hasattr(C, "_cuda_getDevice"):
            _raw_stream = lambda: C._cuda_getCurrentRawStream(C._cuda_getDevice())
        else:  # pragma: no cover - older torch
            _raw_stream = lambda: torch.cuda.current_stream().cuda_stream
    return int(_raw_stream())


def _stream(stream) -> int:
    if stream is None:
        return _current_stream()
    if isinstance(stream, int):
        return stream
    return int(stream.cuda_stream)


def _check(status: int, where: str) -> None:
    if status != 0:
        raise SbxError(status, where)


def gemm_ex(dtype, layout, transA, transB, m, n, k, alpha, A, lda, str_a, B, ldb, str_b, beta,
            C, ldc, str_c, batch=1, algo=ALGO_AUTO, stream=None) -> None:
    """sbx_gemm_ex: dtype-generic, optionally batched, with an algorithm override."""
    real = ctypes.c_float if dtype == F32 else ctypes.c_double
    a = real(alpha)
    b = real(beta)
    st = lib().sbx_gemm_ex(_stream(stream), dtype, int(layout), int(transA), int(transB), m, n,
                           k, ctypes.byref(a), _ptr(A), lda, str_a, _ptr(B), ldb, str_b,
                           ctypes.byref(b), _ptr(C), ldc, str_c, batch, algo)
    _check(st, "sbx_gemm_ex")


def gemm_ex_noalloc(dtype, layout, transA, transB, m, n, k, alpha, A, lda, str_a, B, ldb, str_b,
                    beta, C, ldc, str_c, batch=1, algo=ALGO_AUTO, stream=None) -> None:
    """sbx_gemm_ex_noalloc: sbx_gemm_ex with split-K partials in the fixed
    per-device scratch (no allocation)."""
    real = ctypes.c_float if dtype == F32 else ctypes.c_double
    a = real(alpha)
    b = real(beta)
    st = lib().sbx_gemm_ex_noalloc(_stream(stream), dtype, int(layout), int(transA),
                                   int(transB), m, n, k, ctypes.byref(a), _ptr(A), lda, str_a,
                                   _ptr(B), ldb, str_b, ctypes.byref(b), _ptr(C), ldc, str_c,
                                   batch, algo)
    _check(st, "sbx_gemm_ex_noalloc")


def gemm_fused(dtype, layout, transA, transB, m, n, k, alpha, A, lda, str_a, B, ldb, str_b,
               beta, C, ldc, str_c, batch=1, epilogue=EPILOGUE_RELU, stream=None) -> None:
    """sbx_gemm_fused: C = epilogue(alpha*op(A)*op(B) + beta*C) in one launch."""
    real = ctypes.c_float if dtype == F32 else ctypes.c_double
    a = real(alpha)
    b = real(beta)
    st = lib().sbx_gemm_fused(_stream(stream), dtype, int(layout), int(transA), int(transB), m,
                              n, k, ctypes.byref(a), _ptr(A), lda, str_a, _ptr(B), ldb, str_b,
                              ctypes.byref(b), _ptr(C), ldc, str_c, batch, int(epilogue))
    _check(st, "sbx_gemm_fused")


def relu(x, n=None, dtype=None, stream=None) -> None:
    """sbx_relu in place: x = x > 0 ? x : 0 over n contiguous elements."""
    if dtype is None:
        dtype = F32 if x.element_size() == 4 else F64
    if n is None:
        n = x.numel()
    _check(lib().sbx_relu(_stream(stream), dtype, _ptr(x), n), "sbx_relu")


def sgemm(layout, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
          stream=None) -> None:
    _check(lib().sbx_sgemm(_stream(stream), int(layout), int(transA), int(transB), m, n, k,
                           alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C), ldc), "sbx_sgemm")


def dgemm(layout, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
          stream=None) -> None:
    _check(lib().sbx_dgemm(_stream(stream), int(layout), int(transA), int(transB), m, n, k,
                           alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C), ldc), "sbx_dgemm")


def gemv(dtype, layout, trans, m, n, alpha, A, lda, x, incx, beta, y, incy,
         stream=None) -> None:
    """sbx_sgemv / sbx_dgemv: y = alpha*op(A)*x + beta*y."""
    f = lib().sbx_sgemv if dtype == F32 else lib().sbx_dgemv
    _check(f(_stream(stream), int(layout), int(trans), m, n, alpha, _ptr(A), lda, _ptr(x), incx,
             beta, _ptr(y), incy), "sbx_gemv")


def syrk(dtype, layout, upper, trans, n, k, alpha, A, lda, str_a, beta, C, ldc, str_c,
         batch=1, stream=None) -> None:
    """sbx_{s,d}syrk_strided_batched: one triangle of C = alpha*op(A)*op(A)^T + beta*C."""
    f = lib().sbx_ssyrk_strided_batched if dtype == F32 else lib().sbx_dsyrk_strided_batched
    _check(f(_stream(stream), int(layout), int(upper), int(trans), n, k, alpha, _ptr(A), lda,
             str_a, beta, _ptr(C), ldc, str_c, batch), "sbx_syrk")


def gemm_select(dtype, layout, transA, transB, m, n, k, lda, ldb, ldc, batch=1) -> str:
    buf = ctypes.create_string_buffer(128)
    if batch == 1:
        _check(lib().sbx_gemm_select(dtype, layout, int(transA), int(transB), m, n, k, lda, ldb,
                                     ldc, buf, 128), "sbx_gemm_select")
    else:
        _check(lib().sbx_gemm_select_batched(dtype, layout, int(transA), int(transB), m, n, k,
                                             lda, ldb, ldc, batch, buf, 128),
               "sbx_gemm_select_batched")
    return buf.value.decode()


def _plan_lines(buf):
    out = []
    for line in buf.value.decode().splitlines():
        name, us = line.split()
        out.append((name, float(us)))
    return out


def gemm_plans(dtype, layout, transA, transB, m, n, k, lda, ldb, ldc, batch=1):
    """The candidate plans the heuristics weigh: [(plan name, predicted us)]."""
    buf = ctypes.create_string_buffer(1 << 16)
    _check(lib().sbx_gemm_plans(dtype, layout, int(transA), int(transB), m, n, k, lda, ldb, ldc,
                                batch, buf, len(buf)), "sbx_gemm_plans")
    return _plan_lines(buf)


def syrk_plans(dtype, layout, upper, trans, n, k, lda, ldc):
    """The candidate plans the heuristics weigh for a SYRK: [(plan name, predicted us)]."""
    buf = ctypes.create_string_buffer(1 << 16)
    _check(lib().sbx_syrk_plans(dtype, layout, int(upper), int(trans), n, k, lda, ldc, buf,
                                len(buf)), "sbx_syrk_plans")
    return _plan_lines(buf)


def syrk_ex_plan(dtype, layout, upper, trans, n, k, alpha, A, lda, str_a, beta, C, ldc, str_c,
                 batch=1, plan="", stream=None) -> None:
    """sbx_syrk_ex_plan: sbx_{s,d}syrk_strided_batched with a named plan."""
    real = ctypes.c_float if dtype == F32 else ctypes.c_double
    a = real(alpha)
    b = real(beta)
    st = lib().sbx_syrk_ex_plan(_stream(stream), dtype, int(layout), int(upper), int(trans), n, k,
                                ctypes.byref(a), _ptr(A), lda, str_a, ctypes.byref(b), _ptr(C),
                                ldc, str_c, batch, plan.encode())
    _check(st, "sbx_syrk_ex_plan")


def gemm_ex_plan(dtype, layout, transA, transB, m, n, k, alpha, A, lda, str_a, B, ldb, str_b,
                 beta, C, ldc, str_c, batch=1, plan="", stream=None) -> None:
    """sbx_gemm_ex_plan: sbx_gemm_ex with a named plan instead of the pick."""
    real = ctypes.c_float if dtype == F32 else ctypes.c_double
    a = real(alpha)
    b = real(beta)
    st = lib().sbx_gemm_ex_plan(_stream(stream), dtype, int(layout), int(transA), int(transB), m,
                                n, k, ctypes.byref(a), _ptr(A), lda, str_a, _ptr(B), ldb, str_b,
                                ctypes.byref(b), _ptr(C), ldc, str_c, batch, plan.encode())
    _check(st, "sbx_gemm_ex_plan")


def syrk_select(dtype, layout, upper, trans, n, k, lda, ldc) -> str:
    """Kernel (and split) sbx_{s,d}syrk would run for this problem."""
    buf = ctypes.create_string_buffer(128)
    _check(lib().sbx_syrk_select(dtype, layout, int(upper), int(trans), n, k, lda, ldc, buf, 128),
           "sbx_syrk_select")
    return buf.value.decode()


def fill_uniform(t, seed: int, stream_id: int, stream=None) -> None:
    """Fill a float32/float64 device tensor with Philox uniform [-1, 1)."""
    dtype = F32 if t.element_size() == 4 else F64
    _check(lib().sbx_fill_uniform(_stream(stream), dtype, _ptr(t), t.numel(), seed, stream_id),
           "sbx_fill_uniform")


def fill_normal(t, seed: int, stream_id: int, scale: float = 1.0, stream=None) -> None:
    """Fill a float32/float64 device tensor with Philox N(0, 1) * scale."""
    dtype = F32 if t.element_size() == 4 else F64
    _check(lib().sbx_fill_normal(_stream(stream), dtype, _ptr(t), t.numel(), seed, stream_id,
                                 scale), "sbx_fill_normal")


def version() -> str:
    return lib().sbx_version().decode()
