"""CPU oracle for the SushiBLAS GEMM hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed
CPU baseline).  The product (``sushiblas_amd``) never imports it.

The arithmetic lives in ``oracle/sbo.c`` (plain C + OpenMP); this module is a
numpy/ctypes front end over ``oracle/lib/libsbo.so``.  ``sbo.h`` lists the
reference lines each routine restates and the checks that pin it.
"""
from .sbo import (  # noqa: F401
    build,
    lib_path,
    gemm,
    gemm_strided_batched,
    gemm_naive_ld,
    rel_fro_err,
    philox4x32_10,
    fill_uniform,
    fill_normal,
    relu,
    gemv,
    syrk,
    syrk_strided_batched,
    num_threads,
)
