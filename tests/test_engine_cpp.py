"""Runs the C++ Engine-layer test binary (sushiblas_amd/cpp/tests/engine_tests.cpp):
host-only cases on any machine, device cases (the reference's GEMM,
framework-sim and dependency-stress scenarios through Engine/Tensor/
Level3::gemm) on the GPU.  Each binary run is one process; every case must
report OK."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "sushiblas_amd", "lib", "sushiblas_engine_tests")


def _run(flag, timeout):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built: run __graft_entry__.build()")
    res = subprocess.run([BIN, flag], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                         timeout=timeout)
    print(res.stdout)
    ok = re.findall(r"^\[  OK  \] (\w+)$", res.stdout, flags=re.M)
    failed = re.findall(r"^\[FAILED\] (.*)$", res.stdout, flags=re.M)
    assert res.returncode == 0 and not failed, failed or res.stdout[-2000:]
    return ok


def test_engine_host_cases():
    ok = _run("--cpu", 120)
    assert {"TensorViews", "OpIdIsFnv1a", "GemmValidationThrowsAtRecordTime"} <= set(ok)


@pytest.mark.gpu
def test_engine_device_cases(cuda):
    ok = _run("--gpu", 600)
    assert {"SimpleGEMM3x3", "SimpleGEMMColumnMajor", "FrameworkSimParallelBatchedInference",
            "DependencyManyReadersOneWriter"} <= set(ok)
