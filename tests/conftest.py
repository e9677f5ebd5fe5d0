"""pytest configuration: the `gpu` marker and shared fixtures.

`-m "not gpu"` runs the oracle, host-logic and ABI-export tests on any
machine; `-m gpu` runs the parity tests that launch HIP kernels through the
C ABI and needs an MI355X.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")
