"""Shared test setup.

`gpu`-marked tests need a ROCm GPU and the built HIP library; everything else
runs on the CPU.  The CPU oracle (oracle/) is the parity checker.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "rwkv-metal_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and librwkvq_hip.so")


@pytest.fixture(scope="session")
def O():
    from oracle import oracle as _o
    if not os.path.exists(_o._LIB_PATH):
        _o.build()
    return _o


@pytest.fixture(scope="session")
def rq():
    import rwkvq
    return rwkvq


@pytest.fixture(scope="session")
def dev():
    import torch
    # a gpu-marked test on a machine without a GPU is a failure, not a skip
    assert torch.cuda.is_available(), "gpu-marked test run without a visible ROCm GPU"
    return torch.device("cuda:0")
