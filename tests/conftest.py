"""Shared pytest setup: the `gpu` marker, import paths, device fixtures.

CPU tests (-m "not gpu") cover the oracle against golden vectors and
closed forms, the host logic, and that libllmt.so loads and exports every
symbol of include/llmt.h.  GPU tests (-m gpu) call the HIP library through
its C ABI and compare with the oracle on the same seeded inputs.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT), str(ROOT / "llm.cu_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs libllmt.so kernels)")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def L():
    """The loaded libllmt.so (GPU tests require it to be built in-tree)."""
    import llmt
    return llmt.lib()


def rel_l2(a, b):
    """||a - b|| / ||b|| in float64."""
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))
