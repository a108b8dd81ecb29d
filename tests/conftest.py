"""Shared test setup: import paths, the `gpu` marker and device fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("decision-programs_amd", "oracle"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); parity through the C ABI")


@pytest.fixture(scope="session")
def oracle():
    import pyoracle

    pyoracle.load()
    return pyoracle


@pytest.fixture(scope="session")
def dp():
    import dpgbdt

    dpgbdt.load()
    return dpgbdt


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a HIP device")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def ws(dp, device):
    from dpgbdt import ops

    return ops.Workspace()
