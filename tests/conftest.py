"""pytest configuration: the `gpu` marker and shared helpers.

`-m "not gpu"` runs here (no GPU): oracle vs golden fixtures, host logic and
the C-ABI export check.  `-m gpu` runs on an MI355X and calls the HIP kernels
through the C ABI; those tests fail (not skip) when no GPU is present.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def cuda():
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    from leankv_amd import _lib

    _lib.load()  # fails loudly if the HIP library was not built
    return torch.device("cuda:0")
