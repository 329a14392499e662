"""Shared test set-up: import paths, the `gpu` marker, and helpers.

`-m "not gpu"` tests run on any host (oracle, host logic, library load/exports);
`-m gpu` tests call the HIP library through its C ABI on an MI355X.
"""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "rdna4-gemm-wmma_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls the HIP library")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def mm():
    """The product library; on a GPU run it must load (no fallback)."""
    import mmm

    mmm.lib()
    return mmm


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch


def to_dev(torch, a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()
