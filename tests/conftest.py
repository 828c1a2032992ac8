"""Test configuration: import paths, the ``gpu`` marker and shared fixtures.

CPU tests (``-m "not gpu"``) pin the oracle and check the host-side pieces; GPU
tests (``-m gpu``) compare the HIP library, through custom_rasterizer_cuda and
the C ABI, with the oracle.  GPU tests fail (not skip) when the extension is
missing, so a box without the native build cannot pass them silently.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "custom-3dgs-cuda_amd"
for p in (str(ROOT), str(PKG), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o

    o.build()
    return o


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a HIP device (run CPU tests with -m 'not gpu')")
    return torch.device("cuda")


@pytest.fixture(scope="session")
def crc(device):
    import custom_rasterizer_cuda  # noqa: F401  (fails loudly if the build is missing)

    return custom_rasterizer_cuda
