"""pytest setup: import paths, the ``gpu`` marker, and a GPU device fixture.

``-m "not gpu"`` runs on any host (oracle, host logic, the C ABI's symbol table);
``-m gpu`` needs a ROCm device and the built ``libdspark_rocm.so`` and never skips for
their absence — a GPU test that cannot reach the HIP kernels fails.
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mlx-dspark_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("GPU test without a ROCm device")
    from dspark_rocm import _lib

    _lib.load()  # raise now if the kernel library is missing
    return torch.device("cuda:0")
