"""Shared pytest configuration.

Markers
  gpu   needs a HIP device (MI355X) and the built gfx950 library; the round
        driver runs these with `pytest -m gpu` on the GPU box.

Everything unmarked runs on a CPU-only machine: the oracle against the
reference build and the golden fixtures, the host-side logic, and the C-ABI
library's exports.
"""

from __future__ import annotations

import sys
import warnings
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (str(ROOT), str(ROOT / "tests"), str(ROOT / "tests" / "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device and the built gfx950 library")


@pytest.fixture(autouse=True)
def _quiet_known_warnings():
    with warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="Sparse CSR tensor support is in beta state.*")
        warnings.filterwarnings("ignore", message="The given NumPy array is not writable.*")
        yield


@pytest.fixture(scope="session")
def dev():
    import torch

    import sparsecore_amd

    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but no HIP device is visible")
    if not sparsecore_amd.native_available():
        pytest.fail("gpu test selected but libsparsecore_amd.so is not built")
    return torch.device("cuda:0")
