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


@pytest.fixture
def tune():
    """Forces kernel / schedule choices for one test and restores the
    launchers' own choices afterwards: tune(spmm_kernel=1, spmm_rw=4, ...)
    for the library's knobs (slk_set_tuning), tune(spmm_phases=3) or
    tune(seg=(64, 8)) or tune(bin_shape=(8, 2)) for the host-side schedule
    overrides of ops."""
    from sparsecore_amd import _lib, ops

    host_keys = ("spmm_phases", "seg", "bin_shape", "fused_backward")
    touched = []

    def set_(**kw):
        for k, v in kw.items():
            if k in host_keys:
                ops._overrides[k] = v
            else:
                _lib.set_tuning(k, v)
            touched.append(k)

    yield set_
    for k in touched:
        if k in host_keys:
            ops._overrides.pop(k, None)
        else:
            _lib.set_tuning(k, None)
