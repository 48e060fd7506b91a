"""Shared test helpers: conversions between the product PaddedCSR and the oracle."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

import oracle
from sparsecore_amd import PaddedCSR

GOLDEN = Path(__file__).resolve().parent / "golden"


def to_oracle(p: PaddedCSR) -> oracle.Csr:
    return oracle.Csr(p.nrows, p.ncols, p.values.detach().cpu().numpy(),
                      p.col_indices.cpu().numpy(), p.row_start.cpu().numpy(),
                      p.row_nnz.cpu().numpy(), p.row_capacity.cpu().numpy())


def from_oracle(c: oracle.Csr, device=None) -> PaddedCSR:
    return PaddedCSR(c.nrows, c.ncols, torch.from_numpy(c.values.copy()),
                     torch.from_numpy(c.col_indices.copy()), torch.from_numpy(c.row_start.copy()),
                     torch.from_numpy(c.row_nnz.copy()), torch.from_numpy(c.row_capacity.copy()),
                     device=device)


def make_sparse_W(M: int, K: int, sparsity: float, seed: int = 0):
    """(W_csr on CPU, W_dense) as the reference tests build them (test_spmm.py:52-69)."""
    gen = torch.Generator().manual_seed(seed)
    W = torch.randn(M, K, generator=gen, dtype=torch.float32)
    keep = torch.rand(M, K, generator=gen) >= sparsity
    W_dense = W * keep.float()
    return PaddedCSR.from_dense(W_dense), W_dense


def golden_cases():
    data = np.load(GOLDEN / "kernels.npz")
    names = sorted({k.split("/")[0] for k in data.files})
    out = {}
    for n in names:
        out[n] = {k.split("/", 1)[1]: data[k] for k in data.files if k.startswith(n + "/")}
    return out


def golden_csr(case) -> oracle.Csr:
    M, K, _ = (int(v) for v in case["shape"])
    return oracle.Csr(M, K, case["values"], case["col_indices"], case["row_start"],
                      case["row_nnz"], case["row_capacity"])


def c1_inputs():
    """BASELINE config-1 inputs regenerated from tests/golden/gen.py."""
    import json

    import gen

    meta = json.loads((GOLDEN / "c1.json").read_text())
    g = meta["gen"]
    M, K, N = g["M"], g["K"], g["N"]
    parts = gen.padded_csr(M, K, np.full(M, g["nnz_per_row"], np.int32), g["csr_seed"],
                           g["sigma"], g["padding_ratio"])
    p = oracle.Csr(M, K, *parts)
    X = gen.normalish(g["X_seed"], K * N).reshape(K, N)
    dY = gen.normalish(g["dY_seed"], M * N).reshape(M, N)
    assert gen.digest(p.values) == meta["inputs_sha256"]["values"]
    assert gen.digest(p.col_indices) == meta["inputs_sha256"]["col_indices"]
    assert gen.digest(X) == meta["inputs_sha256"]["X"]
    assert gen.digest(dY) == meta["inputs_sha256"]["dY"]
    return meta, p, X, dY


def assert_bits_equal(a, b, what: str = "") -> None:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, f"{what}: shape {a.shape} != {b.shape}"
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), b.view(np.uint32)
    diff = np.flatnonzero(a.reshape(-1) != b.reshape(-1))
    assert diff.size == 0, (f"{what}: {diff.size} of {a.size} elements differ, first at flat "
                            f"index {int(diff[0])}")


def csr_arrays_equal(a: oracle.Csr, b: oracle.Csr, what: str = "") -> None:
    assert (a.nrows, a.ncols) == (b.nrows, b.ncols), what
    for name in ("values", "col_indices", "row_start", "row_nnz", "row_capacity"):
        assert_bits_equal(getattr(a, name), getattr(b, name), f"{what}.{name}")
