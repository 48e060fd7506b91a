"""CPU tests of the host-side logic (no GPU needed).

Restates the reference's tests/test_padded_csr.py and the host-visible parts
of test_padded_csr_rewrite.py / test_sparse_linear.py / test_spmm.py against
the product's PaddedCSR held in CPU tensors, and pins the product's host
invariant checker to the oracle's restatement of the reference checker.
Kernels are not run here: the product has no CPU path, which is checked too.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import sparsecore_amd as slk
from helpers import assert_bits_equal, from_oracle, to_oracle
from sparsecore_amd import PaddedCSR, SparseLinear
from sparsecore_amd.layout import _compute_row_capacity


# ───────────────────────── construction (test_padded_csr.py) ───────────

def test_empty_constructor_shape():
    p = PaddedCSR(nrows=5, ncols=10)
    assert p.shape == (5, 10) and (p.nrows, p.ncols) == (5, 10)
    assert p.nnz == 0 and p.total_capacity == 0
    assert repr(p) == "PaddedCSR(nrows=5, ncols=10, nnz=0, capacity=0)"


def test_from_dense_known_answer():
    W = torch.tensor([[3.0, 0.0, 0.0, 1.0], [0.0, 0.0, 2.0, 5.0], [4.0, 0.0, 0.0, 0.0]])
    p = PaddedCSR.from_dense(W, padding_ratio=0.5)
    assert p.shape == (3, 4) and p.nnz == 5
    assert p.row_capacity.tolist() == [3, 3, 2]
    assert p.row_nnz.tolist() == [2, 2, 1]
    assert p.row_start.tolist() == [0, 3, 6]
    assert torch.equal(p.to_dense(), W)


def test_from_torch_sparse_csr_matches_from_dense():
    W = torch.tensor([[1.0, 0.0, 2.0], [0.0, 3.0, 0.0]])
    p1 = PaddedCSR.from_dense(W, padding_ratio=0.2)
    p2 = PaddedCSR.from_torch_sparse_csr(W.to_sparse_csr(), padding_ratio=0.2)
    assert torch.equal(p1.to_dense(), W) and torch.equal(p2.to_dense(), W)
    for name in ("values", "col_indices", "row_start", "row_nnz", "row_capacity"):
        assert torch.equal(getattr(p1, name), getattr(p2, name))


def test_from_dense_matches_oracle_layout():
    rng = np.random.default_rng(0)
    W = rng.standard_normal((37, 53)).astype(np.float32)
    W[rng.random((37, 53)) < 0.8] = 0
    for pr in (0.0, 0.2, 0.5, 1.0, 2.0):
        got = to_oracle(PaddedCSR.from_dense(torch.from_numpy(W), padding_ratio=pr))
        want = oracle.from_dense(W, padding_ratio=pr)
        for name in ("values", "col_indices", "row_start", "row_nnz", "row_capacity"):
            assert_bits_equal(getattr(got, name), getattr(want, name), name)


def test_random_factory():
    p = PaddedCSR.random(500, 500, sparsity=0.9, seed=42)
    assert abs(p.sparsity - 0.9) < 0.01
    a = PaddedCSR.random(100, 100, sparsity=0.9, seed=7)
    b = PaddedCSR.random(100, 100, sparsity=0.9, seed=7)
    assert a.nnz == b.nnz and torch.equal(a.values, b.values)
    assert torch.equal(a.col_indices, b.col_indices)
    for bad in (-0.1, 1.0, 1.5):
        with pytest.raises(ValueError, match="sparsity"):
            PaddedCSR.random(10, 10, sparsity=bad)


@pytest.mark.parametrize("shape", [(1, 1), (1, 10), (10, 1), (7, 7), (50, 100)])
def test_round_trip(shape):
    torch.manual_seed(sum(shape))
    W = torch.randn(*shape) * (torch.rand(*shape) > 0.5).float()
    assert torch.equal(PaddedCSR.from_dense(W).to_dense(), W)


def test_round_trip_large_and_dense_row():
    torch.manual_seed(0)
    W = torch.randn(1024, 1024) * (torch.rand(1024, 1024) > 0.95).float()
    assert torch.equal(PaddedCSR.from_dense(W).to_dense(), W)
    W = torch.tensor([[1.0, 2.0, 3.0, 4.0, 5.0], [0.0] * 5])
    assert torch.equal(PaddedCSR.from_dense(W).to_dense(), W)


@pytest.mark.parametrize("padding_ratio", [0.0, 0.2, 0.5, 1.0, 2.0])
@pytest.mark.parametrize("seed", [0, 1, 2, 7, 42])
def test_invariants_after_random_construction(padding_ratio, seed):
    PaddedCSR.random(50, 80, sparsity=0.85, padding_ratio=padding_ratio,
                     seed=seed).assert_invariants()


def test_capacity_rule():
    torch.manual_seed(0)
    W = torch.randn(10, 10) * (torch.rand(10, 10) > 0.5).float()
    p = PaddedCSR.from_dense(W, padding_ratio=0.0)
    for n, cap in zip(p.row_nnz.tolist(), p.row_capacity.tolist()):
        assert cap == max(1, n)
    p = PaddedCSR.random(100, 100, sparsity=0.9, padding_ratio=0.3, seed=1)
    assert p.padding_slots == p.total_capacity - p.nnz
    assert _compute_row_capacity(np.array([0, 1, 5, 10]), 0.5).tolist() == [1, 2, 8, 15]
    for nnz in range(0, 200, 7):
        for pr in (0.0, 0.1, 0.2, 0.3, 1 / 3, 0.7):
            assert (_compute_row_capacity(np.array([nnz]), pr).tolist()
                    == oracle.row_capacity([nnz], pr).tolist())


@pytest.mark.parametrize("padding_ratio", [0.0, 0.1, 0.2, 0.3, 1.0 / 3.0, 0.7, 1.0, 2.5])
def test_transpose_capacity_bound_covers_the_rule(padding_ratio):
    """The transpose sizes its slot arrays by _capacity_bound before it reads
    the exact capacity: the bound must never undercut the capacity rule, for
    any split of nnz over the rows (empty rows, one full row, many short rows,
    random), including padding ratios whose float64 is inexact."""
    from sparsecore_amd.layout import _capacity_bound

    rng = np.random.default_rng(int(padding_ratio * 1000))
    for rows, counts in [
        (1, np.array([0])), (5, np.zeros(5, np.int64)), (3, np.array([0, 0, 1000003])),
        (1000, np.ones(1000, np.int64)), (1000, rng.integers(0, 50, 1000)),
        (16384, rng.integers(0, 2000, 16384)), (7, np.array([1, 2, 3, 5, 8, 13, 21])),
        (4096, rng.zipf(1.3, 4096).clip(0, 100000)),
    ]:
        exact = int(_compute_row_capacity(counts, padding_ratio).astype(np.int64).sum())
        bound = _capacity_bound(int(counts.sum()), rows, padding_ratio)
        assert bound >= exact, (padding_ratio, rows, bound, exact)
        assert bound <= exact + 2 * rows + 2  # and not wasteful


def test_edge_matrices():
    p = PaddedCSR.from_dense(torch.zeros(5, 5))
    assert p.nnz == 0 and p.row_capacity.tolist() == [1] * 5
    assert torch.equal(p.to_dense(), torch.zeros(5, 5))
    p = PaddedCSR.from_dense(torch.tensor([[7.5]]))
    assert p.shape == (1, 1) and p.nnz == 1
    p = PaddedCSR(nrows=0, ncols=5)
    assert p.shape == (0, 5) and p.total_capacity == 0
    p.assert_invariants()
    W = torch.tensor([[0.1, 0.6, 0.0, -0.4], [1.0, -2.0, 0.3, 0.0]])
    p = PaddedCSR.from_dense(W, threshold=0.5)
    assert p.nnz == 3
    assert torch.equal(p.to_dense(), torch.tensor([[0.0, 0.6, 0.0, 0.0],
                                                   [1.0, -2.0, 0.0, 0.0]]))


def test_construction_errors():
    with pytest.raises(ValueError, match="2-D"):
        PaddedCSR.from_dense(torch.zeros(5))
    with pytest.raises(ValueError, match="2-D"):
        PaddedCSR.from_dense(torch.zeros(2, 3, 4))
    with pytest.raises(ValueError, match="padding_ratio"):
        PaddedCSR.from_dense(torch.zeros(3, 3), padding_ratio=-0.1)
    with pytest.raises(ValueError, match="Invariant 2 violated"):
        PaddedCSR(nrows=2, ncols=3, values=[1.0, 2.0, 3.0], col_indices=[0, 1],
                  row_start=[0, 2], row_nnz=[1, 1], row_capacity=[1, 1])
    with pytest.raises(ValueError, match="sorted"):
        PaddedCSR(nrows=1, ncols=5, values=[1.0, 2.0], col_indices=[3, 1], row_start=[0],
                  row_nnz=[2], row_capacity=[2])
    with pytest.raises(ValueError, match="Invariant 6"):
        PaddedCSR(nrows=1, ncols=3, values=[1.0], col_indices=[5], row_start=[0],
                  row_nnz=[1], row_capacity=[1])
    with pytest.raises(TypeError):
        PaddedCSR(2, 2, values=[1.0])


def test_host_checker_matches_oracle_checker():
    """Host invariant checker: message-for-message with the oracle's restatement
    (itself pinned to the reference checker in test_oracle.py)."""
    rng = np.random.default_rng(3)
    base = oracle.uniform_rows(15, 25, 6, seed=2)
    for trial in range(120):
        q = base.copy()
        kind = trial % 7
        i = int(rng.integers(0, q.nrows))
        s, n, cap = int(q.row_start[i]), int(q.row_nnz[i]), int(q.row_capacity[i])
        if kind == 0:
            q.col_indices[s + int(rng.integers(0, n))] = int(rng.integers(-3, 28))
        elif kind == 1:
            q.col_indices[s], q.col_indices[s + 1] = q.col_indices[s + 1], q.col_indices[s]
        elif kind == 2 and cap > n:
            q.col_indices[s + n + int(rng.integers(0, cap - n))] = 4
        elif kind == 3:
            q.row_nnz[i] = int(rng.integers(-2, cap + 3))
        elif kind == 4:
            q.row_start[i] += int(rng.integers(-1, 2))
        elif kind == 5:
            q.row_capacity[i] += 1
        elif kind == 6:
            j = int(rng.integers(0, q.nrows))
            q.col_indices[int(q.row_start[j])] = -1
        expect = oracle.check_invariants(q.nrows, q.ncols, q.values, q.col_indices,
                                         q.row_start, q.row_nnz, q.row_capacity)
        if expect:
            with pytest.raises(ValueError) as ei:
                from_oracle(q)
            assert str(ei.value) == "PaddedCSR invariant check failed: " + expect
        else:
            from_oracle(q).assert_invariants()


# ───────────────────── rewrite_row (test_padded_csr_rewrite.py) ────────

def test_rewrite_row_host_semantics():
    c = oracle.uniform_rows(5, 12, 4, seed=1)
    p = from_oracle(c)
    p.rewrite_row(2, np.array([1, 7, 11], dtype=np.int32), np.array([7.0, 8.0, 9.0]))
    q = oracle.rewrite_row(c, 2, [1, 7, 11], [7.0, 8.0, 9.0])
    got = to_oracle(p)
    for name in ("values", "col_indices", "row_nnz"):
        assert_bits_equal(getattr(got, name), getattr(q, name), name)
    assert p.topology_version == 1 and p.nnz == q.nnz
    p.assert_invariants()
    with pytest.raises(ValueError, match="out of range"):
        p.rewrite_row(-1, [0], [1.0])
    with pytest.raises(ValueError, match="out of range"):
        p.rewrite_row(0, [12], [1.0])
    with pytest.raises(ValueError, match="ascending"):
        p.rewrite_row(0, [5, 2], [1.0, 1.0])
    with pytest.raises(ValueError, match="must equal"):
        p.rewrite_row(0, [1, 2], [1.0])
    with pytest.raises(ValueError, match="capacity"):
        p.rewrite_row(0, list(range(10)), [1.0] * 10)
    with pytest.raises(ValueError, match="1-D"):
        p.rewrite_row(0, [[1]], [[1.0]])
    assert p.topology_version == 1


# ───────────────────────── GPU-only contract ───────────────────────────

def test_kernels_reject_cpu_tensors():
    W = PaddedCSR.random(8, 16, sparsity=0.5, seed=0)
    with pytest.raises(RuntimeError, match="HIP"):
        slk.spmm(W, torch.randn(16, 4))
    with pytest.raises(TypeError, match="PaddedCSR"):
        slk.spmm(torch.randn(8, 16), torch.randn(16, 4))
    with pytest.raises(TypeError, match="torch.Tensor"):
        slk.spmm(W, np.zeros((16, 4), np.float32))
    with pytest.raises(RuntimeError, match="HIP device only"):
        W.transpose()
    layer = SparseLinear(16, 8, sparsity=0.5)
    with pytest.raises(RuntimeError, match="HIP"):
        layer(torch.randn(4, 16))


# ───────────────────────── SparseLinear (host side) ────────────────────

def test_sparse_linear_construction():
    torch.manual_seed(0)
    layer = SparseLinear(64, 32)
    assert layer.in_features == 64 and layer.out_features == 32 and layer.bias is not None
    assert 0.08 < layer.density < 0.12
    with pytest.raises(ValueError, match="sparsity"):
        SparseLinear(8, 4, sparsity=1.0)
    with pytest.raises(ValueError, match="sparsity"):
        SparseLinear(8, 4, sparsity=-0.1)
    assert SparseLinear(16, 8, bias=False).bias is None
    text = repr(SparseLinear(8, 4, sparsity=0.5))
    for field in ("in_features=8", "out_features=4", "sparsity=0.5", "nnz="):
        assert field in text


def test_sparse_linear_values_alias_csr_buffer():
    layer = SparseLinear(16, 8, sparsity=0.5)
    assert layer._values.data_ptr() == layer._csr.values.data_ptr()
    with torch.no_grad():
        layer._values.fill_(0.25)
    assert torch.all(layer._csr.values == 0.25)
    assert {n for n, _ in layer.named_parameters()} == {"_values", "bias"}
    assert {"_values", "bias"} <= set(layer.state_dict())  # plus the topology keys
    layer.double()  # the CSR keeps its float32 buffer, as the reference does
    assert layer._values.dtype == torch.float64 and layer._csr.values.dtype == torch.float32


# ───────────── SparseLinear topology serialization (CPU, no kernels) ─────────

def _layers(seed_a=0, seed_b=5):
    torch.manual_seed(seed_a)
    a = SparseLinear(16, 8, sparsity=0.5)
    torch.manual_seed(seed_b)
    b = SparseLinear(16, 8, sparsity=0.5)
    return a, b


def _same_topology(a, b):
    for name in ("values", "col_indices", "row_start", "row_nnz", "row_capacity"):
        assert torch.equal(getattr(a._csr, name), getattr(b._csr, name)), name
    assert a._csr.topology_version == b._csr.topology_version


def test_state_dict_carries_the_topology():
    a, b = _layers()
    assert not torch.equal(a._csr.col_indices, b._csr.col_indices) or \
        a._csr.total_capacity != b._csr.total_capacity
    sd = a.state_dict()
    assert {"_values", "bias", "csr_col_indices", "csr_row_start", "csr_row_nnz",
            "csr_row_capacity", "csr_topology_version"} == set(sd)
    b.load_state_dict(sd)  # strict: every key is consumed
    _same_topology(a, b)
    assert b._csr.values.data_ptr() == b._values.data_ptr()  # aliasing kept


def test_state_dict_after_rewrite_row_and_torch_save_roundtrip(tmp_path):
    a, b = _layers(1, 2)
    a._csr.rewrite_row(3, [0, 5, 9], [0.5, -1.0, 2.0])
    assert a._csr.topology_version == 1
    path = tmp_path / "layer.pt"
    torch.save(a.state_dict(), path)
    b.load_state_dict(torch.load(path, weights_only=True))
    _same_topology(a, b)
    assert b._csr.row_nnz[3] == 3 and b._csr.topology_version == 1


def test_values_only_state_dict_still_loads():
    """A reference-style checkpoint (no topology keys) loads the values into a
    layer built from the same seed, strictly (tests/test_sparse_linear.py:312-335)."""
    a, b = _layers(0, 0)
    with torch.no_grad():
        a._values.mul_(2.0)
    sd = {k: v for k, v in a.state_dict().items() if not k.startswith("csr_")}
    b.load_state_dict(sd)
    assert torch.equal(a._values, b._values) and b._csr.values.data_ptr() == b._values.data_ptr()


def test_partial_or_invalid_topology_is_rejected():
    a, b = _layers()
    sd = a.state_dict()
    partial = dict(sd)
    del partial["csr_row_nnz"]
    with pytest.raises(RuntimeError, match="partial topology"):
        b.load_state_dict(partial)
    bad = dict(sd)
    cols = bad["csr_col_indices"].clone()
    s0 = int(bad["csr_row_start"][0])
    if int(bad["csr_row_nnz"][0]) >= 2:
        cols[s0], cols[s0 + 1] = cols[s0 + 1].clone(), cols[s0].clone()  # unsorted row 0
    else:
        cols[s0] = 999  # out of range
    bad["csr_col_indices"] = cols
    with pytest.raises(RuntimeError, match="invalid topology"):
        b.load_state_dict(bad)
