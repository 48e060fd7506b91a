"""GPU parity of the topology kernels (threshold select, SET / RigL drop-grow,
dense gradient) against the oracle, and the reference's SET / RigL / router
test suites (tests/test_set.py, test_rigl.py, test_router.py,
test_set_rigl_with_cache.py, test_dense_grad.py) restated on the device.

Bar: bit-exact. The threshold is a selection (exact), the rewritten rows are
integer/data movement decided by exact comparisons, and dense_grad keeps the
reference build's summation order per element.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import oracle
from helpers import assert_bits_equal, csr_arrays_equal, from_oracle, to_oracle
from sparsecore_amd import RigL, SET, SparseLinear, Static, _lib, ops
from sparsecore_amd.ops import _clear_transpose_cache, _dense_grad_token_major

pytestmark = pytest.mark.gpu


def _thr(W, k):
    dev = W.device
    ws = torch.empty(_lib.SLK_KTH_WORKSPACE_BYTES, dtype=torch.uint8, device=dev)
    thr = torch.empty(1, dtype=torch.float32, device=dev)
    _lib.live_abs_kth(W._view(), k, ws, thr)
    return thr.cpu().numpy()


# ───────────────────────────── threshold ───────────────────────────────

@pytest.mark.parametrize("seed", range(3))
def test_live_abs_kth_bit_exact(dev, seed):
    print(f"[kth] seed={seed}", flush=True)
    c = oracle.zipf_rows(300, 500, 0.05, 1.1, seed=seed, sigma=1.0)
    rng = np.random.default_rng(seed)
    live = c.col_indices >= 0
    if seed == 1:  # many ties, signed zeros
        c.values[live] = (rng.integers(-6, 7, size=int(live.sum())) * 0.5).astype(np.float32)
        c.values[np.flatnonzero(live)[:50]] = np.float32(-0.0)
    if seed == 2:  # tiny and huge magnitudes, subnormals
        c.values[live] = (rng.standard_normal(int(live.sum())) *
                          10.0 ** rng.integers(-44, 38, size=int(live.sum()))).astype(np.float32)
    W = from_oracle(c, dev)
    for k in sorted({1, 2, c.nnz // 7, c.nnz // 2, c.nnz - 1, c.nnz}):
        want = np.array([oracle.live_abs_kth(c, k)], np.float32)
        assert_bits_equal(_thr(W, k), want, f"k={k}")


def test_live_abs_kth_rejects_bad_k(dev):
    c = oracle.uniform_rows(4, 8, 2, seed=0)
    W = from_oracle(c, dev)
    with pytest.raises(ValueError, match="k="):
        _thr(W, 0)
    with pytest.raises(ValueError, match="k_drop"):
        W._drop_grow(c.nnz + 1, _lib.SLK_GROW_RANDOM)


# ───────────────────────────── drop / grow ─────────────────────────────

def _matrices():
    yield "uniform", oracle.uniform_rows(64, 100, 10, seed=1, sigma=1.0)
    yield "zipf", oracle.zipf_rows(256, 700, 0.06, 1.1, seed=2, sigma=1.0)
    yield "wide", oracle.uniform_rows(20, 5000, 40, seed=3, sigma=1.0)
    yield "dense_rows", oracle.from_dense(
        np.random.default_rng(4).standard_normal((12, 33)).astype(np.float32))
    W = np.random.default_rng(5).standard_normal((40, 64)).astype(np.float32)
    W[W < 0.8] = 0
    W[::5] = 0  # empty rows
    yield "empty_rows", oracle.from_dense(W)


@pytest.mark.parametrize("rule", ["random", "gradient"])
@pytest.mark.parametrize("df", [0.3, 0.99, 0.01])
def test_drop_grow_bit_exact(dev, rule, df):
    for name, c in _matrices():
        print(f"[drop_grow] {name} rule={rule} df={df}", flush=True)
        k = max(1, int(df * c.nnz))
        rng = np.random.default_rng(7)
        G = rng.standard_normal((c.nrows, c.ncols)).astype(np.float32)
        if name == "zipf":  # heavy ties in |G|
            G = np.round(G * 2) / 2
        want = oracle.drop_grow(c, k, rule, G if rule == "gradient" else None, seed=99)
        W = from_oracle(c, dev)
        v0 = W.topology_version
        W._drop_grow(k, _lib.SLK_GROW_GRADIENT if rule == "gradient" else _lib.SLK_GROW_RANDOM,
                     torch.from_numpy(G).to(dev) if rule == "gradient" else None, 99)
        assert W.topology_version == v0 + 1
        csr_arrays_equal(to_oracle(W), want, f"{name}")
        assert W._check_device() == ""


def test_drop_grow_on_tall_matrix_keeps_row_schedule(dev):
    c = oracle.zipf_rows(3000, 300, 0.05, 1.1, seed=6, sigma=1.0)
    W = from_oracle(c, dev)
    W._view()
    order_before = W._order[1].clone()
    W._drop_grow(max(1, int(0.3 * c.nnz)), _lib.SLK_GROW_RANDOM, None, 5)
    W._view()
    assert torch.equal(W._order[1], order_before)
    want = oracle.drop_grow(c, max(1, int(0.3 * c.nnz)), "random", seed=5)
    csr_arrays_equal(to_oracle(W), want, "tall")
    X = np.random.default_rng(0).standard_normal((300, 96)).astype(np.float32)
    Y = ops._launch_spmm(W, torch.from_numpy(X).to(dev)).cpu().numpy()
    assert_bits_equal(Y, oracle.spmm(want, X), "Y after drop_grow")


# ───────────────────────────── dense gradient ──────────────────────────

@pytest.mark.parametrize("M,K,N", [(5, 7, 4), (32, 64, 16), (128, 256, 32), (1, 1, 1), (1, 8, 4),
                                   (8, 1, 4), (130, 257, 19), (200, 129, 3), (64, 64, 2),
                                   (300, 70, 133)])
def test_dense_grad_bit_exact(dev, M, K, N):
    print(f"[dense_grad] {M}x{K} N={N}", flush=True)
    rng = np.random.default_rng(M * 7 + K + N)
    dY = rng.standard_normal((M, N)).astype(np.float32)
    X = rng.standard_normal((K, N)).astype(np.float32)
    want = oracle.dense_grad(dY, X)
    G = ops.dense_grad(torch.from_numpy(dY).to(dev), torch.from_numpy(X).to(dev))
    assert_bits_equal(G.cpu().numpy(), want, "G")
    Gt = _dense_grad_token_major(torch.from_numpy(dY.T.copy()).to(dev),
                                 torch.from_numpy(X.T.copy()).to(dev))
    assert_bits_equal(Gt.cpu().numpy(), want, "G token-major")
    np.testing.assert_allclose(G.cpu().numpy(), dY.astype(np.float64) @ X.T.astype(np.float64),
                               rtol=1e-4, atol=1e-4)


def test_dense_grad_edges_and_errors(dev):
    G = ops.dense_grad(torch.zeros(0, 4, device=dev), torch.zeros(5, 4, device=dev))
    assert G.shape == (0, 5)
    G = ops.dense_grad(torch.zeros(3, 0, device=dev), torch.zeros(5, 0, device=dev))
    assert G.shape == (3, 5) and torch.count_nonzero(G).item() == 0
    with pytest.raises(ValueError, match="2-D"):
        ops.dense_grad(torch.zeros(5, device=dev), torch.zeros(3, 5, device=dev))
    with pytest.raises(ValueError, match="must equal"):
        ops.dense_grad(torch.zeros(4, 6, device=dev), torch.zeros(3, 5, device=dev))
    dY = torch.randn(128, 32, device=dev)
    X = torch.randn(64, 32, device=dev)
    assert torch.equal(ops.dense_grad(dY, X), ops.dense_grad(dY, X))


def test_dense_grad_matches_sddmm_scalar_at_live_positions(dev):
    """test_dense_grad.py:98-128: dense G at live (i, c) equals dW of the
    scalar-order kernel bit for bit (same running sum)."""
    c = oracle.uniform_rows(40, 90, 11, seed=3, sigma=1.0)
    rng = np.random.default_rng(3)
    dY = rng.standard_normal((40, 77)).astype(np.float32)
    X = rng.standard_normal((90, 77)).astype(np.float32)
    W = from_oracle(c, dev)
    dW = ops._launch_sddmm(W, torch.from_numpy(dY).to(dev), torch.from_numpy(X).to(dev),
                           "scalar").cpu().numpy()
    G = ops.dense_grad(torch.from_numpy(dY).to(dev), torch.from_numpy(X).to(dev)).cpu().numpy()
    slots, rows, cols = oracle.live_slots(c)
    assert_bits_equal(dW[slots], G[rows, cols], "live G")


# ───────────────────────── reference suites, restated ──────────────────

def _layer(i, o, sparsity, dev, bias=True, seed=0):
    torch.manual_seed(seed)
    np.random.seed(seed)
    return SparseLinear(i, o, sparsity=sparsity, bias=bias).to(dev)


def test_router_base_api(dev):
    with pytest.raises(ValueError):
        Static(sparsity=1.0)
    with pytest.raises(ValueError):
        SET(sparsity=0.9, drop_fraction=0.0)
    with pytest.raises(ValueError):
        SET(sparsity=0.9, update_freq=0)
    layer = _layer(16, 8, 0.5, dev)
    algo = Static(sparsity=0.5)
    layer.apply(algo)
    layer.apply(algo)
    assert algo.layers == [layer] and layer._sparsity_algorithm is algo
    with pytest.raises(TypeError):
        algo.attach(nn.Linear(2, 2))
    model = nn.Sequential(nn.Linear(4, 16), _layer(16, 8, 0.5, dev), nn.ReLU(),
                          _layer(8, 4, 0.5, dev))
    a2 = SET(sparsity=0.5, drop_fraction=0.3, update_freq=1)
    model.apply(a2)
    assert len(a2.layers) == 2
    assert "n_layers=2" in repr(a2) and "drop_fraction=0.3" in repr(a2)
    cols = layer._csr.col_indices.clone()
    algo.step()
    assert torch.equal(cols, layer._csr.col_indices)


def test_dynamic_step_gates_update_by_frequency(dev):
    layer = _layer(32, 16, 0.8, dev)
    algo = SET(sparsity=0.8, drop_fraction=0.3, update_freq=3, seed=1)
    layer.apply(algo)
    with torch.no_grad():
        layer._values.data.uniform_(-1.0, 1.0)
    versions = []
    for _ in range(7):
        algo.step()
        versions.append(layer._csr.topology_version)
    assert versions == [0, 0, 1, 1, 1, 2, 2]


def test_set_update_semantics(dev):
    layer = _layer(64, 32, 0.9, dev)
    algo = SET(sparsity=0.9, drop_fraction=0.3, update_freq=1, seed=3)
    layer.apply(algo)
    with torch.no_grad():
        layer._values.data.uniform_(-1.0, 1.0)
    before = to_oracle(layer._csr)
    nnz = layer.nnz
    algo.update()
    after = to_oracle(layer._csr)
    assert layer.nnz == nnz
    assert (before.col_indices != after.col_indices).any()
    layer._csr.assert_invariants()
    live_before = {(i, int(cc)) for i in range(before.nrows)
                   for cc in before.col_indices[before.row_start[i]:before.row_start[i] +
                                                before.row_nnz[i]]}
    for i in range(after.nrows):
        s, n = after.row_start[i], after.row_nnz[i]
        for cc, v in zip(after.col_indices[s:s + n], after.values[s:s + n]):
            if (i, int(cc)) not in live_before:
                assert v == 0.0
    # the same update from the oracle with the seed SET drew
    rng = np.random.default_rng(3)
    seed = int(rng.integers(0, 2**63, dtype=np.int64))
    want = oracle.drop_grow(before, max(1, int(0.3 * nnz)), "random", seed=seed)
    csr_arrays_equal(after, want, "SET update")


def test_set_keeps_every_row_nonempty_and_is_seeded(dev):
    layer = _layer(16, 8, 0.9, dev)
    algo = SET(sparsity=0.9, drop_fraction=0.99, update_freq=1)
    layer.apply(algo)
    with torch.no_grad():
        layer._values.data.uniform_(-1.0, 1.0)
    nz0 = layer._csr.row_nnz.clone()
    algo.update()
    assert torch.equal(layer._csr.row_nnz, nz0)
    layer._csr.assert_invariants()

    def run():
        lay = _layer(16, 16, 0.8, dev)
        a = SET(sparsity=0.8, drop_fraction=0.3, update_freq=1, seed=42)
        lay.apply(a)
        with torch.no_grad():
            lay._values.data.uniform_(-1, 1)
        a.update()
        return lay._csr.col_indices.cpu().numpy()

    np.testing.assert_array_equal(run(), run())


def test_set_training_loop_and_invariants(dev):
    layer = _layer(32, 16, 0.7, dev)
    algo = SET(sparsity=0.7, drop_fraction=0.4, update_freq=1, seed=0)
    layer.apply(algo)
    opt = torch.optim.SGD(layer.parameters(), lr=0.01)
    for _ in range(20):
        opt.zero_grad()
        layer(torch.randn(8, 32, device=dev)).sum().backward()
        opt.step()
        algo.step()
        layer._csr.assert_invariants()


def test_rigl_hooks_and_update(dev):
    layer = _layer(32, 16, 0.7, dev, bias=False)
    algo = RigL(sparsity=0.7, drop_fraction=0.3, update_freq=1, seed=42)
    layer.apply(algo)
    assert len(layer._forward_hooks) >= 1 and len(layer._backward_hooks) >= 1
    nnz = layer.nnz
    algo.update()  # nothing captured yet: no-op
    assert layer._csr.topology_version == 0
    x = torch.randn(8, 32, device=dev, requires_grad=True)
    y = layer(x)
    dy = torch.randn_like(y)
    y.backward(dy)
    assert id(layer) in algo._captured
    before = to_oracle(layer._csr)
    G = oracle.dense_grad(dy.detach().cpu().numpy().T.copy(), x.detach().cpu().numpy().T.copy())
    algo.update()
    assert id(layer) not in algo._captured
    assert layer.nnz == nnz
    want = oracle.drop_grow(before, max(1, int(0.3 * nnz)), "gradient", G)
    csr_arrays_equal(to_oracle(layer._csr), want, "RigL update")


def test_rigl_grows_at_high_gradient_positions(dev):
    """test_rigl.py:127-183 on the device."""
    layer = _layer(20, 1, 0.9, dev, bias=False)
    algo = RigL(sparsity=0.9, drop_fraction=0.5, update_freq=1, seed=0)
    layer.apply(algo)
    layer._csr.rewrite_row(0, np.array([0, 1], np.int32), np.array([0.01, 0.02], np.float32))
    X_fake = torch.zeros(1, 20)
    X_fake[0, 15] = 100.0
    X_fake[0, 12] = 50.0
    algo._captured[id(layer)] = {"X": X_fake, "dY": torch.ones(1, 1)}
    algo.update()
    c = to_oracle(layer._csr)
    cols = c.col_indices[c.row_start[0]:c.row_start[0] + c.row_nnz[0]].tolist()
    assert 15 in cols


def test_rigl_training_loop_invariants_and_seed(dev):
    def run():
        layer = _layer(16, 32, 0.8, dev, bias=False)
        algo = RigL(sparsity=0.8, drop_fraction=0.4, update_freq=1, seed=42)
        layer.apply(algo)
        opt = torch.optim.SGD(layer.parameters(), lr=0.01)
        torch.manual_seed(1)
        for _ in range(10):
            opt.zero_grad()
            x = torch.randn(4, 16, device=dev, requires_grad=True)
            layer(x).sum().backward()
            opt.step()
            algo.step()
            layer._csr.assert_invariants()
        return layer._csr.col_indices.cpu().numpy()

    np.testing.assert_array_equal(run(), run())


@pytest.mark.parametrize("algo_ctor", [
    lambda: SET(sparsity=0.8, drop_fraction=0.3, update_freq=2, seed=7),
    lambda: RigL(sparsity=0.8, drop_fraction=0.3, update_freq=2, seed=7)])
def test_loss_trajectory_cached_vs_fresh_transpose(dev, algo_ctor):
    """test_set_rigl_with_cache.py: the cached-transpose run and a run that
    clears the cache every step follow the same loss trajectory (here: bit
    for bit)."""
    def run(clear):
        torch.manual_seed(0)
        np.random.seed(0)
        model = nn.Sequential(SparseLinear(24, 32, sparsity=0.8), nn.ReLU(),
                              SparseLinear(32, 6, sparsity=0.8)).to(dev)
        algo = algo_ctor()
        model.apply(algo)
        opt = torch.optim.SGD(model.parameters(), lr=0.05)
        g = torch.Generator().manual_seed(1)
        losses = []
        for _ in range(30):
            x = torch.randn(16, 24, generator=g).to(dev)
            y = torch.randint(0, 6, (16,), generator=g).to(dev)
            opt.zero_grad()
            loss = F.cross_entropy(model(x), y)
            loss.backward()
            opt.step()
            algo.step()
            if clear:
                _clear_transpose_cache()
            losses.append(loss.item())
        return losses

    assert run(False) == run(True)
