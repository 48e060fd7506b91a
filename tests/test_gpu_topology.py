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


@pytest.mark.parametrize("nan_frac", [0.3, 0.97])
def test_rigl_never_grows_nan_columns_and_rows_shrink(dev, nan_frac):
    """G with NaN entries: no NaN column is grown (the reference's available
    count, router.py:704-705); a row short of growable columns shrinks, and the
    host's nnz, the row schedule and later kernels follow the new row_nnz."""
    for name, c in [("uniform", oracle.uniform_rows(64, 100, 10, seed=1, sigma=1.0)),
                    ("tall", oracle.zipf_rows(2500, 120, 0.05, 1.1, seed=8, sigma=1.0))]:
        print(f"[drop_grow NaN] {name} nan_frac={nan_frac}", flush=True)
        rng = np.random.default_rng(11)
        G = rng.standard_normal((c.nrows, c.ncols)).astype(np.float32)
        G[rng.random(G.shape) < nan_frac] = np.nan
        k = max(1, int(0.5 * c.nnz))
        want = oracle.drop_grow(c, k, "gradient", G)
        W = from_oracle(c, dev)
        W._view()
        W._drop_grow(k, _lib.SLK_GROW_GRADIENT, torch.from_numpy(G).to(dev))
        csr_arrays_equal(to_oracle(W), want, name)
        assert W.nnz == want.nnz
        if nan_frac > 0.9:
            assert want.nnz < c.nnz  # rows did shrink
        assert W._check_device() == ""
        X = np.random.default_rng(0).standard_normal((c.ncols, 64)).astype(np.float32)
        Y = ops._launch_spmm(W, torch.from_numpy(X).to(dev)).cpu().numpy()
        assert_bits_equal(Y, oracle.spmm(want, X), "Y after shrink")


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


def _cache_trajectory(dev, algo_ctor, n_steps, batch, clear_every_step, seed=42):
    """test_set_rigl_with_cache.py's training loop on the general path: two
    SparseLinear layers with more than 64 outputs (narrow layers keep no
    transpose cache) and an input that needs its gradient, so both layers'
    backward computes dX through _cached_transpose. Returns the losses and
    the topology versions seen."""
    torch.manual_seed(seed)
    np.random.seed(seed)
    l1 = SparseLinear(32, 96, sparsity=0.8, bias=False)
    l2 = SparseLinear(96, 80, sparsity=0.8, bias=False)
    model = nn.Sequential(l1, nn.ReLU(), l2).to(dev)
    algo = algo_ctor()
    model.apply(algo)
    opt = torch.optim.SGD(model.parameters(), lr=0.05)
    g = torch.Generator().manual_seed(seed + 1000)
    data_x = torch.randn(n_steps * batch, 32, generator=g).to(dev)
    data_y = torch.randn(n_steps * batch, 80, generator=g).to(dev)
    losses, versions = [], []
    for step in range(n_steps):
        if clear_every_step:
            _clear_transpose_cache()
        x = data_x[step * batch:(step + 1) * batch].clone().requires_grad_(True)
        y = data_y[step * batch:(step + 1) * batch]
        opt.zero_grad()
        loss = F.mse_loss(model(x), y)
        loss.backward()
        # both layers went through the transpose cache in this backward
        for layer in (l1, l2):
            entry = ops._transpose_cache.get(id(layer._csr))
            assert entry is not None and entry[0] == layer._csr.topology_version
        opt.step()
        algo.step()
        losses.append(loss.item())
        versions.append((l1._csr.topology_version, l2._csr.topology_version))
    return losses, versions


@pytest.mark.parametrize("algo_ctor,n_steps,batch", [
    (lambda: SET(sparsity=0.8, drop_fraction=0.3, update_freq=25, seed=123), 250, 16),
    (lambda: RigL(sparsity=0.8, drop_fraction=0.3, update_freq=25, seed=123), 250, 16),
    (lambda: SET(sparsity=0.7, drop_fraction=0.4, update_freq=5, seed=7), 100, 8)],
    ids=["set-250", "rigl-250", "set-aggressive-100"])
def test_loss_trajectory_cached_vs_fresh_transpose(dev, algo_ctor, n_steps, batch):
    """test_set_rigl_with_cache.py:109-236 on the general path: the run that
    keeps the transpose cache and a run that clears it before every step
    follow the same loss trajectory, here bit for bit, across every SET / RigL
    rewrite (each bumps topology_version and must invalidate the entry)."""
    print(f"[cache trajectory] {n_steps} steps batch {batch}", flush=True)
    _clear_transpose_cache()
    cached, v_cached = _cache_trajectory(dev, algo_ctor, n_steps, batch, False)
    _clear_transpose_cache()
    fresh, v_fresh = _cache_trajectory(dev, algo_ctor, n_steps, batch, True)
    assert v_cached == v_fresh
    assert len(set(v_cached)) > 3  # the topology did change, several times
    diverged = [i for i, (a, b) in enumerate(zip(cached, fresh)) if a != b]
    assert not diverged, f"cached and fresh trajectories differ from step {diverged[0]}"
    assert sum(cached[-10:]) / 10 < sum(cached[:10]) / 10  # training happened


# ─────────────────── RigL from the certified approximate gradient ──────────

def _rigl_inputs(M, K, N, seed, kind="normal"):
    rng = np.random.default_rng(seed)
    dY = rng.standard_normal((M, N)).astype(np.float32)
    X = rng.standard_normal((K, N)).astype(np.float32)
    if kind == "ties":  # small integers: many exactly equal |G|, exact G' parts
        dY = rng.integers(-2, 3, (M, N)).astype(np.float32)
        X = rng.integers(-2, 3, (K, N)).astype(np.float32)
    elif kind == "scaled":  # rows and columns over many orders of magnitude
        dY *= (10.0 ** rng.integers(-15, 15, (M, 1))).astype(np.float32)
        X *= (10.0 ** rng.integers(-15, 15, (K, 1))).astype(np.float32)
    elif kind == "nonfinite-rows":  # exact rows: every empty column computed exactly
        dY[1, 3] = np.nan   # the whole G row is NaN: nothing growable, the row shrinks
        dY[4, 0] = np.inf   # |G| = inf (NaN where X[k, 0] = 0)
        dY[6, :] *= 1e30    # a norm beyond the certified range
    elif kind == "nonfinite-cols":  # a NaN column leaves no row certifiable
        X[2, 5] = np.nan
        X[7, 1] = -np.inf
    elif kind == "cancel":
        # partial sums climb to ~|a_i|·N/2 and cancel back down: dY_i = a_i on
        # the first half of j and -a_i on the second, X_k = 1 + noise/2, so
        # |G| ~ |a_i|·sqrt(N)/2 while the running sums peak 2^5 x higher and
        # the bound's c2·pm term outweighs its c1·n_i·n_k term
        a = rng.standard_normal((M, 1)).astype(np.float32)
        sign = np.where(np.arange(N) < N // 2, 1.0, -1.0).astype(np.float32)
        dY = a * sign[None, :]
        X = (1.0 + 0.5 * rng.standard_normal((K, N))).astype(np.float32)
    return dY, X


@pytest.mark.parametrize("M,K,N,kind", [
    (256, 384, 4096, "normal"), (130, 257, 1000, "normal"), (64, 64, 7, "normal"),
    (300, 200, 513, "scaled"), (128, 128, 1, "normal"), (200, 300, 96, "ties"),
    (192, 320, 4096, "cancel")])
def test_dense_grad_approx_within_certified_bound(dev, M, K, N, kind):
    """|G' - G| <= c1·n_i·n_k + c2·2^(code - 127) + 2^-100·(1 + n_i + n_k) for
    every element, G the reference-arithmetic dense gradient (itself pinned to
    the reference build); the norms bound the true row norms, and each code
    bounds the element's sum of |partial sums| at the 128-term chunk ends
    (checked against float64 partial sums)."""
    print(f"[rigl bound] {M}x{K} N={N} {kind}", flush=True)
    dY_np, X_np = _rigl_inputs(M, K, N, M + K + N, kind)
    dY, X = torch.from_numpy(dY_np).to(dev), torch.from_numpy(X_np).to(dev)
    nd = torch.empty(M, device=dev)
    nx = torch.empty(K, device=dev)
    _lib.rigl_norms(dY, X, nd, nx)
    nd64 = np.linalg.norm(dY_np.astype(np.float64), axis=1)
    nx64 = np.linalg.norm(X_np.astype(np.float64), axis=1)
    assert np.all(nd.cpu().numpy().astype(np.float64) >= nd64)
    assert np.all(nx.cpu().numpy().astype(np.float64) >= nx64)
    Gp = torch.empty(M, K, device=dev)
    Gc = torch.empty(M, K, dtype=torch.uint8, device=dev)
    _lib.dense_grad_approx(dY, X, Gp, Gc)
    G = ops.dense_grad(dY, X).cpu().numpy().astype(np.float64)
    c1, c2 = _lib.rigl_bound_factor(N), _lib.rigl_partial_factor(N)
    code = Gc.cpu().numpy().astype(np.float64)
    assert np.all((code >= 1) & (code <= 255))
    pbound = np.exp2(code - 127.0)
    # the codes bound the exact partial sums' magnitudes, up to the
    # approximation's own error (C·c_approx·n_i·n_k, c_approx < 1e-4, which the
    # bound's c1 carries)
    x64, y64 = dY_np.astype(np.float64), X_np.astype(np.float64)
    if np.all(np.isfinite(x64)) and np.all(np.isfinite(y64)) and np.max(np.abs(x64)) < 1e15:
        pm = np.zeros((M, K))
        for j0 in range(0, N, 128):
            part = x64[:, :min(N, j0 + 128)] @ y64[:, :min(N, j0 + 128)].T
            pm += np.abs(part)
        nn = (np.linalg.norm(x64, axis=1)[:, None] * np.linalg.norm(y64, axis=1)[None, :])
        slack = -(-N // 128) * 1e-4 * nn + 2.0 ** -90
        assert np.all(pm <= pbound * (1 + 1e-5) + slack), float(np.max(pm / (pbound + slack)))
    E = (c1 * nd.cpu().numpy().astype(np.float64)[:, None] * nx.cpu().numpy().astype(np.float64)[None, :]
         + c2 * pbound + 2.0 ** -100 * (1 + nd.cpu().numpy()[:, None] + nx.cpu().numpy()[None, :]))
    err = np.abs(Gp.cpu().numpy().astype(np.float64) - G)
    assert np.all(err <= E), float(np.max(err / E))
    # the bound is a bound, not noise: the approximation is far inside it
    assert float(np.max(err / E)) < 0.5
    if kind == "cancel":
        # the partial-sum term decides the bound here: it is the larger term
        # for nearly every element, and |G| sits far below the running sums
        nn_b = c1 * nd.cpu().numpy().astype(np.float64)[:, None] * \
            nx.cpu().numpy().astype(np.float64)[None, :]
        assert np.mean(c2 * pbound > nn_b) > 0.95
        assert np.median(pm / (-(-N // 128)) / np.maximum(np.abs(G), 1e-30)) > 8


@pytest.mark.parametrize("M,K,N,kind", [
    (256, 384, 4096, "normal"), (130, 257, 1000, "normal"), (300, 200, 513, "scaled"),
    (64, 64, 7, "normal"), (520, 136, 260, "ties"), (1, 1, 1, "normal"),
    (192, 320, 4096, "cancel")])
def test_dense_grad_approx_tilings_agree(dev, tune, M, K, N, kind):
    """The 256 x 128 direct-load kernel and the 128 x 128 register-staged one
    run each element's matrix-core sequence in the same order: identical G'
    and codes, bit for bit (partial tiles, N not a multiple of the stage)."""
    print(f"[G' tilings] {M}x{K} N={N} {kind}", flush=True)
    dY_np, X_np = _rigl_inputs(M, K, N, M * 3 + K + N, kind)
    dY, X = torch.from_numpy(dY_np).to(dev), torch.from_numpy(X_np).to(dev)
    out = []
    for tile in (None, 128):
        tune(rigl_tile=tile)
        Gp = torch.full((M, K), float("nan"), device=dev)
        Gc = torch.zeros(M, K, dtype=torch.uint8, device=dev)
        _lib.dense_grad_approx(dY, X, Gp, Gc)
        out.append((Gp.cpu().numpy(), Gc.cpu().numpy()))
    assert_bits_equal(out[0][0], out[1][0], "G'")
    assert_bits_equal(out[0][1], out[1][1], "G' codes")


def _rigl_case(name):
    if name == "uniform":
        return oracle.uniform_rows(96, 300, 40, seed=31, sigma=1.0), 512, "normal"
    if name == "zipf":
        return oracle.zipf_rows(400, 700, 0.06, 1.1, seed=32, sigma=1.0), 1024, "normal"
    if name == "ties":
        return oracle.uniform_rows(64, 200, 30, seed=33, sigma=1.0), 96, "ties"
    if name == "scaled":
        return oracle.uniform_rows(80, 260, 50, seed=34, sigma=1.0), 513, "scaled"
    if name == "nonfinite-rows":
        return oracle.uniform_rows(200, 90, 20, seed=35, sigma=1.0), 64, "nonfinite-rows"
    if name == "nonfinite-cols":
        return oracle.uniform_rows(40, 90, 20, seed=39, sigma=1.0), 64, "nonfinite-cols"
    if name == "n-odd":
        return oracle.zipf_rows(150, 129, 0.2, 1.1, seed=36, sigma=1.0), 37, "normal"
    if name == "cancel":
        return oracle.uniform_rows(96, 300, 40, seed=41, sigma=1.0), 4096, "cancel"
    if name == "dense-rows":
        W = np.random.default_rng(37).standard_normal((30, 50)).astype(np.float32)
        W[::3, :] *= (np.random.default_rng(38).random((10, 50)) < 0.1)  # some sparse rows
        return oracle.from_dense(W), 256, "normal"
    # ncols % 16 == 0: the count kernel that holds a row in registers and
    # lists the columns itself (4, 8 and 16 registers of keys per thread)
    if name == "uniform-k16":
        return oracle.uniform_rows(96, 320, 40, seed=51, sigma=1.0), 512, "normal"
    if name == "zipf-k16":
        return oracle.zipf_rows(400, 704, 0.06, 1.1, seed=52, sigma=1.0), 1024, "normal"
    if name == "ties-k16":
        return oracle.uniform_rows(64, 208, 30, seed=53, sigma=1.0), 96, "ties"
    if name == "nonfinite-rows-k16":
        return oracle.uniform_rows(200, 96, 20, seed=54, sigma=1.0), 64, "nonfinite-rows"
    if name == "nonfinite-cols-k16":
        return oracle.uniform_rows(40, 96, 20, seed=55, sigma=1.0), 64, "nonfinite-cols"
    if name == "cancel-k16":
        return oracle.uniform_rows(96, 320, 40, seed=56, sigma=1.0), 4096, "cancel"
    if name == "wide-u8":
        return oracle.zipf_rows(48, 6144, 0.05, 1.1, seed=57, sigma=1.0), 64, "normal"
    if name == "wide-u16":
        return oracle.uniform_rows(32, 12288, 600, seed=58, sigma=1.0), 48, "normal"
    raise KeyError(name)


@pytest.mark.parametrize("df", [0.3, 0.9])
@pytest.mark.parametrize("name", ["uniform", "zipf", "ties", "scaled", "nonfinite-rows",
                                  "nonfinite-cols", "n-odd", "dense-rows", "cancel",
                                  "uniform-k16", "zipf-k16", "ties-k16", "nonfinite-rows-k16",
                                  "nonfinite-cols-k16", "cancel-k16", "wide-u8", "wide-u16"])
def test_rigl_certified_matches_exact_drop_grow(dev, name, df):
    """The certified path (matrix-core G', exact G only where the bound cannot
    decide) rewrites every row exactly as the exact-G drop/grow does, and as
    the oracle's RigL rule does with the oracle's G."""
    c, N, kind = _rigl_case(name)
    print(f"[rigl certified] {name} df={df} {c.nrows}x{c.ncols} N={N}", flush=True)
    dY_np, X_np = _rigl_inputs(c.nrows, c.ncols, N, 40 + c.nrows, kind)
    dY, X = torch.from_numpy(dY_np).to(dev), torch.from_numpy(X_np).to(dev)
    k = max(1, int(df * c.nnz))
    W_exact, W_cert = from_oracle(c, dev), from_oracle(c, dev)
    W_exact._drop_grow(k, _lib.SLK_GROW_GRADIENT, ops.dense_grad(dY, X))
    W_cert._rigl_update(k, dY, X)
    csr_arrays_equal(to_oracle(W_cert), to_oracle(W_exact), f"{name} certified vs exact")
    assert W_cert.nnz == W_exact.nnz and W_cert.topology_version == 1
    want = oracle.drop_grow(c, k, "gradient", oracle.dense_grad(dY_np, X_np))
    csr_arrays_equal(to_oracle(W_cert), want, f"{name} certified vs oracle")
    if name.startswith("nonfinite-rows"):
        assert want.nnz < c.nnz  # the NaN row shrank
    if name.startswith("cancel"):
        # the certified path decided this case (not the exact fallback), with
        # undecided columns left for the exact finish
        W = from_oracle(c, dev)
        view = W._view()
        thr = torch.empty(1, device=dev)
        _lib.live_abs_kth(view, k, torch.empty(_lib.SLK_KTH_WORKSPACE_BYTES, dtype=torch.uint8,
                                               device=dev), thr)
        nd, nx = torch.empty(c.nrows, device=dev), torch.empty(c.ncols, device=dev)
        _lib.rigl_norms(dY, X, nd, nx)
        Gp = torch.empty(c.nrows, c.ncols, device=dev)
        Gc = torch.empty(c.nrows, c.ncols, dtype=torch.uint8, device=dev)
        _lib.dense_grad_approx(dY, X, Gp, Gc)
        info = torch.empty(c.nrows * _lib.RIGL_INFO_BYTES, dtype=torch.uint8, device=dev)
        off = torch.empty(2 * c.nrows + 1, dtype=torch.int64, device=dev)
        total = torch.empty(1, dtype=torch.int64, device=dev)
        amb = torch.empty(8 * c.nrows * c.ncols, dtype=torch.uint8, device=dev)
        stage = torch.empty(_lib.drop_grow_workspace_bytes(view), dtype=torch.uint8, device=dev)
        _lib.rigl_count(view, thr, Gp, Gc, nd, nx, N, info, off, total, amb, stage)
        n_amb = int(total.item())
        assert 0 < n_amb <= W._RIGL_EXACT_SHARE * (c.nrows * c.ncols - c.nnz), n_amb


@pytest.mark.parametrize("name", ["cancel", "cancel-k16", "ties", "zipf-k16"])
def test_rigl_list_overflow_rewrites_no_row_and_takes_the_exact_path(dev, name):
    """The finish is queued before the undecided count is read. With lists too
    small for the count (a capacity of one pair here), its row rewrite leaves
    every row alone, and the exact-G drop/grow the host then runs gives the
    exact path's rows."""
    c, N, kind = _rigl_case(name)
    print(f"[rigl overflow] {name} {c.nrows}x{c.ncols} N={N}", flush=True)
    dY_np, X_np = _rigl_inputs(c.nrows, c.ncols, N, 40 + c.nrows, kind)
    dY, X = torch.from_numpy(dY_np).to(dev), torch.from_numpy(X_np).to(dev)
    k = max(1, int(0.3 * c.nnz))
    W_exact, W_cert = from_oracle(c, dev), from_oracle(c, dev)
    W_exact._drop_grow(k, _lib.SLK_GROW_GRADIENT, ops.dense_grad(dY, X))
    W_cert._RIGL_EXACT_SHARE = 1e-30  # lists of one pair: every case here has more
    took_exact = []
    inner = W_cert._drop_grow
    W_cert._drop_grow = lambda *a: (took_exact.append(1), inner(*a))[1]
    W_cert._rigl_update(k, dY, X)
    assert took_exact, "the count fit the one-pair lists: the case does not test the overflow"
    csr_arrays_equal(to_oracle(W_cert), to_oracle(W_exact), f"{name} overflow vs exact")
    assert W_cert.nnz == W_exact.nnz and W_cert.topology_version == 1


@pytest.mark.parametrize("name,share", [("zipf-k16", None), ("nonfinite-rows-k16", None),
                                        ("nonfinite-rows", None), ("cancel-k16", 1e-30)])
def test_rigl_update_with_cached_rebuild_matches_separate_calls(dev, name, share):
    """ops._rigl_update_cached (the rebuild queued behind the rewrite, one host
    read) leaves W and its cached transpose exactly as _rigl_update followed
    by _cached_transpose: rows that shrink (NaN rows), and the exact path taken
    when the undecided lists overflow."""
    c, N, kind = _rigl_case(name)
    print(f"[rigl+rebuild] {name} share={share}", flush=True)
    dY_np, X_np = _rigl_inputs(c.nrows, c.ncols, N, 40 + c.nrows, kind)
    dY, X = torch.from_numpy(dY_np).to(dev), torch.from_numpy(X_np).to(dev)
    k = max(1, int(0.3 * c.nnz))
    A, B = from_oracle(c, dev), from_oracle(c, dev)
    for W in (A, B):
        if share is not None:
            W._RIGL_EXACT_SHARE = share
        ops._cached_transpose(W)
    A._rigl_update(k, dY, X)
    WT_a = ops._cached_transpose(A)
    ops._rigl_update_cached(B, k, dY, X)
    entry = ops._transpose_cache[id(B)]
    assert entry[0] == B.topology_version == A.topology_version
    WT_b = ops._cached_transpose(B)  # a hit: the entry the merged call stored
    assert WT_b is entry[2]
    csr_arrays_equal(to_oracle(B), to_oracle(A), f"{name} W")
    assert B.nnz == A.nnz and WT_b.nnz == WT_a.nnz == A.nnz
    csr_arrays_equal(to_oracle(WT_b), to_oracle(WT_a), f"{name} WT")
    assert torch.equal(entry[3], ops._transpose_cache[id(A)][3])
    assert WT_b._view().n_heavy_rows == WT_a._view().n_heavy_rows
    if name.startswith("nonfinite-rows"):
        assert A.nnz < c.nnz  # rows shrank


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (finite inputs)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return b.astype(np.uint16)


def _bf16_value(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def test_rigl_mfma_accumulation_model(dev):
    """The matrix-core instruction the certified RigL bound models
    (v_mfma_f32_32x32x16_bf16, run by slk_rigl_mfma_probe with the operand
    layout of slk_dense_grad_approx): D = C + sum of 16 exact bf16 products.
    Small integers (every sum exact) must come out exact, which pins the lane
    layout; on random, wide-range, cancelling and tie-breaking operands the
    error against the exact sum stays within gamma_16(2u)·(|C| + sum|a b|),
    the per-step allowance the bound's c1 and c2 are built on."""
    rng = np.random.default_rng(2024)
    n_per = 16
    cases = []
    # exact: small integers
    A = rng.integers(-3, 4, (n_per, 32, 16)).astype(np.float32)
    B = rng.integers(-3, 4, (n_per, 32, 16)).astype(np.float32)
    C = rng.integers(-50, 51, (n_per, 32, 32)).astype(np.float32)
    cases.append(("integers", A, B, C, True))
    # random normal operands, accumulators over several magnitudes
    A = rng.standard_normal((n_per, 32, 16)).astype(np.float32)
    B = rng.standard_normal((n_per, 32, 16)).astype(np.float32)
    C = (rng.standard_normal((n_per, 32, 32)) * 10.0 ** rng.integers(-3, 4, (n_per, 32, 32))
         ).astype(np.float32)
    cases.append(("normal", A, B, C, False))
    # products over 2^-20 .. 2^20 against a unit accumulator
    A = (rng.standard_normal((n_per, 32, 16)) * 2.0 ** rng.integers(-10, 11, (n_per, 32, 16))
         ).astype(np.float32)
    B = (rng.standard_normal((n_per, 32, 16)) * 2.0 ** rng.integers(-10, 11, (n_per, 32, 16))
         ).astype(np.float32)
    C = rng.standard_normal((n_per, 32, 32)).astype(np.float32)
    cases.append(("wide", A, B, C, False))
    # cancellation: C = -(the products' sum)·(1 + tiny)
    A = rng.standard_normal((n_per, 32, 16)).astype(np.float32)
    B = rng.standard_normal((n_per, 32, 16)).astype(np.float32)
    Av, Bv = _bf16_value(_bf16_bits(A)), _bf16_value(_bf16_bits(B))
    S = np.einsum("tik,tjk->tij", Av.astype(np.float64), Bv.astype(np.float64))
    C = (-S * (1 + 1e-6 * rng.standard_normal(S.shape))).astype(np.float32)
    cases.append(("cancel", A, B, C, False))
    # ties: 1 + 2^-24 exactly halfway between two floats, and 1 + 3·2^-25
    A = np.zeros((n_per, 32, 16), np.float32)
    B = np.zeros((n_per, 32, 16), np.float32)
    A[:, :, 0] = 2.0 ** -12
    B[:, :, 0] = 2.0 ** -12
    A[:, ::2, 1] = 2.0 ** -13
    B[:, :, 1] = 2.0 ** -12
    C = np.ones((n_per, 32, 32), np.float32)
    cases.append(("ties", A, B, C, False))

    u = 2.0 ** -24
    gamma = 16 * 2 * u / (1 - 16 * 2 * u)
    worst = 0.0
    for name, A, B, C, exact in cases:
        Ab, Bb = _bf16_bits(A), _bf16_bits(B)
        Av = _bf16_value(Ab).astype(np.float64)
        Bv = _bf16_value(Bb).astype(np.float64)
        P = Av[:, :, None, :] * Bv[:, None, :, :]          # t, i, j, k: exact products
        want = C.astype(np.float64) + P.sum(axis=3)
        mag = np.abs(C.astype(np.float64)) + np.abs(P).sum(axis=3)
        D = torch.empty(C.shape, device=dev)
        _lib.rigl_mfma_probe(torch.from_numpy(Ab.view(np.int16)).to(dev),
                             torch.from_numpy(Bb.view(np.int16)).to(dev),
                             torch.from_numpy(C).to(dev), D)
        got = D.cpu().numpy().astype(np.float64)
        err = np.abs(got - want)
        print(f"[mfma probe] {name}: max err / (u·mag) = {float(np.max(err / (u * mag))):.3f}",
              flush=True)
        if exact:
            assert_bits_equal(got.astype(np.float32), want.astype(np.float32), f"{name} exact")
        assert np.all(err <= gamma * mag + 2.0 ** -126), name
        worst = max(worst, float(np.max(err / (u * mag))))
    assert worst <= 32.0
