"""GPU parity at the benchmark workloads' full sizes, through the default
launchers (no schedule or kernel forced).

The launchers choose their kernels and schedules from the problem shape, so
the choices these sizes make are only reached here: the LDS-staged SpMM with
its heavy-row split at 16384 rows, the 4-phase gather sweep, the 128- and
64-column segment dW kernels, the device transpose of 13.4M slots, the RigL
drop/grow at 16384 columns and the dense gradient at 16384 x 16384 x 4096.

Layers:
  C3  10M char GPT, N = 8192 tokens: QKV 1152x384 and O 384x384 at 70%,
      FFN up 1536x384 and down 384x1536 at 90% (uniform-random masks)
  C4  60M mini-GPT, N = 8192: QKV 2304x768, O 768x768 at 70%, up 3072x768,
      down 768x3072 at 90%, plus one SET rewrite and the rebuilt transpose
  C5  16384 x 16384, Zipf(1.1) rows at 95% and 99%, N = 4096, plus one RigL
      rewrite (G = dY·Xᵀ) and the rebuilt transpose

Oracle on samples: Y and dW on 48 rows that include the 8 longest and the 8
shortest rows; dX on 48 columns chosen the same way (rows of the transpose);
the full transpose (every WT array and perm); the topology update on sampled
rows given the device's threshold (itself checked against the oracle's).
Bar: bit-exact, as everywhere else on this path.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from helpers import assert_bits_equal, csr_arrays_equal, from_oracle, to_oracle
from sparsecore_amd import _lib, ops

pytestmark = pytest.mark.gpu

N_SAMPLE = 48


def _sample(nnz: np.ndarray, seed: int) -> np.ndarray:
    """8 longest, 8 shortest and 32 seeded random rows (distinct)."""
    order = np.argsort(nnz, kind="stable")
    picked = list(order[-8:]) + list(order[:8])
    rng = np.random.default_rng(seed)
    rest = np.setdiff1d(np.arange(nnz.size), picked)
    picked += list(rng.choice(rest, size=min(N_SAMPLE - 16, rest.size), replace=False))
    return np.array(sorted(set(int(r) for r in picked)), dtype=np.int64)


def _layer_parity(name, W, X, dY, seed):
    """Forward, dW and dX of one layer through ops' default launchers, checked
    on sampled rows / columns; the transpose checked in full. Returns the
    oracle copy of W (host)."""
    print(f"[config {name}] {W.nrows}x{W.ncols} nnz={W.nnz} N={X.shape[1]}", flush=True)
    Y = ops._launch_spmm(W, X)
    dW = ops._launch_sddmm(W, dY, X, "simd")
    WT = ops._cached_transpose(W)
    dX = ops._launch_spmm(WT, dY)
    torch.cuda.synchronize()

    c = to_oracle(W)
    rows = _sample(c.row_nnz, seed)
    sub, src = oracle.sub_rows(c, rows)
    X_h = X.cpu().numpy()
    dY_rows = dY[torch.from_numpy(rows).to(dY.device)].cpu().numpy()
    assert_bits_equal(Y[torch.from_numpy(rows).to(Y.device)].cpu().numpy(),
                      oracle.spmm(sub, X_h), f"{name}: Y on sampled rows")
    assert_bits_equal(dW.cpu().numpy()[src], oracle.sddmm(sub, dY_rows, X_h),
                      f"{name}: dW on sampled rows")
    del X_h

    WT_o, perm_o = oracle.transpose_with_perm(c)
    csr_arrays_equal(to_oracle(WT), WT_o, f"{name}: WT")
    perm = ops._transpose_cache[id(W)][3]
    assert_bits_equal(perm.cpu().numpy(), perm_o, f"{name}: perm")
    cols = _sample(WT_o.row_nnz, seed + 1)
    subT, _ = oracle.sub_rows(WT_o, cols)
    assert_bits_equal(dX[torch.from_numpy(cols).to(dX.device)].cpu().numpy(),
                      oracle.spmm(subT, dY.cpu().numpy()), f"{name}: dX on sampled columns")
    return c


def _uniform_layer(M, K, sparsity, seed, dev):
    c = oracle.bernoulli(M, K, sparsity, seed=seed, scale=0.05)
    return from_oracle(c, dev)


def _dense_inputs(M, K, N, seed, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randn(K, N, generator=g, device=dev), torch.randn(M, N, generator=g, device=dev)


# ───────────────────────────── C3, C4 ───────────────────────────────────

C3_LAYERS = [("qkv", 1152, 384, 0.7), ("o", 384, 384, 0.7), ("up", 1536, 384, 0.9),
             ("down", 384, 1536, 0.9)]
C4_LAYERS = [("qkv", 2304, 768, 0.7), ("o", 768, 768, 0.7), ("up", 3072, 768, 0.9),
             ("down", 768, 3072, 0.9)]


@pytest.mark.parametrize("cfg,layer", [("c3", l) for l in C3_LAYERS] +
                         [("c4", l) for l in C4_LAYERS], ids=lambda v: v if isinstance(v, str)
                         else v[0])
def test_gpt_layer_at_full_size(dev, cfg, layer):
    tag, M, K, sp = layer
    seed = (3 if cfg == "c3" else 4) * 100 + [l[0] for l in C3_LAYERS].index(tag)
    W = _uniform_layer(M, K, sp, seed, dev)
    X, dY = _dense_inputs(M, K, 8192, seed + 1, dev)
    _layer_parity(f"{cfg} {tag}", W, X, dY, seed)


def test_c4_sparse_linear_step_and_set_rewrite(dev):
    """The C4 FFN-up layer as a SparseLinear with bias at N = 8192 (token-major
    input, fused bias in the forward store and in the dW launch, library
    transposes), then one SET rewrite on the device and the rebuilt
    transpose."""
    import sparsecore_amd as slk

    torch.manual_seed(3)
    layer = slk.SparseLinear(768, 3072, sparsity=0.9).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    x = torch.randn(8192, 768, generator=g, device=dev, requires_grad=True)
    up = torch.randn(8192, 3072, generator=g, device=dev)
    y = layer(x)
    y.backward(up)
    torch.cuda.synchronize()
    W = layer._csr
    c = to_oracle(W)
    rows = _sample(c.row_nnz, 5)
    sub, src = oracle.sub_rows(c, rows)
    X_h = x.detach().t().contiguous().cpu().numpy()
    dY_rows = up.t()[torch.from_numpy(rows).to(dev)].contiguous().cpu().numpy()
    b = layer.bias.detach().cpu().numpy()
    print("[config c4 SparseLinear] y, dW, dbias, dx", flush=True)
    assert_bits_equal(y.detach().t()[torch.from_numpy(rows).to(dev)].cpu().numpy(),
                      oracle.spmm(sub, X_h) + b[rows][:, None], "y on sampled rows")
    assert_bits_equal(layer._values.grad.cpu().numpy()[src], oracle.sddmm(sub, dY_rows, X_h),
                      "dW on sampled rows")
    WT_o, _ = oracle.transpose_with_perm(c)
    cols = _sample(WT_o.row_nnz, 6)
    subT, _ = oracle.sub_rows(WT_o, cols)
    dx_cols = x.grad.t()[torch.from_numpy(cols).to(dev)].cpu().numpy()
    assert_bits_equal(dx_cols, oracle.spmm(subT, up.t().contiguous().cpu().numpy()),
                      "dx on sampled columns")
    db = layer.bias.grad.cpu().numpy()
    np.testing.assert_allclose(db, up.sum(0).cpu().numpy(), rtol=1e-4, atol=1e-3)

    # one SET rewrite (the C4 step's topology update), then the rebuilt WT
    k = max(1, int(0.3 * W.nnz))
    dev_thr = torch.empty(1, device=dev)
    _lib.live_abs_kth(W._view(), k,
                      torch.empty(_lib.SLK_KTH_WORKSPACE_BYTES, dtype=torch.uint8, device=dev),
                      dev_thr)
    thr = dev_thr.cpu().numpy()[0]
    assert thr.view(np.uint32) == np.float32(oracle.live_abs_kth(c, k)).view(np.uint32)
    print("[config c4 SparseLinear] SET rewrite", flush=True)
    W._drop_grow(k, _lib.SLK_GROW_RANDOM, None, 77)
    after = to_oracle(W)
    for r in rows:
        s, n = int(c.row_start[r]), int(c.row_nnz[r])
        wc, wv = oracle.drop_grow_row(c.col_indices[s:s + n], c.values[s:s + n], thr, "random",
                                      c.ncols, seed=77, row=int(r))
        m = int(after.row_nnz[r])
        assert m == wc.size, r
        assert_bits_equal(after.col_indices[s:s + m], wc, f"SET cols row {r}")
        assert_bits_equal(after.values[s:s + m], wv, f"SET vals row {r}")
    WT = ops._cached_transpose(W)
    WT_o2, perm_o2 = oracle.transpose_with_perm(after)
    csr_arrays_equal(to_oracle(WT), WT_o2, "WT after SET")
    assert_bits_equal(ops._transpose_cache[id(W)][3].cpu().numpy(), perm_o2, "perm after SET")


def _device_copy(W):
    """A device copy of W's arrays (no host round trip, no re-validation)."""
    from sparsecore_amd import PaddedCSR

    return PaddedCSR._from_parts(W.nrows, W.ncols, W.values.detach().clone(),
                                 W.col_indices.clone(), W.row_start.clone(), W.row_nnz.clone(),
                                 W.row_capacity.clone(), W.nnz, W.topology_version)


def _device_rows_equal(A, B, what):
    """Every row of two device PaddedCSRs: the same row_nnz, and the same
    column and value bits over each row's capacity (live slots and padding)."""
    assert A.nnz == B.nnz, what
    for name in ("row_nnz", "row_start", "row_capacity", "col_indices"):
        a, b = getattr(A, name), getattr(B, name)
        bad = torch.nonzero(a != b)
        assert bad.numel() == 0, f"{what}: {name} differs at {bad[:8].flatten().tolist()}"
    va, vb = A.values.detach().view(torch.int32), B.values.detach().view(torch.int32)
    bad = torch.nonzero(va != vb)
    assert bad.numel() == 0, f"{what}: value bits differ at slots {bad[:8].flatten().tolist()}"


def test_c4_ffn_rigl_certified_every_row(dev):
    """The C4 FFN-up layer (3072 x 768 at 90%, N = 8192) through one RigL
    update: the certified path (matrix-core G', exact G only where undecided)
    rewrites every row exactly as the exact-G drop/grow does; the exact path is
    checked against the oracle's row rule on sampled rows."""
    W = _uniform_layer(3072, 768, 0.9, 405, dev)
    X, dY = _dense_inputs(3072, 768, 8192, 406, dev)
    c = to_oracle(W)
    W_exact = _device_copy(W)
    k = max(1, int(0.3 * W.nnz))
    print("[config c4 RigL] certified update", flush=True)
    W._rigl_update(k, dY, X)
    G = ops.dense_grad(dY, X)
    W_exact._drop_grow(k, _lib.SLK_GROW_GRADIENT, G)
    _device_rows_equal(W, W_exact, "c4 ffn certified vs exact, every row")
    thr = np.float32(oracle.live_abs_kth(c, k))
    after = to_oracle(W_exact)
    rows = _sample(c.row_nnz, 7)
    G_rows = G[torch.from_numpy(rows).to(dev)].cpu().numpy()
    for r, g_row in zip(rows, G_rows):
        s, n = int(c.row_start[r]), int(c.row_nnz[r])
        wc, wv = oracle.drop_grow_row(c.col_indices[s:s + n], c.values[s:s + n], thr, "gradient",
                                      c.ncols, g_row, row=int(r))
        m = int(after.row_nnz[r])
        assert m == wc.size, r
        assert_bits_equal(after.col_indices[s:s + m], wc, f"exact RigL cols row {r}")
        assert_bits_equal(after.values[s:s + m], wv, f"exact RigL vals row {r}")


# ───────────────────────────── C5 ───────────────────────────────────────

@pytest.fixture(scope="module")
def c5_layers(dev):
    """Builds each C5 matrix once per module (13.4M / 2.7M live slots)."""
    import bench

    cache = {}

    def get(density):
        if density not in cache:
            counts = bench.zipf_row_counts(16384, 16384, density, 1.1, 0)
            W = bench.device_rows_csr(counts, 16384, 0.01, 1, dev)
            X, dY = _dense_inputs(16384, 16384, 4096, 2, dev)
            cache.clear()  # one C5 layer resident at a time
            torch.cuda.empty_cache()
            cache[density] = (W, X, dY)
        return cache[density]

    yield get
    cache.clear()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("density", [0.05, 0.01], ids=["95", "99"])
def test_c5_layer_at_full_size(dev, c5_layers, density):
    W, X, dY = c5_layers(density)
    assert W.nnz == int(round(density * 16384 * 16384))
    _layer_parity(f"c5-{int(round(100 * (1 - density)))}", W, X, dY, 9)


@pytest.mark.parametrize("density", [0.05, 0.01], ids=["95", "99"])
def test_c5_rigl_rewrite_at_full_size(dev, c5_layers, density):
    """One RigL step of the C5 workload as bench.py runs it: the exact G = dY·Xᵀ
    (checked on 4 sampled rows against the oracle), the global threshold
    (checked exactly), the certified RigL update (matrix-core G', exact G
    where undecided; checked on sampled rows against the oracle's row rule
    with the exact G row),
    then the rebuilt transpose (checked in full) and the forward on the new
    topology (sampled rows)."""
    W, X, dY = c5_layers(density)
    c = to_oracle(W)
    W_exact = _device_copy(W)  # the exact-G drop/grow, pinned to the oracle below
    print(f"[config c5 RigL] density={density} dense_grad", flush=True)
    G = ops.dense_grad(dY, X)
    torch.cuda.synchronize()
    g_rows = _sample(c.row_nnz, 12)[:4]
    X_h = X.cpu().numpy()
    assert_bits_equal(G[torch.from_numpy(g_rows).to(dev)].cpu().numpy(),
                      oracle.dense_grad(dY[torch.from_numpy(g_rows).to(dev)].cpu().numpy(), X_h),
                      "G on sampled rows")
    k = max(1, int(0.3 * W.nnz))
    thr_dev = torch.empty(1, device=dev)
    _lib.live_abs_kth(W._view(), k,
                      torch.empty(_lib.SLK_KTH_WORKSPACE_BYTES, dtype=torch.uint8, device=dev),
                      thr_dev)
    thr = thr_dev.cpu().numpy()[0]
    assert thr.view(np.uint32) == np.float32(oracle.live_abs_kth(c, k)).view(np.uint32)
    print(f"[config c5 RigL] density={density} certified RigL update", flush=True)
    W._rigl_update(k, dY, X)
    # every row: the certified update against the exact-G drop/grow on a copy
    print(f"[config c5 RigL] density={density} every row against exact G", flush=True)
    W_exact._drop_grow(k, _lib.SLK_GROW_GRADIENT, G)
    _device_rows_equal(W, W_exact, f"c5 {density} certified vs exact, every row")
    del W_exact
    after = to_oracle(W)
    rows = _sample(c.row_nnz, 13)
    G_rows = G[torch.from_numpy(rows).to(dev)].cpu().numpy()
    del G
    for r, g_row in zip(rows, G_rows):
        s, n = int(c.row_start[r]), int(c.row_nnz[r])
        wc, wv = oracle.drop_grow_row(c.col_indices[s:s + n], c.values[s:s + n], thr, "gradient",
                                      c.ncols, g_row, row=int(r))
        m = int(after.row_nnz[r])
        assert m == wc.size, r
        assert_bits_equal(after.col_indices[s:s + m], wc, f"RigL cols row {r}")
        assert_bits_equal(after.values[s:s + m], wv, f"RigL vals row {r}")
    print(f"[config c5 RigL] density={density} rebuild + forward", flush=True)
    WT = ops._cached_transpose(W)
    WT_o, perm_o = oracle.transpose_with_perm(after)
    csr_arrays_equal(to_oracle(WT), WT_o, "WT after RigL")
    assert_bits_equal(ops._transpose_cache[id(W)][3].cpu().numpy(), perm_o, "perm after RigL")
    Y = ops._launch_spmm(W, X)
    sub, _ = oracle.sub_rows(after, rows)
    assert_bits_equal(Y[torch.from_numpy(rows).to(dev)].cpu().numpy(), oracle.spmm(sub, X_h),
                      "Y after RigL on sampled rows")
