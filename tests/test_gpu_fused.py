"""GPU parity of slk_backward_fused: a small layer's dW (SIMD order), dbias
and dX = Wᵀ·dY in one launch, W's values read through the transpose's slot
map instead of a refresh.

The bar is bit-exact against the separate launches it replaces (slk_sddmm in
the SIMD order, slk_transpose_refresh + slk_spmm on WT), which are pinned to
the oracle elsewhere; dW and dX are also checked against the oracle directly.
Cases: ragged and empty rows, transpose rows longer than one 64-slot piece,
N not a multiple of 64 or of 4, values changed after the transpose was built
(stale WT values are never read), bias, and the autograd path with the fused
launch forced on and off.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from helpers import assert_bits_equal, from_oracle
from sparsecore_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _case(kind, seed):
    if kind == "c1":
        return oracle.uniform_rows(512, 784, 78, seed=seed, sigma=0.02)
    if kind == "zipf":  # long columns: transpose rows of several 64-slot pieces
        return oracle.zipf_rows(300, 200, 0.3, 1.1, seed=seed, sigma=1.0)
    if kind == "empty":  # empty rows and empty columns
        W = np.random.default_rng(seed).standard_normal((70, 90)).astype(np.float32)
        W *= np.random.default_rng(seed + 1).random((70, 90)) < 0.1
        W[5:9] = 0.0
        W[:, 20:30] = 0.0
        return oracle.from_dense(W)
    if kind == "dense-col":  # one column in every row: a 200-slot transpose row
        W = np.random.default_rng(seed).standard_normal((200, 40)).astype(np.float32)
        W *= np.random.default_rng(seed + 1).random((200, 40)) < 0.2
        W[:, 7] = np.random.default_rng(seed + 2).standard_normal(200)
        return oracle.from_dense(W)
    raise KeyError(kind)


def _separate(W, dY, X, dbias):
    """The launches the fused one replaces: slk_sddmm(_bias) in the SIMD
    order, then the refresh and slk_spmm on the cached transpose."""
    dW = ops._launch_sddmm(W, dY, X, "simd", dbias)
    WT = ops._cached_transpose(W)
    dX = ops._launch_spmm(WT, dY)
    return dW, dX


@pytest.mark.parametrize("N", [256, 100, 6, 64, 330])
@pytest.mark.parametrize("kind", ["c1", "zipf", "empty", "dense-col"])
def test_backward_fused_bits(dev, kind, N):
    print(f"[fused backward] {kind} N={N}", flush=True)
    c = _case(kind, seed=N + len(kind))
    rng = np.random.default_rng(N)
    X_np = rng.standard_normal((c.ncols, N)).astype(np.float32)
    dY_np = rng.standard_normal((c.nrows, N)).astype(np.float32)
    W = from_oracle(c, dev)
    X, dY = _t(X_np, dev), _t(dY_np, dev)
    for with_bias in (False, True):
        db_sep = torch.full((c.nrows,), float("nan"), device=dev) if with_bias else None
        dW_sep, dX_sep = _separate(W, dY, X, db_sep)
        WT, perm = ops._cached_transpose_structure(W)
        dW = torch.full((W.total_capacity,), float("nan"), device=dev)
        dX = torch.full((c.ncols, N), float("nan"), device=dev)
        db = torch.full((c.nrows,), float("nan"), device=dev) if with_bias else None
        _lib.backward_fused(W._view(), WT._view(), perm, dY, X, dW, db, dX)
        assert_bits_equal(dW.cpu().numpy(), dW_sep.cpu().numpy(), f"dW bias={with_bias}")
        assert_bits_equal(dX.cpu().numpy(), dX_sep.cpu().numpy(), f"dX bias={with_bias}")
        if with_bias:
            assert_bits_equal(db.cpu().numpy(), db_sep.cpu().numpy(), "dbias")
    # and against the oracle itself
    cT, _ = oracle.transpose_with_perm(c)
    assert_bits_equal(dX.cpu().numpy(), oracle.spmm(cT, dY_np), "dX vs oracle")
    assert_bits_equal(dW.cpu().numpy(), oracle.sddmm(c, dY_np, X_np, "simd"), "dW vs oracle")


def test_backward_fused_reads_current_values(dev):
    """The transpose's values go stale when W's values change in place (an
    optimizer step); the fused launch reads W's through perm, so dX follows."""
    c = _case("c1", seed=5)
    rng = np.random.default_rng(5)
    X = _t(rng.standard_normal((c.ncols, 256)).astype(np.float32), dev)
    dY = _t(rng.standard_normal((c.nrows, 256)).astype(np.float32), dev)
    W = from_oracle(c, dev)
    ops._cached_transpose(W)  # WT holds the old values
    with torch.no_grad():
        W.values.mul_(-1.5).add_(0.25)
    WT, perm = ops._cached_transpose_structure(W)
    dW = torch.empty(W.total_capacity, device=dev)
    dX = torch.empty(c.ncols, 256, device=dev)
    _lib.backward_fused(W._view(), WT._view(), perm, dY, X, dW, None, dX)
    dW_sep, dX_sep = _separate(W, dY, X, None)  # refreshes first
    assert_bits_equal(dX.cpu().numpy(), dX_sep.cpu().numpy(), "dX after a values change")
    assert_bits_equal(dW.cpu().numpy(), dW_sep.cpu().numpy(), "dW after a values change")


@pytest.mark.parametrize("fused", [True, False])
def test_autograd_backward_fused_or_not_same_bits(dev, tune, fused):
    """ops.spmm's backward takes the fused launch for small layers; forced on
    or off, the gradients are the same bits."""
    tune(fused_backward=fused)
    c = _case("c1", seed=9)
    rng = np.random.default_rng(9)
    X_np = rng.standard_normal((c.ncols, 256)).astype(np.float32)
    g_np = rng.standard_normal((c.nrows, 256)).astype(np.float32)
    grads = []
    for force in (fused, not fused):
        ops._overrides["fused_backward"] = force
        W = from_oracle(c, dev)
        vals = W.values.clone().requires_grad_(True)
        X = _t(X_np, dev).requires_grad_(True)
        Y = ops._SpMMFunction.apply(vals, W, X, "auto")
        Y.backward(_t(g_np, dev))
        grads.append((vals.grad.cpu().numpy(), X.grad.cpu().numpy()))
    want_dW = oracle.sddmm(c, g_np, X_np, "simd")
    assert_bits_equal(grads[0][0], want_dW, "dW vs oracle")
    assert_bits_equal(grads[0][0], grads[1][0], "dW")
    assert_bits_equal(grads[0][1], grads[1][1], "dX")


def test_backward_fused_errors(dev):
    c = _case("empty", seed=1)
    W = from_oracle(c, dev)
    WT, perm = ops._cached_transpose_structure(W)
    dY = torch.zeros(c.nrows, 8, device=dev)
    X = torch.zeros(c.ncols, 8, device=dev)
    dW = torch.empty(W.total_capacity, device=dev)
    dX = torch.empty(c.ncols, 8, device=dev)
    with pytest.raises(ValueError, match="WT is not W's transpose"):
        _lib.backward_fused(W._view(), W._view(), perm, dY, X, dW, None, dX)
    with pytest.raises(ValueError, match="NULL perm"):
        _lib.backward_fused(W._view(), WT._view(), torch.empty(0, dtype=torch.int64, device=dev),
                            dY, X, dW, None, dX)
