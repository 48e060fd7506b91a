"""GPU tests of the public API, restating the reference's own test suite.

Mirrors sparselab's tests/test_spmm.py, test_spmm_grad.py, test_spmm_autograd.py,
test_sparse_linear.py and test_transpose_cache.py on the HIP device: same
shapes, same oracles (dense torch products, float32 tolerance 1e-5 where the
reference uses it; gradcheck at eps=1e-3, atol=rtol=1e-2) and the same error
types and message substrings. Where the reference asserted CPU-only behaviour
(test_spmm_rejects_non_cpu_X) the contract is inverted: CPU tensors are
rejected instead.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
import sparsecore_amd as slk
from helpers import assert_bits_equal, from_oracle, make_sparse_W, to_oracle
from sparsecore_amd import PaddedCSR, SparseLinear, _lib
from sparsecore_amd.ops import (_SpMMFunction, _cached_transpose, _clear_transpose_cache,
                                _transpose_cache)

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def clean_cache():
    _clear_transpose_cache()
    yield
    _clear_transpose_cache()


def _W(M, K, sparsity, seed, dev, padding_ratio=0.2):
    W_csr, W_dense = make_sparse_W(M, K, sparsity, seed)
    if padding_ratio != 0.2:
        W_csr = PaddedCSR.from_dense(W_dense, padding_ratio=padding_ratio)
    return W_csr.to(dev), W_dense.to(dev)


# ───────────────────────── spmm (test_spmm.py) ─────────────────────────

@pytest.mark.parametrize("M,K,N", [(32, 32, 32), (128, 64, 16), (64, 128, 256), (7, 13, 5),
                                   (1, 1, 1)])
@pytest.mark.parametrize("sparsity", [0.0, 0.5, 0.9, 0.99])
def test_spmm_matches_dense_matmul(dev, M, K, N, sparsity):
    if M * K < 4 and sparsity >= 0.9:
        pytest.skip("not enough cells for >=90% sparsity")
    W, Wd = _W(M, K, sparsity, 42, dev)
    X = torch.randn(K, N, generator=torch.Generator().manual_seed(M * K + N)).to(dev)
    Y = slk.spmm(W, X)
    assert Y.shape == (M, N) and Y.dtype == torch.float32 and Y.device == X.device
    # float64 product; the float32 chain's error is bounded relative to the
    # sum of |terms| (a plain rtol=1e-5 is too tight where terms cancel)
    Y64 = Wd.double() @ X.double()
    bound = 1e-5 * (Wd.double().abs() @ X.double().abs()) + 1e-6
    err = (Y.double() - Y64).abs()
    assert bool((err <= bound).all()), f"max err {err.max().item():.3e}"
    # and bit-exact against the reference arithmetic
    assert_bits_equal(Y.cpu().numpy(), oracle.spmm(to_oracle(W), X.cpu().numpy()), "Y")


def test_spmm_edge_cases(dev):
    assert torch.equal(slk.spmm(PaddedCSR.from_dense(torch.zeros(10, 20)).to(dev),
                                torch.randn(20, 5, device=dev)), torch.zeros(10, 5, device=dev))
    Y = slk.spmm(PaddedCSR(nrows=8, ncols=16, device=dev), torch.randn(16, 4, device=dev))
    assert Y.shape == (8, 4) and torch.equal(Y, torch.zeros(8, 4, device=dev))
    Wd = torch.zeros(4, 6)
    Wd[2, 3] = 2.5
    X = torch.randn(6, 3, device=dev)
    Y = slk.spmm(PaddedCSR.from_dense(Wd).to(dev), X)
    for r in (0, 1, 3):
        assert torch.equal(Y[r], torch.zeros(3, device=dev))
    assert torch.equal(Y[2], 2.5 * X[3])  # one fma from +0.0 is the rounded product
    W, Wd = _W(32, 24, 0.8, 1, dev)
    x = torch.randn(24, 1, device=dev)
    assert torch.allclose(slk.spmm(W, x), Wd @ x, rtol=1e-5, atol=1e-5)
    W, Wd = _W(16, 32, 0.7, 5, dev, padding_ratio=1.0)
    X = torch.randn(32, 8, device=dev)
    assert torch.allclose(slk.spmm(W, X), Wd @ X, rtol=1e-5, atol=1e-5)


def test_spmm_errors(dev):
    W, _ = _W(8, 16, 0.5, 0, dev)
    with pytest.raises(ValueError, match="2-D"):
        slk.spmm(W, torch.randn(16, device=dev))
    with pytest.raises(ValueError, match="shape|match|ncols"):
        slk.spmm(W, torch.randn(17, 4, device=dev))
    with pytest.raises(TypeError, match="PaddedCSR"):
        slk.spmm(torch.randn(8, 16, device=dev), torch.randn(16, 4, device=dev))
    with pytest.raises(TypeError, match="torch.Tensor"):
        slk.spmm(W, np.random.randn(16, 4).astype(np.float32))
    with pytest.raises(RuntimeError, match="HIP"):
        slk.spmm(W, torch.randn(16, 4))
    with pytest.raises(RuntimeError, match="HIP device only"):
        slk.spmm(W.cpu(), torch.randn(16, 4, device=dev))
    with pytest.raises(ValueError, match="unknown kernel"):
        slk.spmm(W, torch.randn(16, 4, device=dev), kernel="neon")


def test_spmm_dtype_and_layout_coercion(dev):
    W, Wd = _W(16, 24, 0.7, 2, dev)
    X64 = torch.randn(24, 8, dtype=torch.float64, device=dev)
    Y = slk.spmm(W, X64)
    assert Y.dtype == torch.float32
    assert torch.allclose(Y, Wd @ X64.float(), rtol=1e-5, atol=1e-5)
    W, Wd = _W(10, 20, 0.5, 3, dev)
    Xv = torch.randn(8, 20, device=dev).T
    assert not Xv.is_contiguous()
    assert torch.allclose(slk.spmm(W, Xv), Wd @ Xv, rtol=1e-5, atol=1e-5)


def test_spmm_idempotent(dev):
    W, _ = _W(32, 32, 0.8, 7, dev)
    X = torch.randn(32, 16, device=dev)
    Y1 = slk.spmm(W, X)
    for _ in range(3):
        assert torch.equal(slk.spmm(W, X), Y1)


# ─────────────────────── dW (test_spmm_grad.py) ────────────────────────

def _dense_grad(Wd, X, dY):
    return (dY.double() @ X.double().T)


@pytest.mark.parametrize("M,K,N,sparsity", [(4, 5, 3, 0.5), (16, 16, 8, 0.5), (32, 16, 4, 0.8),
                                            (8, 32, 16, 0.9), (64, 64, 32, 0.95),
                                            (1, 16, 8, 0.0), (16, 1, 8, 0.0), (16, 16, 1, 0.5)])
@pytest.mark.parametrize("kernel", ["scalar", "simd"])
def test_dw_matches_dense_autograd(dev, M, K, N, sparsity, kernel):
    torch.manual_seed(42)
    Wd = torch.randn(M, K) * (torch.rand(M, K) >= sparsity).float()
    X = torch.randn(K, N)
    dY = torch.randn(M, N)
    W = PaddedCSR.from_dense(Wd).to(dev)
    vals = W.values.clone().requires_grad_(True)
    Y = _SpMMFunction.apply(vals, W, X.to(dev), kernel)
    Y.backward(dY.to(dev))
    dW = vals.grad.cpu().numpy()
    assert dW.shape == (W.total_capacity,)
    c = to_oracle(W)
    slots, rows, cols = oracle.live_slots(c)
    G = _dense_grad(Wd, X, dY).numpy()
    np.testing.assert_allclose(dW[slots], G[rows, cols], rtol=1e-5, atol=1e-5)
    assert np.all(dW[oracle.padding_slots(c)] == 0.0)
    assert_bits_equal(dW, oracle.sddmm(c, dY.numpy(), X.numpy(), kernel), "dW vs oracle")


@pytest.mark.parametrize("padding_ratio", [0.0, 0.2, 0.5, 1.0])
def test_dw_padding_exactly_zero(dev, padding_ratio):
    torch.manual_seed(1)
    Wd = torch.randn(10, 12) * (torch.rand(10, 12) >= 0.6).float()
    W = PaddedCSR.from_dense(Wd, padding_ratio=padding_ratio).to(dev)
    vals = W.values.clone().requires_grad_(True)
    _SpMMFunction.apply(vals, W, torch.randn(12, 5, device=dev), "simd").backward(
        torch.randn(10, 5, device=dev))
    pads = oracle.padding_slots(to_oracle(W))
    assert np.all(vals.grad.cpu().numpy()[pads] == 0.0)


# ─────────────────────── autograd (test_spmm_autograd.py) ──────────────

@pytest.mark.parametrize("M,K,N,sparsity", [(4, 5, 3, 0.0), (4, 5, 3, 0.5), (8, 6, 4, 0.75),
                                            (6, 8, 2, 0.5)])
def test_gradcheck_dX(dev, M, K, N, sparsity):
    torch.manual_seed(42)
    Wd = torch.randn(M, K, dtype=torch.float64) * (torch.rand(M, K) >= sparsity).double()
    W = PaddedCSR.from_dense(Wd.float()).to(dev)
    X = torch.randn(K, N, dtype=torch.float64, device=dev, requires_grad=True)
    assert torch.autograd.gradcheck(lambda x: slk.spmm(W, x.float()).double(), (X,), eps=1e-3,
                                    atol=1e-2, rtol=1e-2, check_undefined_grad=False)


@pytest.mark.parametrize("kernel", ["scalar", "simd"])
def test_gradcheck_dW_values(dev, kernel):
    torch.manual_seed(42)
    M, K, N = 4, 5, 3
    Wd = torch.randn(M, K, dtype=torch.float64) * (torch.rand(M, K) >= 0.5).double()
    W = PaddedCSR.from_dense(Wd.float()).to(dev)
    wv = W.values.detach().double().clone().requires_grad_(True)
    X = torch.randn(K, N, dtype=torch.float64, device=dev)

    def fn(wv_double):
        wv_f32 = wv_double.float().contiguous()
        with torch.no_grad():
            W.values.copy_(wv_f32)
        return _SpMMFunction.apply(wv_f32, W, X.float(), kernel).double()

    assert torch.autograd.gradcheck(fn, (wv,), eps=1e-3, atol=1e-2, rtol=1e-2,
                                    check_undefined_grad=False)


@pytest.mark.parametrize("M,K,N,sparsity", [(16, 16, 8, 0.0), (16, 16, 8, 0.5),
                                            (16, 32, 8, 0.9), (32, 16, 16, 0.8)])
def test_backward_dX_matches_dense(dev, M, K, N, sparsity):
    torch.manual_seed(1)
    Wd = torch.randn(M, K) * (torch.rand(M, K) >= sparsity).float()
    W = PaddedCSR.from_dense(Wd).to(dev)
    X0 = torch.randn(K, N)
    up = torch.randn(M, N)
    X = X0.clone().to(dev).requires_grad_(True)
    slk.spmm(W, X).backward(up.to(dev))
    Xr = X0.clone().double().requires_grad_(True)
    (Wd.double() @ Xr).backward(up.double())
    assert torch.allclose(X.grad.cpu(), Xr.grad.float(), rtol=1e-5, atol=1e-5)
    WT, _ = oracle.transpose_with_perm(to_oracle(W))
    assert_bits_equal(X.grad.cpu().numpy(), oracle.spmm(WT, up.numpy()), "dX vs oracle")


def test_no_gradient_computed_when_not_needed(dev):
    W, _ = _W(16, 16, 0.5, 0, dev)
    vals = W.values.clone().requires_grad_(True)
    X = torch.randn(16, 4, device=dev)  # no grad: dX is skipped, so is the transpose
    _SpMMFunction.apply(vals, W, X, "simd").sum().backward()
    assert vals.grad is not None and len(_transpose_cache) == 0


# ─────────────────────── SparseLinear (test_sparse_linear.py) ──────────

def test_sparse_linear_forward_matches_dense(dev):
    torch.manual_seed(42)
    layer = SparseLinear(32, 16, sparsity=0.5).to(dev)
    x = torch.randn(6, 32, device=dev)
    y = layer(x)
    W = layer._csr.to_dense()
    torch.testing.assert_close(y, x @ W.t() + layer.bias, rtol=1e-5, atol=1e-5)
    layer = SparseLinear(16, 8, sparsity=0.5, bias=False).to(dev)
    assert layer(torch.randn(2, 5, 16, device=dev)).shape == (2, 5, 8)
    with pytest.raises(ValueError, match="last dim"):
        layer(torch.randn(4, 12, device=dev))


@pytest.mark.parametrize("batch", [1, 37, 256])
def test_sparse_linear_with_bias_bit_exact_vs_oracle(dev, batch):
    """SparseLinear's forward (bias fused into the SpMM store) gives the bits of
    the reference's spmm followed by its separate `y + bias`; dW and dX are
    the oracle's bit for bit and dbias is Σ over the batch. The second layer
    takes the first one's transposed-view output directly (no input copy)."""
    torch.manual_seed(batch)
    l1 = SparseLinear(784, 512, sparsity=0.9).to(dev)
    l2 = SparseLinear(512, 10, sparsity=0.9).to(dev)
    x = torch.rand(batch, 784, device=dev)
    h = torch.relu(l1(x)).detach().requires_grad_(True)
    y = l2(h)
    up = torch.randn_like(y)
    y.backward(up)
    c = to_oracle(l2._csr)
    b = l2.bias.detach().cpu().numpy()
    H_col = h.detach().t().contiguous().cpu().numpy()
    dY_col = up.t().contiguous().cpu().numpy()
    assert_bits_equal(y.detach().t().cpu().numpy(), oracle.spmm(c, H_col) + b[:, None], "y")
    assert_bits_equal(l2._values.grad.cpu().numpy(), oracle.sddmm(c, dY_col, H_col), "dW")
    WT, _ = oracle.transpose_with_perm(c)
    assert_bits_equal(h.grad.t().cpu().numpy(), oracle.spmm(WT, dY_col), "dX")
    torch.testing.assert_close(l2.bias.grad, up.sum(0), rtol=1e-5, atol=1e-5)
    c1 = to_oracle(l1._csr)
    X_col = x.t().contiguous().cpu().numpy()
    h_ref = np.maximum(oracle.spmm(c1, X_col) + l1.bias.detach().cpu().numpy()[:, None], 0)
    assert_bits_equal(h.detach().t().cpu().numpy(), h_ref, "relu(l1)")


@pytest.mark.parametrize("out_features,batch", [(10, 256), (1, 37), (64, 5), (33, 130)])
def test_narrow_layer_matches_general_path_bits(dev, monkeypatch, out_features, batch):
    """A layer with at most 64 outputs runs the narrow path (token-major store,
    one backward launch, no transpose cache); its output and all three
    gradients are the general path's bit for bit, and the output comes back
    contiguous."""
    from sparsecore_amd import ops

    torch.manual_seed(out_features)
    layer = SparseLinear(300, out_features, sparsity=0.9).to(dev)
    assert ops._narrow_layer(layer._csr)
    x = torch.rand(batch, 300, device=dev)
    up = torch.randn(batch, out_features, device=dev)
    runs = []
    for narrow in (True, False):
        if not narrow:
            monkeypatch.setattr(ops, "_narrow_layer", lambda W: False)
        layer.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_(True)
        y = layer(xi)
        assert y.is_contiguous() or not narrow
        y.backward(up)
        runs.append((y.detach().clone(), layer._values.grad.clone(), layer.bias.grad.clone(),
                     xi.grad.clone()))
    for a, b, what in zip(runs[0], runs[1], ("y", "dW", "dbias", "dx")):
        assert_bits_equal(a.cpu().numpy(), b.cpu().numpy(), what)


def test_narrow_layer_gradcheck(dev):
    torch.manual_seed(0)
    layer = SparseLinear(8, 4, sparsity=0.5).to(dev).double()
    x = torch.randn(3, 8, dtype=torch.double, device=dev, requires_grad=True)
    assert torch.autograd.gradcheck(lambda x: layer(x).sum(), (x,), eps=1e-3, atol=1e-3,
                                    rtol=1e-3)


def test_sparse_linear_zero_sparsity_matches_nn_linear(dev):
    torch.manual_seed(7)
    layer = SparseLinear(16, 8, sparsity=0.0).to(dev)
    ref = nn.Linear(16, 8).to(dev)
    with torch.no_grad():
        ref.weight.copy_(layer._csr.to_dense())
        ref.bias.copy_(layer.bias)
    x = torch.randn(3, 16, device=dev)
    torch.testing.assert_close(layer(x), ref(x), rtol=1e-5, atol=1e-5)


def test_sparse_linear_backward_and_optimizers(dev):
    torch.manual_seed(0)
    layer = SparseLinear(16, 8, sparsity=0.7).to(dev)
    x = torch.randn(4, 16, device=dev)
    layer(x).sum().backward()
    assert layer._values.grad.shape == layer._values.shape
    assert torch.isfinite(layer._values.grad).all() and layer.bias.grad.shape == (8,)
    pads = oracle.padding_slots(to_oracle(layer._csr))
    assert torch.all(layer._values.grad.cpu()[pads] == 0)
    opt = torch.optim.SGD(layer.parameters(), lr=0.01)
    v0, b0 = layer._values.detach().clone(), layer.bias.detach().clone()
    opt.step()
    assert not torch.equal(v0, layer._values) and not torch.equal(b0, layer.bias)
    assert layer._csr.values.data_ptr() == layer._values.data_ptr()  # aliasing kept
    adam = torch.optim.Adam(layer.parameters(), lr=0.01)
    for _ in range(3):
        adam.zero_grad()
        layer(torch.randn(4, 16, device=dev)).sum().backward()
        adam.step()
    assert torch.isfinite(layer._values).all()


def test_optimizer_update_reaches_csr_buffer(dev):
    torch.manual_seed(0)
    layer = SparseLinear(16, 8, sparsity=0.5).to(dev)
    x = torch.randn(4, 16, device=dev)
    y_before = layer(x).detach().clone()
    with torch.no_grad():
        layer._values.data.fill_(0.0)
    y_after = layer(x).detach()
    torch.testing.assert_close(y_after, layer.bias.expand_as(y_after), rtol=1e-5, atol=1e-5)
    assert not torch.allclose(y_before, y_after)


def test_mini_training_loop_decreases_loss(dev):
    torch.manual_seed(0)
    T = torch.randn(16, 32, device=dev) * 0.1
    layer = SparseLinear(32, 16, sparsity=0.5, bias=False).to(dev)
    opt = torch.optim.SGD(layer.parameters(), lr=0.1)
    losses = []
    for _ in range(20):
        x = torch.randn(64, 32, device=dev)
        opt.zero_grad()
        loss = ((layer(x) - x @ T.t()) ** 2).mean()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert losses[-1] < losses[0] * 0.7


def test_state_dict_roundtrip_and_reset(dev):
    torch.manual_seed(0)
    a = SparseLinear(16, 8, sparsity=0.5).to(dev)
    torch.manual_seed(0)
    b = SparseLinear(16, 8, sparsity=0.5).to(dev)
    opt = torch.optim.SGD(a.parameters(), lr=0.1)
    a(torch.randn(4, 16, device=dev)).sum().backward()
    opt.step()
    b.load_state_dict(a.state_dict())
    x = torch.randn(4, 16, device=dev)
    torch.testing.assert_close(a(x), b(x), rtol=1e-5, atol=1e-5)
    v1 = b._values.detach().clone()
    torch.manual_seed(123)
    b.reset_parameters()
    assert b._values.device == x.device and b._csr.values.data_ptr() == b._values.data_ptr()
    assert not torch.equal(b._values.detach(), v1) or v1.numel() != b._values.numel()
    assert b(x).shape == (4, 8)


def test_matches_reference_init_stream(dev):
    """Same torch RNG draws as the reference (uniform weights, rand mask, bias)."""
    torch.manual_seed(3)
    layer = SparseLinear(20, 10, sparsity=0.6)
    torch.manual_seed(3)
    bound = 1.0 / np.sqrt(max(1.0, 20 * 0.4))
    Wd = torch.empty(10, 20)
    nn.init.uniform_(Wd, -bound, bound)
    Wd = Wd * (torch.rand(10, 20) >= 0.6).float()
    b = torch.empty(10)
    nn.init.uniform_(b, -bound, bound)
    assert torch.equal(layer._csr.to_dense(), Wd) and torch.equal(layer.bias.data, b)
    layer = layer.to(dev)
    assert torch.equal(layer._csr.to_dense().cpu(), Wd)


# ───────────────── transpose cache (test_transpose_cache.py) ───────────

@pytest.fixture
def general_path(monkeypatch):
    """Layers with at most 64 outputs take the narrow path, which has no
    transpose cache (slk_backward_narrow). The cache tests below restate the
    reference's own (tests/test_transpose_cache.py) on its shapes, so they
    pin the general path."""
    from sparsecore_amd import ops

    monkeypatch.setattr(ops, "_narrow_layer", lambda W: False)


def test_cache_hit_miss_refresh(dev):
    W = PaddedCSR.random(8, 16, sparsity=0.5, seed=0).to(dev)
    WT1 = _cached_transpose(W)
    assert _cached_transpose(W) is WT1
    v0 = W.topology_version
    W.rewrite_row(0, np.array([0, 5], dtype=np.int32), np.array([1.0, 2.0], dtype=np.float32))
    assert W.topology_version > v0
    WT2 = _cached_transpose(W)
    assert WT2 is not WT1
    before = WT2.values.clone()
    with torch.no_grad():
        W.values.mul_(10.0)
    WT3 = _cached_transpose(W)
    assert WT3 is WT2 and not torch.allclose(before, WT3.values)
    fresh = W.transpose()
    assert torch.equal(WT3.to_dense(), fresh.to_dense())
    assert torch.equal(WT3.values, fresh.values)


def test_cache_entry_dropped_with_matrix(dev):
    W = PaddedCSR.random(8, 16, sparsity=0.5, seed=1).to(dev)
    _cached_transpose(W)
    assert len(_transpose_cache) == 1
    del W
    import gc

    gc.collect()
    assert len(_transpose_cache) == 0


def test_cached_and_fresh_gradients_match(dev, general_path):
    torch.manual_seed(0)
    la = SparseLinear(16, 8, sparsity=0.5, bias=False).to(dev)
    torch.manual_seed(0)
    lb = SparseLinear(16, 8, sparsity=0.5, bias=False).to(dev)
    x = torch.randn(4, 16, device=dev)
    xa = x.clone().requires_grad_(True)
    xb = x.clone().requires_grad_(True)
    la(xa).sum().backward()
    _clear_transpose_cache()
    lb(xb).sum().backward()
    assert torch.equal(la._values.grad, lb._values.grad) and torch.equal(xa.grad, xb.grad)
    with torch.no_grad():
        la._values.mul_(0.95)
        lb._values.mul_(0.95)
    la._values.grad = None
    lb._values.grad = None
    xa.grad = None
    xb.grad = None
    la(xa).sum().backward()  # cache hit + refresh
    _clear_transpose_cache()
    lb(xb).sum().backward()  # rebuild
    assert torch.equal(xa.grad, xb.grad)
    (cached_version, shape, WT, perm) = list(_transpose_cache.values())[0]
    assert shape == (8, 16) and perm.dtype == torch.int64


def test_rewrite_invalidates_cache_in_training(dev, general_path):
    torch.manual_seed(0)
    layer = SparseLinear(16, 8, sparsity=0.5, bias=False).to(dev)
    layer(torch.randn(4, 16, device=dev, requires_grad=True)).sum().backward()
    (v0, _, _, _) = list(_transpose_cache.values())[0]
    layer._csr.rewrite_row(3, [1, 2, 3], [0.5, 0.25, 0.125])
    x = torch.randn(4, 16, device=dev, requires_grad=True)
    layer(x).sum().backward()
    (v1, _, WT, _) = list(_transpose_cache.values())[0]
    assert v1 != v0
    dense = layer._csr.to_dense()
    torch.testing.assert_close(x.grad, torch.ones(4, 8, device=dev) @ dense, rtol=1e-5,
                               atol=1e-5)


def test_batched_transpose_build_matches_single_builds(dev):
    """transposes_with_perm over several matrices gives each one's
    transpose_with_perm arrays exactly (one capacity read for all)."""
    from sparsecore_amd import layout

    Ws = [PaddedCSR.random(m, k, sparsity=s, seed=i).to(dev)
          for i, (m, k, s) in enumerate([(40, 70, 0.7), (5, 300, 0.9), (128, 16, 0.2), (1, 1, 0.0)])]
    for W, (WT, perm) in zip(Ws, layout.transposes_with_perm(Ws)):
        WT1, perm1 = layout.transpose_with_perm(W)
        for a in ("values", "col_indices", "row_start", "row_nnz", "row_capacity"):
            assert torch.equal(getattr(WT, a), getattr(WT1, a)), a
        assert torch.equal(perm, perm1)
    assert layout.transposes_with_perm([]) == []


def test_set_step_rebuilds_stale_transposes_in_one_batch(dev, general_path):
    """After SET rewrites the layers, their cached transposes are current (the
    next backward hits the cache) and equal fresh transposes."""
    torch.manual_seed(0)
    model = nn.Sequential(SparseLinear(64, 96, sparsity=0.8), nn.ReLU(),
                          SparseLinear(96, 80, sparsity=0.8)).to(dev)
    algo = slk.SET(sparsity=0.8, drop_fraction=0.3, update_freq=1, seed=3)
    model.apply(algo)
    x = torch.randn(32, 64, device=dev, requires_grad=True)
    model(x).sum().backward()
    layers = [model[0], model[2]]
    versions = [l._csr.topology_version for l in layers]
    with torch.no_grad():
        for l in layers:
            l._values.add_(torch.randn_like(l._values) * 0.01)
    algo.step()
    for l, v0 in zip(layers, versions):
        W = l._csr
        assert W.topology_version != v0
        ver, shape, WT, perm = _transpose_cache[id(W)]
        assert ver == W.topology_version and shape == (W.nrows, W.ncols)
        fresh = W.transpose()
        assert torch.equal(WT.col_indices, fresh.col_indices)
        assert torch.equal(WT.values, fresh.values)


def test_gradcheck_with_cache_enabled(dev, general_path):
    torch.manual_seed(0)
    layer = SparseLinear(8, 4, sparsity=0.5, bias=False).to(dev)
    x = torch.randn(3, 8, dtype=torch.double, device=dev, requires_grad=True)
    layer.double()
    assert layer._csr.values.dtype == torch.float32
    assert torch.autograd.gradcheck(lambda x: layer(x).sum(), (x,), eps=1e-3, atol=1e-3,
                                    rtol=1e-3)


# ──────────────────── device invariants and rewrite_row ────────────────

def _corrupt(c: oracle.Csr, kind: int, rng) -> oracle.Csr:
    q = c.copy()
    i = int(rng.integers(0, q.nrows))
    s, n, cap = int(q.row_start[i]), int(q.row_nnz[i]), int(q.row_capacity[i])
    if kind == 0 and n:
        q.col_indices[s + int(rng.integers(0, n))] = int(rng.integers(-3, q.ncols + 3))
    elif kind == 1 and n >= 2:
        q.col_indices[s], q.col_indices[s + 1] = q.col_indices[s + 1], q.col_indices[s]
    elif kind == 2 and cap > n:
        q.col_indices[s + n] = int(rng.integers(0, q.ncols))
    elif kind == 3:
        q.row_nnz[i] = cap + 1
    elif kind == 4 and i > 0:
        q.row_start[i] += 1
    elif kind == 5:
        q.row_start[0] = 1
    return q


def test_device_invariant_checker_matches_reference_messages(dev):
    rng = np.random.default_rng(0)
    base = oracle.uniform_rows(12, 20, 5, seed=1)
    for trial in range(36):
        q = _corrupt(base, trial % 6, rng)
        expect = oracle.check_invariants(q.nrows, q.ncols, q.values, q.col_indices, q.row_start,
                                         q.row_nnz, q.row_capacity)
        args = [torch.from_numpy(a.copy()).to(dev) for a in
                (q.values, q.col_indices, q.row_start, q.row_nnz, q.row_capacity)]
        if expect:
            with pytest.raises(ValueError) as ei:
                PaddedCSR(q.nrows, q.ncols, *args)
            assert str(ei.value) == "PaddedCSR invariant check failed: " + expect
        else:
            PaddedCSR(q.nrows, q.ncols, *args).assert_invariants()


def test_rewrite_row_on_device_matches_reference(dev):
    c = oracle.uniform_rows(6, 30, 8, seed=4)
    W = from_oracle(c, dev)
    q = c
    for row, cols in [(0, [1, 5, 9]), (3, []), (5, list(range(0, 27, 3))), (3, [29])]:
        vals = np.arange(len(cols), dtype=np.float32) + 0.5
        W.rewrite_row(row, np.array(cols, dtype=np.int32), vals)
        q = oracle.rewrite_row(q, row, cols, vals)
    got = to_oracle(W)
    for name in ("values", "col_indices", "row_nnz"):
        assert_bits_equal(getattr(got, name), getattr(q, name), name)
    assert W.topology_version == 4 and W.nnz == q.nnz
    W.assert_invariants()
    with pytest.raises(ValueError, match="out of range"):
        W.rewrite_row(6, [1], [1.0])
    with pytest.raises(ValueError, match="ascending"):
        W.rewrite_row(0, [3, 3], [1.0, 2.0])
    with pytest.raises(ValueError, match="capacity"):
        W.rewrite_row(0, list(range(20)), [1.0] * 20)
    with pytest.raises(ValueError, match="must equal"):
        W.rewrite_row(0, [1, 2], [1.0])


# ───────────── device construction and topology serialization ──────────

@pytest.mark.parametrize("padding_ratio,threshold", [(0.2, 0.0), (0.0, 0.0), (1.0, 0.5)])
def test_device_factories_match_host_build(dev, padding_ratio, threshold):
    """from_dense / from_torch_sparse_csr of HIP tensors build on the device and
    give the same arrays as the host build (empty rows included)."""
    g = torch.Generator().manual_seed(11)
    W = torch.randn(37, 53, generator=g) * (torch.rand(37, 53, generator=g) < 0.2)
    W[5] = 0.0
    host = PaddedCSR.from_dense(W, padding_ratio=padding_ratio, threshold=threshold)
    devb = PaddedCSR.from_dense(W.to(dev), padding_ratio=padding_ratio, threshold=threshold)
    assert devb.device.type == "cuda"
    for name in ("values", "col_indices", "row_start", "row_nnz", "row_capacity"):
        assert torch.equal(getattr(devb, name).cpu(), getattr(host, name)), name
    sp = W.to_sparse_csr().to(dev)
    devc = PaddedCSR.from_torch_sparse_csr(sp, padding_ratio=padding_ratio)
    hostc = PaddedCSR.from_torch_sparse_csr(W.to_sparse_csr(), padding_ratio=padding_ratio)
    for name in ("values", "col_indices", "row_start", "row_nnz", "row_capacity"):
        assert torch.equal(getattr(devc, name).cpu(), getattr(hostc, name)), name


def test_device_sparse_csr_with_unsorted_row_is_rejected(dev):
    crow = torch.tensor([0, 2, 3], device=dev)
    col = torch.tensor([3, 1, 0], device=dev)
    val = torch.tensor([1.0, 2.0, 3.0], device=dev)
    sp = torch.sparse_csr_tensor(crow, col, val, (2, 4))
    with pytest.raises(ValueError, match="Invariant 6"):
        PaddedCSR.from_torch_sparse_csr(sp)


def test_state_dict_topology_roundtrip_on_device(dev):
    """A receiver with another mask adopts the saved topology, including one
    rewritten on the device by SET, and then computes the same bits."""
    torch.manual_seed(0)
    a = SparseLinear(64, 32, sparsity=0.8).to(dev)
    torch.manual_seed(9)
    b = SparseLinear(64, 32, sparsity=0.8).to(dev)
    a._csr._drop_grow(max(1, int(0.3 * a.nnz)), slk._lib.SLK_GROW_RANDOM, None, 123)
    b.load_state_dict(a.state_dict())
    for name in ("values", "col_indices", "row_start", "row_nnz", "row_capacity"):
        assert torch.equal(getattr(a._csr, name), getattr(b._csr, name)), name
    assert b._csr.topology_version == a._csr.topology_version
    x = torch.randn(24, 64, device=dev)
    ya, yb = a(x), b(x)
    assert torch.equal(ya, yb)
    up = torch.randn_like(ya)
    ya.backward(up)
    yb.backward(up)
    assert torch.equal(a._values.grad, b._values.grad) and torch.equal(a.bias.grad, b.bias.grad)


@pytest.mark.parametrize("sparsity,batch", [(0.7, 1024), (0.95, 1100), (0.9, 1032)])
def test_sparse_linear_dW_through_the_default_schedules(dev, monkeypatch, sparsity, batch):
    """SparseLinear's weight gradient through the schedule the library picks
    for large layers (a segment list from _SEG_MIN_NNZ live slots at N >= 1024,
    with the block width and segment size _seg_shape gives), with the threshold
    lowered so a small layer takes it: dW is the oracle's SIMD-order dW of the
    same layer and upstream gradient, bit for bit, and dbias its row sums."""
    from sparsecore_amd import ops

    monkeypatch.setattr(ops, "_SEG_MIN_NNZ", 1000)
    torch.manual_seed(int(sparsity * 100) + batch)
    layer = SparseLinear(300, 200, sparsity=sparsity).to(dev)
    W = layer._csr
    x = torch.randn(batch, 300, device=dev)
    view = ops._sddmm_view(W, x.t().contiguous())
    want_shape = ops._seg_shape(W, 300, batch)
    assert view.seg_start is not None and (view.seg_block, view.seg_slots) == want_shape
    up = torch.randn(batch, 200, device=dev)
    layer(x).backward(up)
    c = to_oracle(W)
    ref = oracle.sddmm(c, up.t().contiguous().cpu().numpy(), x.t().contiguous().cpu().numpy())
    assert_bits_equal(layer._values.grad.cpu().numpy(), ref, "dW (segment schedule)")
    db = torch.empty(200, device=dev)
    _lib.sddmm(W._view(), up.t().contiguous(), x.t().contiguous(),
               torch.empty(W.total_capacity, device=dev), _lib.SLK_DW_SIMD, db)
    assert torch.equal(layer.bias.grad, db)
