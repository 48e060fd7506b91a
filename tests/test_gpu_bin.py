"""GPU parity of slk_spmm's binned-stream kernel (slk_csr.bin_*) and of the
stream's device builder (slk_bin_build).

The builder's arrays equal the stream's numpy restatement
(tests/helpers.bin_stream) entry for entry; the kernel, forced onto every
rows-per-wave x halves x read-ahead variant, gives the oracle's bits on
shapes that reach its edges: partial row blocks and column tiles, K not a
multiple of the chunk, rows dense enough that a wave's chunk takes several
64-entry passes, empty rows, heavy rows on the LDS kernel beside the binned
rest (one grid, and two launches when the rest is small), bias, and values
changed after the stream was built (read through the slot index).
Bar: bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from helpers import assert_bits_equal, bin_stream, from_oracle
from sparsecore_amd import _lib, ops

pytestmark = pytest.mark.gpu

SHAPES = [(8, 2), (4, 2), (2, 2), (1, 2), (8, 1), (4, 1)]


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _dense_rows(M, K, seed, frac=0.5):
    W = np.random.default_rng(seed).standard_normal((M, K)).astype(np.float32)
    W[::2] *= np.random.default_rng(seed + 1).random((-(-M // 2), K)) < 0.05
    W[1::2] *= np.random.default_rng(seed + 2).random((M // 2, K)) < frac
    return oracle.from_dense(W)


@pytest.mark.parametrize("rw,h", SHAPES)
@pytest.mark.parametrize("kind", ["uniform", "zipf", "dense"])
def test_bin_build_matches_the_restatement(dev, rw, h, kind):
    print(f"[bin build] {kind} rw={rw} h={h}", flush=True)
    if kind == "uniform":
        c = oracle.uniform_rows(300, 500, 30, seed=rw + h, sigma=1.0)
    elif kind == "zipf":
        c = oracle.zipf_rows(2500, 700, 0.04, 1.1, seed=rw * h, sigma=1.0)
    else:
        c = _dense_rows(100, 250, seed=rw)
    W = from_oracle(c, dev)
    first, n_bin = W._bin_coverage()
    v = W._view_binned(rw, h)
    order = v.row_order
    order_np = W._order[1].cpu().numpy() if W._order is not None else None
    assert (first > 0) == (kind == "zipf")
    off, slot, cnt, start = W._binned[3]
    want = bin_stream(c, first, order_np, rw, h)
    assert int(start[-1].item()) == len(want[0]) == n_bin
    assert_bits_equal(off.cpu().numpy()[:n_bin], want[0], "bin_off")
    assert_bits_equal(slot.cpu().numpy()[:n_bin], want[1], "bin_slot")
    assert_bits_equal(cnt.cpu().numpy().view(np.uint32)[:len(want[2])], want[2], "bin_cnt")
    assert_bits_equal(start.cpu().numpy(), want[3], "bin_start")
    assert order is not None or first == 0


@pytest.mark.parametrize("G", [1, 2, 4])
@pytest.mark.parametrize("rw,h", SHAPES)
@pytest.mark.parametrize("M,K,N,kind", [
    (63, 127, 1024, "uniform"), (300, 1000, 1032, "uniform"), (130, 5000, 1040, "uniform"),
    (100, 250, 1024, "dense"), (2600, 700, 1280, "zipf"), (40, 90, 1024, "empty")])
def test_bin_spmm_bit_exact(dev, tune, rw, h, G, M, K, N, kind):
    tune(bin_shape=(rw, h))
    tune(spmm_g=G)
    print(f"[bin spmm] rw={rw} h={h} G={G} {M}x{K} N={N} {kind}", flush=True)
    seed = M + K + N + rw * 10 + h
    if kind == "uniform":
        c = oracle.uniform_rows(M, K, max(1, K // 20), seed=seed, sigma=1.0)
    elif kind == "dense":
        c = _dense_rows(M, K, seed)
    elif kind == "zipf":
        c = oracle.zipf_rows(M, K, 0.05, 1.1, seed=seed, sigma=1.0)
    else:
        c = oracle.uniform_rows(M, K, 0, seed=seed, sigma=1.0)
    rng = np.random.default_rng(seed)
    X_np = rng.standard_normal((K, N)).astype(np.float32)
    b_np = rng.standard_normal(M).astype(np.float32)
    W = from_oracle(c, dev)
    view = ops._spmm_view(W, _t(X_np, dev))
    assert view.bin_off is not None and view.bin_rw == rw and view.bin_h == h
    assert (view.bin_first > 0) == (kind == "zipf")
    X = _t(X_np, dev)
    want = oracle.spmm(c, X_np)
    Y = torch.full((M, N), float("nan"), device=dev)
    _lib.spmm(view, X, Y)
    assert_bits_equal(Y.cpu().numpy(), want, "Y")
    _lib.spmm(view, X, Y, _t(b_np, dev))
    assert_bits_equal(Y.cpu().numpy(), want + b_np[:, None], "Y+bias")


@pytest.mark.parametrize("first", [1, 1748, 2047])
def test_bin_heavy_rows_with_a_small_rest(dev, first):
    """Heavy rows (the head of the longest-first order) on the LDS kernel beside
    the binned rest, for split points where the rest fills fewer than 8
    workgroups (two launches) and more (one grid)."""
    c = oracle.zipf_rows(2048, 700, 0.05, 1.1, seed=11, sigma=1.0)
    X_np = np.random.default_rng(11).standard_normal((700, 1024)).astype(np.float32)
    W = from_oracle(c, dev)
    base = W._view()
    assert base.row_order is not None
    order = W._order[1].cpu().numpy()
    n_bin = int(c.row_nnz[order[first:]].sum())
    off, slot, cnt, start = _lib.bin_build(base, first, 8, 2, n_bin, dev)
    view = W._derived(base, bin_off=_lib.ptr(off), bin_slot=_lib.ptr(slot),
                      bin_cnt=_lib.ptr(cnt), bin_start=_lib.ptr(start), bin_first=first,
                      bin_rw=8, bin_h=2, n_bin=n_bin)
    print(f"[bin split] first={first} rest blocks={-(-(2048 - first) // 128) * 2}", flush=True)
    Y = torch.full((2048, 1024), float("nan"), device=dev)
    _lib.spmm(view, _t(X_np, dev), Y)
    assert_bits_equal(Y.cpu().numpy(), oracle.spmm(c, X_np), "Y")


def test_bin_stream_reads_current_values(dev, tune):
    """The stream holds slot indices, not values: after the values change in
    place (an optimizer step), the cached stream gives the new values' bits."""
    tune(bin_shape=(8, 2))
    c = oracle.uniform_rows(400, 600, 40, seed=12, sigma=1.0)
    X_np = np.random.default_rng(12).standard_normal((600, 1024)).astype(np.float32)
    W = from_oracle(c, dev)
    X = _t(X_np, dev)
    Y0 = ops._launch_spmm(W, X)
    assert_bits_equal(Y0.cpu().numpy(), oracle.spmm(c, X_np), "Y before")
    with torch.no_grad():
        W.values.mul_(-0.5).add_(0.125)
    c.values[:] = W.values.cpu().numpy()
    assert W._binned is not None
    Y1 = ops._launch_spmm(W, X)
    assert_bits_equal(Y1.cpu().numpy(), oracle.spmm(c, X_np), "Y after the values changed")


def test_bin_is_ignored_where_it_cannot_run(dev, tune):
    """A binned view with unaligned X, or with the stream switched off, takes
    the other kernels: same bits."""
    tune(bin_shape=(4, 2))
    c = oracle.uniform_rows(200, 300, 20, seed=13, sigma=1.0)
    rng = np.random.default_rng(13)
    X_np = rng.standard_normal((300, 1024)).astype(np.float32)
    W = from_oracle(c, dev)
    want = oracle.spmm(c, X_np)
    Xbuf = torch.empty(300 * 1024 + 1, device=dev)
    Xbuf[1:].copy_(_t(X_np, dev).reshape(-1))
    Xu = Xbuf[1:].view(300, 1024)
    view = ops._spmm_view(W, Xu)
    assert view.bin_off is not None
    Y = torch.empty(200, 1024, device=dev)
    _lib.spmm(view, Xu, Y)
    assert_bits_equal(Y.cpu().numpy(), want, "Y (unaligned X)")
    tune(spmm_bin=0)
    _lib.spmm(view, _t(X_np, dev), Y)
    assert_bits_equal(Y.cpu().numpy(), want, "Y (stream switched off)")
