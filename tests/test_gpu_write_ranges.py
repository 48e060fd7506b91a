"""Every entry point the 10M char-GPT (C3) training step calls writes inside
its outputs and nowhere else, at that step's layer shapes (N = 8192 tokens).

Each output is the middle of a larger buffer whose two guard zones (64 Ki
elements each) hold a byte pattern; after the call the guard zones must still
hold it, and every input (X, dY, the matrix's arrays) must be unchanged. The
schedules are the launchers' own at these sizes (row order, segment list,
phase bounds where chosen), built with guarded arrays too. A narrow layer
(<= 64 rows) covers the token-major forward and the one-launch backward.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

import oracle
from helpers import from_oracle
from sparsecore_amd import _lib, ops

pytestmark = pytest.mark.gpu

GUARD = 1 << 16
PATTERN = 0xA5
N_TOKENS = 8192

C3_LAYERS = [("qkv", 1152, 384, 0.7), ("o", 384, 384, 0.7), ("up", 1536, 384, 0.9),
             ("down", 384, 1536, 0.9)]


class Guarded:
    """A device tensor of n elements with guard zones on both sides."""

    def __init__(self, n: int, dtype, dev):
        self.n = n
        self.buf = torch.empty(n + 2 * GUARD, dtype=dtype, device=dev)
        self.buf.view(torch.uint8).fill_(PATTERN)
        self.t = self.buf[GUARD:GUARD + n]

    def check(self, what: str) -> None:
        b = self.buf.view(torch.uint8)
        es = self.buf.element_size()
        lo, hi = b[:GUARD * es], b[(GUARD + self.n) * es:]
        bad_lo = int((lo != PATTERN).sum())
        bad_hi = int((hi != PATTERN).sum())
        assert bad_lo == 0 and bad_hi == 0, (
            f"{what}: {bad_lo} bytes written below and {bad_hi} above the output")


def _snapshot(*ts):
    return [t.clone() for t in ts]


def _unchanged(before, after, what):
    for i, (a, b) in enumerate(zip(before, after)):
        assert torch.equal(a, b), f"{what}: input {i} was modified"


def _matrix_arrays(W):
    return [W.values, W.col_indices, W.row_start, W.row_nnz, W.row_capacity]


def _guarded_seg_view(W, base, block_cols, seg_slots, dev, guards):
    lib = _lib.load()
    n = max(int(lib.slk_seg_list_capacity(ctypes.byref(base), block_cols, seg_slots)),
            _lib.SEG_GROUP)
    arrs = [Guarded(n, torch.int32, dev) for _ in range(3)]
    groups = Guarded(1, torch.int32, dev)
    nbytes = int(lib.slk_seg_list_workspace_bytes(ctypes.byref(base), block_cols))
    ws = Guarded(max(nbytes, 1), torch.uint8, dev)
    rc = lib.slk_seg_list_build(ctypes.byref(base), block_cols, seg_slots, ws.t.data_ptr(),
                                nbytes, arrs[0].t.data_ptr(), arrs[1].t.data_ptr(),
                                arrs[2].t.data_ptr(), n, groups.t.data_ptr(),
                                _lib.stream_of(groups.t))
    assert rc == 0, _lib.load().slk_last_error()
    guards += [("seg_start", arrs[0]), ("seg_row", arrs[1]), ("seg_count", arrs[2]),
               ("seg_groups", groups), ("seg workspace", ws)]
    return W._derived(base, seg_start=arrs[0].t.data_ptr(), seg_row=arrs[1].t.data_ptr(),
                      seg_count=arrs[2].t.data_ptr(), seg_groups=groups.t.data_ptr(),
                      n_seg=n, seg_block=block_cols, seg_slots=seg_slots)


def _guarded_phase_view(W, base, n_phases, dev, guards):
    lo = Guarded(max(1, base.nrows * (n_phases + 1)), torch.int32, dev)
    rc = _lib.load().slk_phase_bounds_build(ctypes.byref(base), n_phases, lo.t.data_ptr(),
                                            _lib.stream_of(lo.t))
    assert rc == 0
    guards.append(("phase_lo", lo))
    return W._derived(base, phase_lo=lo.t.data_ptr(), n_phases=n_phases)


def _spmm_view(W, X, dev, guards):
    """The view ops' launcher would use, its schedule arrays guarded."""
    v = ops._spmm_view(W, X)
    base = W._view()
    if v.n_phases > 1:
        return _guarded_phase_view(W, base, int(v.n_phases), dev, guards)
    return base


def _sddmm_view(W, X, dev, guards):
    v = ops._sddmm_view(W, X)
    base = W._view()
    if v.n_seg:
        return _guarded_seg_view(W, base, int(v.seg_block), int(v.seg_slots), dev, guards)
    return base


def _transpose_guarded(W, dev, guards):
    """slk_transpose_count / slk_transpose_fill into guarded arrays; returns
    (WT as a PaddedCSR over the guarded arrays, perm)."""
    view = W._view()
    K, M = W.ncols, W.nrows
    ws = Guarded(_lib.transpose_workspace_bytes(view), torch.uint8, dev)
    rs_t, nnz_t, cap_t = (Guarded(K, torch.int32, dev) for _ in range(3))
    capT_dev = Guarded(1, torch.int64, dev)
    _lib.transpose_count(view, 0.2, ws.t, rs_t.t, nnz_t.t, cap_t.t, capT_dev.t)
    capT = int(capT_dev.t.item())
    val_t = Guarded(capT, torch.float32, dev)
    col_t = Guarded(capT, torch.int32, dev)
    perm = Guarded(capT, torch.int64, dev)
    _lib.transpose_fill(view, ws.t, rs_t.t, nnz_t.t, cap_t.t, capT, val_t.t, col_t.t, perm.t)
    guards += [("transpose workspace", ws), ("WT row_start", rs_t), ("WT row_nnz", nnz_t),
               ("WT row_capacity", cap_t), ("capT", capT_dev), ("WT values", val_t),
               ("WT col_indices", col_t), ("perm", perm)]
    from sparsecore_amd.layout import PaddedCSR
    WT = PaddedCSR._from_parts(K, M, val_t.t, col_t.t, rs_t.t, nnz_t.t, cap_t.t, W.nnz)
    return WT, perm.t


@pytest.mark.parametrize("layer", C3_LAYERS, ids=[l[0] for l in C3_LAYERS])
def test_c3_step_entry_points_write_inside_their_outputs(dev, layer):
    tag, M, K, sp = layer
    seed = 700 + [l[0] for l in C3_LAYERS].index(tag)
    W = from_oracle(oracle.bernoulli(M, K, sp, seed=seed, scale=0.05), dev)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    Xt = torch.randn(N_TOKENS, K, generator=g, device=dev)   # token-major layer input
    dY = torch.randn(M, N_TOKENS, generator=g, device=dev)
    bias = torch.randn(M, generator=g, device=dev)
    print(f"[write ranges c3 {tag}] {M}x{K} nnz={W.nnz} N={N_TOKENS}", flush=True)
    inputs = [Xt, dY, bias] + _matrix_arrays(W)
    before = _snapshot(*inputs)
    guards: list = []

    # the layout copy of the input (x_flat.t().contiguous())
    X = Guarded(K * N_TOKENS, torch.float32, dev)
    _lib.transpose_dense(Xt, X.t.view(K, N_TOKENS))
    guards.append(("transpose_dense dst", X))
    Xc = X.t.view(K, N_TOKENS)
    torch.cuda.synchronize()
    assert torch.equal(Xc, Xt.t().contiguous())

    # forward with the fused bias
    Y = Guarded(M * N_TOKENS, torch.float32, dev)
    _lib.spmm(_spmm_view(W, Xc, dev, guards), Xc, Y.t.view(M, N_TOKENS), bias)
    guards.append(("Y", Y))

    # dW and dbias in one launch
    dW = Guarded(W.total_capacity, torch.float32, dev)
    dbias = Guarded(M, torch.float32, dev)
    _lib.sddmm(_sddmm_view(W, Xc, dev, guards), dY, Xc, dW.t, _lib.SLK_DW_SIMD, dbias.t)
    guards += [("dW", dW), ("dbias", dbias)]

    # transpose rebuild, refresh and dX on WT
    WT, perm = _transpose_guarded(W, dev, guards)
    _lib.transpose_refresh(W.values, perm, WT.values)
    dX = Guarded(K * N_TOKENS, torch.float32, dev)
    _lib.spmm(_spmm_view(WT, dY, dev, guards), dY, dX.t.view(K, N_TOKENS))
    guards.append(("dX", dX))

    # the invariant check's result words
    words = Guarded(5, torch.int64, dev)
    _lib.check_invariants(W._view(), W.total_capacity, words.t)
    guards.append(("invariant words", words))
    torch.cuda.synchronize()

    for what, gz in guards:
        gz.check(f"c3 {tag}: {what}")
    _unchanged(before, inputs, f"c3 {tag}")
    # and the guarded calls computed what the package computes
    assert torch.equal(Y.t.view(M, N_TOKENS), ops._launch_spmm(W, Xc, bias))
    assert torch.equal(dX.t.view(K, N_TOKENS), ops._launch_spmm(ops._cached_transpose(W), dY))


def test_narrow_layer_entry_points_write_inside_their_outputs(dev):
    """slk_spmm_t and slk_backward_narrow (a layer of 10 rows over 512
    columns at 90%, N = 8192)."""
    M, K = 10, 512
    W = from_oracle(oracle.bernoulli(M, K, 0.9, seed=77, scale=0.05), dev)
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    X = torch.randn(K, N_TOKENS, generator=g, device=dev)
    dYt = torch.randn(N_TOKENS, M, generator=g, device=dev)
    bias = torch.randn(M, generator=g, device=dev)
    inputs = [X, dYt, bias] + _matrix_arrays(W)
    before = _snapshot(*inputs)
    Yt = Guarded(N_TOKENS * M, torch.float32, dev)
    _lib.spmm_t(W._view(), X, Yt.t.view(N_TOKENS, M), bias)
    dW = Guarded(W.total_capacity, torch.float32, dev)
    dbias = Guarded(M, torch.float32, dev)
    dX = Guarded(K * N_TOKENS, torch.float32, dev)
    _lib.backward_narrow(W._view(), dYt, X, dW.t, dbias.t, dX.t.view(K, N_TOKENS),
                         _lib.SLK_DW_SIMD)
    torch.cuda.synchronize()
    for what, gz in (("Yt", Yt), ("dW", dW), ("dbias", dbias), ("dX", dX)):
        gz.check(f"narrow: {what}")
    _unchanged(before, inputs, "narrow")
