"""slk_drop_grow_noalloc: the allocation-free variant of slk_drop_grow.

Called through the C-ABI (ctypes) twice in a row — a larger matrix, then a
smaller one — for each grow rule, and checked bit for bit against
slk_drop_grow on an identical copy of the matrix (values, columns, row_nnz
and the removed-slot count), and against the oracle. The second, smaller
call runs on a scratch array that still holds the first call's contents.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from helpers import csr_arrays_equal, from_oracle, to_oracle
from sparsecore_amd import _lib

pytestmark = pytest.mark.gpu


def _threshold(W, k):
    dev = W.device
    thr = torch.empty(1, dtype=torch.float32, device=dev)
    _lib.live_abs_kth(W._view(), k,
                      torch.empty(_lib.SLK_KTH_WORKSPACE_BYTES, dtype=torch.uint8, device=dev),
                      thr)
    return thr


def _run(W, thr, rule, G, seed, noalloc):
    """One pass through the C-ABI; returns the removed-slot count."""
    lib = _lib.load()
    view = W._view()
    dev = W.device
    removed = torch.full((1,), -1, dtype=torch.int64, device=dev)
    ldg = G.stride(0) if G is not None else 0
    stream = torch.cuda.current_stream(dev).cuda_stream
    if noalloc:
        rc = lib.slk_drop_grow_noalloc(ctypes.byref(view), view.values, view.col_indices,
                                       view.row_nnz, thr.data_ptr(), rule, _lib.ptr(G), ldg,
                                       seed, removed.data_ptr(), stream)
    else:
        nbytes = int(lib.slk_drop_grow_workspace_bytes(ctypes.byref(view)))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        rc = lib.slk_drop_grow(ctypes.byref(view), view.values, view.col_indices,
                               view.row_nnz, thr.data_ptr(), rule, _lib.ptr(G), ldg, seed,
                               ws.data_ptr(), nbytes, removed.data_ptr(), stream)
    assert rc == 0, lib.slk_last_error().decode()
    torch.cuda.synchronize()
    return int(removed.item())


@pytest.mark.parametrize("rule", ["random", "gradient"])
def test_noalloc_matches_workspace_entry_point_on_two_calls(dev, rule):
    cases = [oracle.zipf_rows(3000, 2000, 0.05, 1.1, seed=21, sigma=1.0),   # larger first
             oracle.uniform_rows(40, 64, 9, seed=22, sigma=1.0)]            # then smaller
    assert cases[0].total_capacity <= _lib.DROP_GROW_NOALLOC_MAX_SLOTS
    assert cases[1].total_capacity < cases[0].total_capacity
    for n, c in enumerate(cases):
        print(f"[noalloc] rule={rule} call {n}: {c.nrows}x{c.ncols} cap={c.total_capacity}",
              flush=True)
        rng = np.random.default_rng(30 + n)
        G_np = None
        if rule == "gradient":
            G_np = rng.standard_normal((c.nrows, c.ncols)).astype(np.float32)
            if n == 1:  # NaN columns: some rows run out of growable columns and shrink
                G_np[rng.random(G_np.shape) < 0.95] = np.nan
        G = torch.from_numpy(G_np).to(dev) if G_np is not None else None
        code = _lib.SLK_GROW_GRADIENT if rule == "gradient" else _lib.SLK_GROW_RANDOM
        k = max(1, int(0.4 * c.nnz))
        Wa, Wb = from_oracle(c, dev), from_oracle(c, dev)
        thr = _threshold(Wa, k)
        removed_a = _run(Wa, thr, code, G, 1234 + n, noalloc=False)
        removed_b = _run(Wb, thr, code, G, 1234 + n, noalloc=True)
        assert removed_b == removed_a
        got_a, got_b = to_oracle(Wa), to_oracle(Wb)
        csr_arrays_equal(got_b, got_a, f"noalloc vs workspace, call {n}")
        want = oracle.drop_grow(c, k, rule, G_np, seed=1234 + n)
        csr_arrays_equal(got_b, want, f"noalloc vs oracle, call {n}")
        assert removed_b == c.nnz - want.nnz
        if rule == "gradient" and n == 1:
            assert removed_b > 0  # the shrink path ran


def test_noalloc_rejects_matrices_beyond_the_scratch(dev):
    lib = _lib.load()
    big = _lib.DROP_GROW_NOALLOC_MAX_SLOTS + 1
    # fake, never dereferenced pointers: the size check answers first
    v = _lib.CsrView(4, 6, big, 8, 8, 1, 1, 1)
    rc = lib.slk_drop_grow_noalloc(ctypes.byref(v), 8, 8, 1, 1, _lib.SLK_GROW_RANDOM, None, 0,
                                   0, 1, None)
    assert rc == _lib.SLK_EINVAL
    assert "exceeds the static scratch" in lib.slk_last_error().decode()
