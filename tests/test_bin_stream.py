"""The binned slot stream of slk_spmm's LDS-staged kernel, on the CPU: its
definition restated in numpy (tests/helpers.bin_stream), and the kernel's
traversal of it simulated (tests/helpers.bin_visit_order) — windows of 64
entries, passes over dense chunks, each row's run clipped to a pass, the
first G slots of every row before the rest. The simulation must visit every
covered row's live slots exactly once and in slot order (that order is what
makes each output element the reference's fma chain), with every index
inside its array. The device builder is compared with bin_stream on the GPU
(tests/test_gpu_bin.py)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import bin_stream, bin_visit_order


def _cases():
    yield "uniform", oracle.uniform_rows(200, 300, 15, seed=1, sigma=1.0)
    yield "zipf", oracle.zipf_rows(400, 700, 0.06, 1.1, seed=2, sigma=1.0)
    W = np.random.default_rng(3).standard_normal((40, 170)).astype(np.float32)
    W[::2] *= np.random.default_rng(4).random((20, 170)) < 0.05
    yield "dense-rows", oracle.from_dense(W)  # runs of 40-80 per chunk: several passes
    yield "empty-rows", oracle.uniform_rows(50, 90, 0, seed=5, sigma=1.0)


@pytest.mark.parametrize("G", [1, 2, 4])
@pytest.mark.parametrize("rw,h", [(8, 2), (4, 2), (2, 2), (1, 2), (8, 1), (4, 1)])
@pytest.mark.parametrize("name,c", list(_cases()), ids=[n for n, _ in _cases()])
def test_bin_traversal_visits_each_row_in_slot_order(name, c, rw, h, G):
    order = np.argsort(-c.row_nnz, kind="stable").astype(np.int32)
    mean = c.row_nnz.mean() if c.nrows else 0.0
    heavy = int(np.count_nonzero(c.row_nnz > 2 * mean))
    for first in sorted({0, heavy, min(c.nrows, 3)}):
        seen = bin_visit_order(c, first, order, rw, h, G)
        covered = order[first:] if first > 0 else np.arange(c.nrows)
        assert sorted(seen) == sorted(int(r) for r in covered)
        for r, slots in seen.items():
            s0, n = int(c.row_start[r]), int(c.row_nnz[r])
            assert slots == list(range(s0, s0 + n)), (name, first, r)


def test_bin_stream_counts_and_starts():
    c = oracle.zipf_rows(300, 500, 0.05, 1.1, seed=7, sigma=1.0)
    off, slot, words, start = bin_stream(c, 0, None, 8, 2)
    assert start[-1] == c.nnz == len(off) == len(slot)
    assert sorted(slot.tolist()) == sorted(
        s for r in range(c.nrows) for s in range(c.row_start[r], c.row_start[r] + c.row_nnz[r]))
    counts = sum(int((w >> np.uint32(8 * b)) & np.uint32(0xFF)) for w in words for b in range(4))
    assert counts == c.nnz
