"""Shared test helpers: conversions between the product PaddedCSR and the oracle."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

import oracle
from sparsecore_amd import PaddedCSR

GOLDEN = Path(__file__).resolve().parent / "golden"


def to_oracle(p: PaddedCSR) -> oracle.Csr:
    return oracle.Csr(p.nrows, p.ncols, p.values.detach().cpu().numpy(),
                      p.col_indices.cpu().numpy(), p.row_start.cpu().numpy(),
                      p.row_nnz.cpu().numpy(), p.row_capacity.cpu().numpy())


def from_oracle(c: oracle.Csr, device=None) -> PaddedCSR:
    return PaddedCSR(c.nrows, c.ncols, torch.from_numpy(c.values.copy()),
                     torch.from_numpy(c.col_indices.copy()), torch.from_numpy(c.row_start.copy()),
                     torch.from_numpy(c.row_nnz.copy()), torch.from_numpy(c.row_capacity.copy()),
                     device=device)


def make_sparse_W(M: int, K: int, sparsity: float, seed: int = 0):
    """(W_csr on CPU, W_dense) as the reference tests build them (test_spmm.py:52-69)."""
    gen = torch.Generator().manual_seed(seed)
    W = torch.randn(M, K, generator=gen, dtype=torch.float32)
    keep = torch.rand(M, K, generator=gen) >= sparsity
    W_dense = W * keep.float()
    return PaddedCSR.from_dense(W_dense), W_dense


def golden_cases():
    data = np.load(GOLDEN / "kernels.npz")
    names = sorted({k.split("/")[0] for k in data.files})
    out = {}
    for n in names:
        out[n] = {k.split("/", 1)[1]: data[k] for k in data.files if k.startswith(n + "/")}
    return out


def golden_csr(case) -> oracle.Csr:
    M, K, _ = (int(v) for v in case["shape"])
    return oracle.Csr(M, K, case["values"], case["col_indices"], case["row_start"],
                      case["row_nnz"], case["row_capacity"])


def c1_inputs():
    """BASELINE config-1 inputs regenerated from tests/golden/gen.py."""
    import json

    import gen

    meta = json.loads((GOLDEN / "c1.json").read_text())
    g = meta["gen"]
    M, K, N = g["M"], g["K"], g["N"]
    parts = gen.padded_csr(M, K, np.full(M, g["nnz_per_row"], np.int32), g["csr_seed"],
                           g["sigma"], g["padding_ratio"])
    p = oracle.Csr(M, K, *parts)
    X = gen.normalish(g["X_seed"], K * N).reshape(K, N)
    dY = gen.normalish(g["dY_seed"], M * N).reshape(M, N)
    assert gen.digest(p.values) == meta["inputs_sha256"]["values"]
    assert gen.digest(p.col_indices) == meta["inputs_sha256"]["col_indices"]
    assert gen.digest(X) == meta["inputs_sha256"]["X"]
    assert gen.digest(dY) == meta["inputs_sha256"]["dY"]
    return meta, p, X, dY


def assert_bits_equal(a, b, what: str = "") -> None:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, f"{what}: shape {a.shape} != {b.shape}"
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), b.view(np.uint32)
    diff = np.flatnonzero(a.reshape(-1) != b.reshape(-1))
    assert diff.size == 0, (f"{what}: {diff.size} of {a.size} elements differ, first at flat "
                            f"index {int(diff[0])}")


def csr_arrays_equal(a: oracle.Csr, b: oracle.Csr, what: str = "") -> None:
    assert (a.nrows, a.ncols) == (b.nrows, b.ncols), what
    for name in ("values", "col_indices", "row_start", "row_nnz", "row_capacity"):
        assert_bits_equal(getattr(a, name), getattr(b, name), f"{what}.{name}")


# ─────────────────── binned slot stream (slk_csr.bin_*) ────────────────────

BIN_WAVES = 16
BIN_CHUNK_ROWS = 80


def bin_rows(nrows: int, first: int, order, rw: int) -> np.ndarray:
    """rows[u, j] of the binned stream's units (-1 past the covered positions):
    position q = p - first goes to unit (q // (16 rw)) * 16 + q % 16, row j =
    (q // 16) % rw; rows are order[p] when first > 0, else p."""
    P = nrows - first
    units = -(-P // (BIN_WAVES * rw)) * BIN_WAVES
    rows = np.full((units, rw), -1, dtype=np.int64)
    for u in range(units):
        for j in range(rw):
            q = (u // BIN_WAVES) * BIN_WAVES * rw + u % BIN_WAVES + BIN_WAVES * j
            if q < P:
                rows[u, j] = order[first + q] if first > 0 else q
    return rows


def bin_stream(c, first: int, order, rw: int, h: int):
    """(off, slot, cnt, start) of the binned slot stream, restated from its
    definition in include/sparsecore_amd.h: per unit, chunk by chunk (chunks of
    80 / h columns), row by row, each row's slots of the chunk in slot order;
    off = (c mod kc) * h * 1024, slot = the slot index; cnt[u, ch, j] the
    counts as uint32 words (row j's byte at bits 8 (j mod 4) of word j // 4);
    start the exclusive scan of the units' slot counts."""
    kc = BIN_CHUNK_ROWS // h
    nch = -(-c.ncols // kc)
    rows = bin_rows(c.nrows, first, order, rw)
    units = rows.shape[0]
    cnt = np.zeros((units, nch, 8), dtype=np.int64)
    off, slot, start = [], [], [0]
    for u in range(units):
        runs = {}
        for j in range(rw):
            r = rows[u, j]
            if r < 0:
                continue
            s0, n = int(c.row_start[r]), int(c.row_nnz[r])
            for s in range(s0, s0 + n):
                ch = int(c.col_indices[s]) // kc
                runs.setdefault((ch, j), []).append(s)
                cnt[u, ch, j] += 1
        for key in sorted(runs):
            for s in runs[key]:
                off.append((int(c.col_indices[s]) - key[0] * kc) * h * 1024)
                slot.append(s)
        start.append(len(off))
    words = np.zeros((units, nch, 2), dtype=np.uint32)
    for j in range(8):
        words[:, :, j // 4] |= (cnt[:, :, j].astype(np.uint32) << np.uint32(8 * (j % 4)))
    return (np.array(off, dtype=np.int32), np.array(slot, dtype=np.int32),
            words.reshape(-1), np.array(start, dtype=np.int32))


def bin_visit_order(c, first: int, order, rw: int, h: int, G: int, window: int = 64):
    """The slots of each covered row in the order the binned kernel applies
    them, following its loop: per chunk, one pass per `window` entries of the
    unit's chunk run (each row's run clipped to the pass's window), in each
    pass first G slots of every row, then the rest of each row. Checks every
    index the kernel forms against its array (window positions, stream entries,
    the staged chunk's rows) and returns {row: [slots...]}."""
    off, slot, words, start = bin_stream(c, first, order, rw, h)
    kc = BIN_CHUNK_ROWS // h
    nch = -(-c.ncols // kc)
    rows = bin_rows(c.nrows, first, order, rw)
    units = rows.shape[0]
    seen = {int(r): [] for r in rows.reshape(-1) if r >= 0}
    cnt = words.reshape(units, nch, 2)
    for u in range(units):
        e = int(start[u])
        for ch in range(nch):
            nr = [int((cnt[u, ch, j // 4] >> (8 * (j % 4))) & 0xFF) for j in range(rw)]
            tot = sum(nr)
            for wb in range(0, max(tot, 1), window):
                if wb >= tot:
                    break
                rs = 0
                pj, nj = [], []
                for j in range(rw):
                    lo, hi = max(rs, wb), min(rs + nr[j], wb + window)
                    pj.append(lo - wb)
                    nj.append(max(hi - lo, 0))
                    rs += nr[j]
                visits = []
                for j in range(rw):  # pass 1
                    visits += [(j, pj[j] + t) for t in range(min(G, nj[j]))]
                for j in range(rw):  # pass 2
                    visits += [(j, pj[j] + t) for t in range(G, nj[j])]
                for j, p in visits:
                    assert 0 <= p < window
                    i = e + wb + p
                    assert start[u] <= i < start[u + 1]
                    o = int(off[i])
                    assert o % (h * 1024) == 0 and 0 <= o // (h * 1024) < kc
                    s = int(slot[i])
                    assert int(c.col_indices[s]) == ch * kc + o // (h * 1024)
                    seen[int(rows[u, j])].append(s)
            e += tot
        assert e == start[u + 1]
    return seen
