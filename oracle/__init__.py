"""CPU oracle for the padded-CSR hot path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker (or the timed CPU baseline) — never as the thing measured or shipped.
The ``sparsecore_amd`` product never imports it.

Contents
  * ctypes bindings to ``_build/liboracle.so`` — our C restatement of the
    reference kernels (``oracle.c``), bit-exact by construction:
      spmm            csrc/kernels/spmm_avx2.cpp:123-262
      sddmm (simd)    csrc/kernels/spmm_grad_avx2.cpp:108-258
      sddmm (scalar)  csrc/kernels/spmm_grad.cpp:85-108
      dense_grad      csrc/kernels/dense_grad.cpp:57-83
      fmaf            libm's fmaf elementwise (the reference's fma), for
                      tests of the device's fma-equivalent instructions
  * ctypes bindings to ``_ref/libslref.so`` — the reference's own kernels,
    when that library was built (``make -C oracle ref``; needs the reference
    checkout, so it exists only where it was built and travels with the tree).
  * numpy restatements of the host-side algorithms:
      row_capacity        sparselab/layout.py:46-68
      from_dense          sparselab/layout.py:75-165, 172-208
      to_dense            sparselab/layout.py:262-292
      transpose_with_perm sparselab/layout.py:460-536
      refresh             sparselab/ops.py:83-94
      check_invariants    csrc/kernels/padded_csr.cpp:79-196
      rewrite_row         csrc/kernels/padded_csr.cpp:219-296
      live_abs_kth        sparselab/router.py:394-412 (global drop threshold)
      drop_grow           sparselab/router.py:414-478 (SET), :663-732 (RigL)
      splitmix_keys       SET's grow keys (our generator; see drop_grow)

How each function is pinned (see tests/test_oracle.py):
  spmm / sddmm / dense_grad — bit-exact against the reference build where it
      exists, and against float64 dense products (W_dense @ X, dY @ X^T) at
      the reference tests' tolerance everywhere.
  transpose_with_perm — to_dense(WT) == to_dense(W).T bit-exactly, the
      invariants of WT (which fix the layout uniquely), a brute-force
      per-column scan on small inputs, and the reference tests' literal cases.
  row_capacity / from_dense — the reference tests' known answers
      (capacities [3, 3, 2], starts [0, 3, 6]) and round trips.
  check_invariants — message-for-message against the reference checker.
  rewrite_row — array-for-array against the reference's rewrite_row.
  live_abs_kth — np.partition is the reference's own expression; also
      against a full sort.
  drop_grow — survivors against a literal per-row restatement of the
      reference's keep rule; RigL grows against the reference's argpartition
      choice (set equality where |G| has no ties at the cut) and its known
      answer (column 15 grown); nnz, invariants and zero-init grows;
      splitmix_keys against the generator's published first output; SET grow
      uniformity by a chi-square test over seeds.
"""

from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "_build" / "liboracle.so"
REF_LIB = HERE / "_ref" / "libslref.so"

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64 = ctypes.c_int64

_oracle = None
_ref = None


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctype)


def build(with_ref: bool | None = None) -> None:
    """Compile the oracle (and the reference build when the checkout exists)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    ref_dir = os.environ.get("REF_KERNELS", "/root/reference/csrc/kernels")
    if with_ref is None:
        with_ref = Path(ref_dir).is_dir()
    if with_ref:
        subprocess.run(["make", "-s", "-C", str(HERE), "ref", f"REF_KERNELS={ref_dir}"],
                       check=True)


def _lib():
    global _oracle
    if _oracle is None:
        if not ORACLE_LIB.exists():
            build(with_ref=False)
        lib = ctypes.CDLL(str(ORACLE_LIB))
        lib.orc_spmm.argtypes = [_i64, _i32p, _i32p, _i32p, _f32p, _f32p, _i64, _i64, _f32p,
                                 ctypes.c_int]
        for name in ("orc_sddmm_simd", "orc_sddmm_scalar"):
            getattr(lib, name).argtypes = [_i64, _i32p, _i32p, _i32p, _i64, _f32p, _f32p, _i64,
                                           _i64, _f32p, ctypes.c_int]
        lib.orc_dense_grad.argtypes = [_i64, _i64, _i64, _f32p, _f32p, _f32p, ctypes.c_int]
        lib.orc_fmaf.argtypes = [_i64, _f32p, _f32p, _f32p, _f32p]
        _oracle = lib
    return _oracle


# ───────────────────────────── CSR arrays ──────────────────────────────


class Csr:
    """Plain host arrays of a padded-CSR matrix (reference padded_csr.hpp:47-74)."""

    __slots__ = ("nrows", "ncols", "values", "col_indices", "row_start", "row_nnz",
                 "row_capacity")

    def __init__(self, nrows, ncols, values, col_indices, row_start, row_nnz, row_capacity):
        self.nrows = int(nrows)
        self.ncols = int(ncols)
        self.values = np.ascontiguousarray(values, dtype=np.float32)
        self.col_indices = np.ascontiguousarray(col_indices, dtype=np.int32)
        self.row_start = np.ascontiguousarray(row_start, dtype=np.int32)
        self.row_nnz = np.ascontiguousarray(row_nnz, dtype=np.int32)
        self.row_capacity = np.ascontiguousarray(row_capacity, dtype=np.int32)

    @property
    def total_capacity(self) -> int:
        return int(self.values.shape[0])

    @property
    def nnz(self) -> int:
        return int(self.row_nnz.astype(np.int64).sum())

    def copy(self) -> "Csr":
        return Csr(self.nrows, self.ncols, self.values.copy(), self.col_indices.copy(),
                   self.row_start.copy(), self.row_nnz.copy(), self.row_capacity.copy())


def row_capacity(row_nnz, padding_ratio: float) -> np.ndarray:
    """capacity = max(1, ceil(nnz * (1 + pr))) in float64 (layout.py:46-68)."""
    if padding_ratio < 0:
        raise ValueError(f"padding_ratio must be >= 0, got {padding_ratio}")
    grown = np.ceil(np.asarray(row_nnz, dtype=np.float64) * (1.0 + padding_ratio))
    return np.where(grown < 1.0, 1.0, grown).astype(np.int32)


def from_row_lists(nrows, ncols, cols_per_row, vals_per_row, padding_ratio=0.2) -> Csr:
    """Padded-CSR from per-row (sorted cols, values) lists (layout.py:122-165)."""
    nnz = np.array([len(c) for c in cols_per_row], dtype=np.int32)
    cap = row_capacity(nnz, padding_ratio) if nrows else np.zeros(0, np.int32)
    start = np.zeros(nrows, dtype=np.int64)
    if nrows:
        start[1:] = np.cumsum(cap[:-1], dtype=np.int64)
    total = int(cap.astype(np.int64).sum())
    values = np.zeros(total, dtype=np.float32)
    cols = np.full(total, -1, dtype=np.int32)
    for i in range(nrows):
        n = int(nnz[i])
        values[start[i]:start[i] + n] = vals_per_row[i]
        cols[start[i]:start[i] + n] = cols_per_row[i]
    return Csr(nrows, ncols, values, cols, start.astype(np.int32), nnz, cap)


def from_dense(W, threshold: float = 0.0, padding_ratio: float = 0.2) -> Csr:
    """Live entries are W != 0 after zeroing |W| <= threshold (layout.py:172-208)."""
    W = np.asarray(W, dtype=np.float32)
    if W.ndim != 2:
        raise ValueError(f"from_dense expected 2-D tensor, got {W.ndim}-D")
    if threshold > 0:
        W = np.where(np.abs(W) > threshold, W, np.float32(0))
    M, K = W.shape
    cols = [np.flatnonzero(W[i] != 0).astype(np.int32) for i in range(M)]
    vals = [W[i, c] for i, c in enumerate(cols)]
    return from_row_lists(M, K, cols, vals, padding_ratio)


def to_dense(p: Csr) -> np.ndarray:
    out = np.zeros((p.nrows, p.ncols), dtype=np.float32)
    for i in range(p.nrows):
        s, n = int(p.row_start[i]), int(p.row_nnz[i])
        out[i, p.col_indices[s:s + n]] = p.values[s:s + n]
    return out


def live_slots(p: Csr):
    """(slots, rows, cols) of every live entry in row-major order."""
    rows = np.repeat(np.arange(p.nrows, dtype=np.int64), p.row_nnz.astype(np.int64))
    offs = np.arange(rows.shape[0], dtype=np.int64)
    first = np.zeros(p.nrows, dtype=np.int64)
    if p.nrows:
        first[1:] = np.cumsum(p.row_nnz.astype(np.int64))[:-1]
    slots = p.row_start.astype(np.int64)[rows] + (offs - first[rows])
    return slots, rows, p.col_indices[slots].astype(np.int64)


def padding_slots(p: Csr) -> np.ndarray:
    mask = np.ones(p.total_capacity, dtype=bool)
    mask[live_slots(p)[0]] = False
    return np.flatnonzero(mask)


def transpose_with_perm(p: Csr, padding_ratio: float = 0.2):
    """(WT, perm) as layout.py:460-536 defines them, via a lexicographic sort.

    WT row c holds the live entries of column c ordered by source row; perm[t]
    is the W slot of WT slot t (int64, -1 on padding).
    """
    slots, rows, cols = live_slots(p)
    K, M = p.ncols, p.nrows
    nnz_t = np.bincount(cols, minlength=K).astype(np.int32) if K else np.zeros(0, np.int32)
    cap_t = row_capacity(nnz_t, padding_ratio) if K else np.zeros(0, np.int32)
    start_t = np.zeros(K, dtype=np.int64)
    if K:
        start_t[1:] = np.cumsum(cap_t[:-1], dtype=np.int64)
    total = int(cap_t.astype(np.int64).sum())
    order = np.lexsort((rows, cols))  # by column, then source row
    c_sorted = cols[order]
    group_first = np.zeros(K + 1, dtype=np.int64)
    if K:
        group_first[1:] = np.cumsum(nnz_t, dtype=np.int64)
    rank = np.arange(order.shape[0], dtype=np.int64) - group_first[c_sorted]
    dest = start_t[c_sorted] + rank
    values = np.zeros(total, dtype=np.float32)
    col_t = np.full(total, -1, dtype=np.int32)
    perm = np.full(total, -1, dtype=np.int64)
    values[dest] = p.values[slots[order]]
    col_t[dest] = rows[order].astype(np.int32)
    perm[dest] = slots[order]
    WT = Csr(K, M, values, col_t, start_t.astype(np.int32), nnz_t, cap_t)
    return WT, perm


def sub_rows(p: Csr, rows) -> tuple[Csr, np.ndarray]:
    """The matrix made of the given rows of p (each with its own capacity, in
    the order given), and for each of its slots the slot of p it came from.
    Every row's arithmetic in spmm / sddmm depends on that row alone, so the
    sub-matrix reproduces those rows of p's results at a fraction of the
    cost (used to check full-size workloads on sampled rows)."""
    rows = np.asarray(rows, dtype=np.int64)
    cap = p.row_capacity[rows].astype(np.int64)
    start = np.zeros(rows.size, dtype=np.int64)
    if rows.size:
        start[1:] = np.cumsum(cap[:-1])
    src = np.concatenate([np.arange(int(p.row_start[r]), int(p.row_start[r]) + int(c),
                                    dtype=np.int64) for r, c in zip(rows, cap)]
                         + [np.zeros(0, np.int64)])
    q = Csr(rows.size, p.ncols, p.values[src], p.col_indices[src], start.astype(np.int32),
            p.row_nnz[rows], p.row_capacity[rows])
    return q, src


def refresh(WT_values: np.ndarray, W_values: np.ndarray, perm: np.ndarray) -> np.ndarray:
    """Cache-hit value refresh (ops.py:83-94): live WT slots re-read W."""
    out = WT_values.copy()
    live = perm >= 0
    out[live] = W_values[perm[live]]
    return out


def check_invariants(nrows, ncols, values, col_indices, row_start, row_nnz,
                     row_capacity) -> str:
    """Reference check_invariants_str (padded_csr.cpp:79-196): '' or the first violation."""
    if nrows < 0 or ncols < 0:
        return f"Invariant 1 violated: shape must be non-negative, got ({nrows}, {ncols})."
    if not (len(row_start) == len(row_nnz) == len(row_capacity) == nrows):
        return (f"Metadata array length mismatch: row_start={len(row_start)}, "
                f"row_nnz={len(row_nnz)}, row_capacity={len(row_capacity)}, "
                f"expected nrows={nrows}.")
    if len(values) != len(col_indices):
        return (f"Invariant 2 violated: values ({len(values)}) and col_indices "
                f"({len(col_indices)}) must have the same length.")
    total = int(sum(int(c) for c in row_capacity))
    if len(values) != total:
        return (f"Invariant 2 violated: values.size()={len(values)} does not match "
                f"total_capacity={total} (sum of row_capacity).")
    if nrows > 0 and int(row_start[0]) != 0:
        return f"Invariant 3 violated: row_start[0] must be 0, got {int(row_start[0])}."
    for i in range(1, nrows):
        exp = int(row_start[i - 1]) + int(row_capacity[i - 1])
        if int(row_start[i]) != exp:
            return (f"Invariant 3 violated: row_start[{i}]={int(row_start[i])} should equal "
                    f"row_start[{i - 1}] + row_capacity[{i - 1}] = {exp}.")
    for i in range(nrows):
        if int(row_nnz[i]) < 0 or int(row_nnz[i]) > int(row_capacity[i]):
            return (f"Invariant 4 violated at row {i}: row_nnz={int(row_nnz[i])} must be in "
                    f"[0, {int(row_capacity[i])}].")
    for i in range(nrows):
        s, n, cap = int(row_start[i]), int(row_nnz[i]), int(row_capacity[i])
        prev = -1
        for k in range(n):
            c = int(col_indices[s + k])
            if c < 0 or c >= ncols:
                return (f"Invariant 6 violated at row {i}, slot {k}: col_indices={c} must be "
                        f"in [0, {ncols}).")
            if c <= prev:
                return (f"Invariant 6 violated at row {i}, slot {k}: col_indices={c} must be "
                        f"strictly greater than previous={prev} (live columns must be sorted "
                        f"ascending and distinct).")
            prev = c
        for k in range(n, cap):
            if int(col_indices[s + k]) != -1:
                return (f"Invariants 5+7 violated at row {i}, slot {k}: padding "
                        f"col_indices={int(col_indices[s + k])} must be -1.")
    return ""


def rewrite_row(p: Csr, row: int, cols, vals) -> Csr:
    """Reference rewrite_row (padded_csr.cpp:219-296) on a copy of p."""
    q = p.copy()
    cols = np.asarray(cols, dtype=np.int32)
    vals = np.asarray(vals, dtype=np.float32)
    s, cap = int(q.row_start[row]), int(q.row_capacity[row])
    n = cols.shape[0]
    q.col_indices[s:s + n] = cols
    q.values[s:s + n] = vals
    q.col_indices[s + n:s + cap] = -1
    q.values[s + n:s + cap] = 0.0
    q.row_nnz[row] = n
    return q


# ───────────────────────────── kernels (C) ─────────────────────────────


def live_abs_kth(p: Csr, k: int) -> np.float32:
    """k-th smallest |v| over the live slots (router.py:394-412)."""
    live = np.concatenate([p.values[s:s + n] for s, n in zip(p.row_start, p.row_nnz)]
                          + [np.zeros(0, np.float32)])
    return np.partition(np.abs(live), k - 1)[k - 1]


_GAMMA = np.uint64(0x9E3779B97F4A7C15)


def splitmix_keys(seed: int, row: int, ncols: int, cols: np.ndarray) -> np.ndarray:
    """32-bit grow keys of SET: the high half of splitmix64 output number
    row*ncols + c + 1 of the stream seeded by ``seed`` (published generator:
    Steele, Lea & Flood 2014; first output for seed 0 is 0xE220A8397B1DCDAF)."""
    with np.errstate(over="ignore"):
        idx = np.uint64(row) * np.uint64(ncols) + cols.astype(np.uint64) + np.uint64(1)
        z = np.uint64(seed & (2**64 - 1)) + idx * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return (z >> np.uint64(32)).astype(np.uint32)


def _grow_keys_rigl(g_row: np.ndarray) -> np.ndarray:
    """Smaller key = preferred: ~bits(|G|) (largest |G| first). Only taken
    for columns whose |G| is not NaN."""
    a = np.abs(g_row.astype(np.float32))
    return ~a.view(np.uint32)


def drop_grow_row(cols: np.ndarray, vals: np.ndarray, thr, rule: str, ncols: int,
                  g_row: np.ndarray | None = None, seed: int = 0, row: int = 0):
    """One row of a SET ("random") / RigL ("gradient") update: the new live
    (cols, vals), sorted by column.

    Follows the per-row loop of router.py:414-478 (SET) and :663-732 (RigL):
    keep |v| > threshold (the row's first largest |v| if none survive), grow
    n_grow = min(dropped, growable) columns outside the kept set with value 0,
    rewrite the row sorted by column. Growable: SET, every column outside the
    kept set; RigL, those whose |G| is not NaN (router.py:704-705 counts
    ``available`` as the empties with |G| > -inf), so a RigL row short of them
    shrinks. Grow choice: the n_grow smallest keys, ties to the lower column;
    keys are ~bits(|G[i]|) (RigL: largest |G| first) or
    splitmix_keys(seed, row, ...) (SET).
    """
    keep = np.abs(vals) > thr
    if not keep.any():
        keep[int(np.argmax(np.abs(vals)))] = True
    kc, kv = cols[keep], vals[keep]
    n_drop = len(cols) - int(keep.sum())
    empty = np.setdiff1d(np.arange(ncols, dtype=np.int64), kc.astype(np.int64))
    if rule == "gradient":
        empty = empty[~np.isnan(g_row[empty])]
    n_grow = min(n_drop, empty.size)
    if n_grow > 0:
        if rule == "gradient":
            keys = _grow_keys_rigl(g_row[empty])
        else:
            keys = splitmix_keys(seed, row, ncols, empty)
        order = np.lexsort((empty, keys))  # by key, then column
        grow = np.sort(empty[order[:n_grow]]).astype(np.int32)
    else:
        grow = np.zeros(0, np.int32)
    mc = np.concatenate([kc, grow])
    mv = np.concatenate([kv, np.zeros(grow.size, np.float32)])
    o = np.argsort(mc, kind="stable")
    return mc[o].astype(np.int32), mv[o].astype(np.float32)


def drop_grow(p: Csr, k_drop: int, rule: str, G: np.ndarray | None = None,
              seed: int = 0) -> Csr:
    """One SET / RigL update of every row (drop_grow_row), on a copy: the
    threshold is the k_drop-th smallest live |v| (router.py:394-412); a row
    that shrinks pads its tail with (-1, 0) and lowers its row_nnz."""
    q = p.copy()
    thr = live_abs_kth(p, k_drop)
    for i in range(p.nrows):
        s, n = int(p.row_start[i]), int(p.row_nnz[i])
        if n == 0:
            continue
        nc, nv = drop_grow_row(p.col_indices[s:s + n], p.values[s:s + n], thr, rule, p.ncols,
                               None if G is None else G[i], seed, i)
        m = nc.size
        q.col_indices[s:s + m] = nc
        q.values[s:s + m] = nv
        q.col_indices[s + m:s + n] = -1
        q.values[s + m:s + n] = 0.0
        q.row_nnz[i] = m
    return q


def spmm(p: Csr, X: np.ndarray, nthreads: int = 0) -> np.ndarray:
    X = np.ascontiguousarray(X, dtype=np.float32)
    K, N = X.shape
    Y = np.empty((p.nrows, N), dtype=np.float32)
    _lib().orc_spmm(p.nrows, _ptr(p.row_start, _i32p), _ptr(p.row_nnz, _i32p),
                    _ptr(p.col_indices, _i32p), _ptr(p.values, _f32p), _ptr(X, _f32p), K, N,
                    _ptr(Y, _f32p), nthreads)
    return Y


def sddmm(p: Csr, dY: np.ndarray, X: np.ndarray, order: str = "simd",
          nthreads: int = 0) -> np.ndarray:
    dY = np.ascontiguousarray(dY, dtype=np.float32)
    X = np.ascontiguousarray(X, dtype=np.float32)
    K, N = X.shape
    dW = np.empty(p.total_capacity, dtype=np.float32)
    fn = _lib().orc_sddmm_simd if order == "simd" else _lib().orc_sddmm_scalar
    fn(p.nrows, _ptr(p.row_start, _i32p), _ptr(p.row_nnz, _i32p), _ptr(p.col_indices, _i32p),
       p.total_capacity, _ptr(dY, _f32p), _ptr(X, _f32p), K, N, _ptr(dW, _f32p), nthreads)
    return dW


def dense_grad(dY: np.ndarray, X: np.ndarray, nthreads: int = 0) -> np.ndarray:
    dY = np.ascontiguousarray(dY, dtype=np.float32)
    X = np.ascontiguousarray(X, dtype=np.float32)
    M, N = dY.shape
    K = X.shape[0]
    G = np.empty((M, K), dtype=np.float32)
    _lib().orc_dense_grad(M, K, N, _ptr(dY, _f32p), _ptr(X, _f32p), _ptr(G, _f32p), nthreads)
    return G


def fmaf(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """Elementwise correctly rounded fmaf(a, b, c) (C libm), float32."""
    a, b, c = (np.ascontiguousarray(np.broadcast_to(v, np.broadcast(a, b, c).shape),
                                    dtype=np.float32) for v in (a, b, c))
    out = np.empty(a.shape, dtype=np.float32)
    _lib().orc_fmaf(a.size, _ptr(a, _f32p), _ptr(b, _f32p), _ptr(c, _f32p), _ptr(out, _f32p))
    return out


# ─────────────────────── the reference's own build ─────────────────────


def ref_available() -> bool:
    return REF_LIB.exists()


def _ref_lib():
    global _ref
    if _ref is None:
        lib = ctypes.CDLL(str(REF_LIB))
        lib.ref_last_error.restype = ctypes.c_char_p
        lib.ref_csr_new.restype = ctypes.c_void_p
        lib.ref_csr_new.argtypes = [_i64, _i64, _i64, _f32p, _i32p, _i32p, _i32p, _i32p]
        lib.ref_csr_free.argtypes = [ctypes.c_void_p]
        lib.ref_check_invariants.argtypes = [ctypes.c_void_p, ctypes.c_char_p, _i64]
        for name in ("ref_spmm_simd", "ref_spmm_scalar"):
            getattr(lib, name).argtypes = [ctypes.c_void_p, _f32p, _i64, _i64, _f32p]
        for name in ("ref_spmm_grad_w_simd", "ref_spmm_grad_w"):
            getattr(lib, name).argtypes = [ctypes.c_void_p, _f32p, _i64, _f32p, _i64, _f32p]
        lib.ref_dense_grad.argtypes = [_i64, _i64, _i64, _f32p, _f32p, _f32p]
        lib.ref_rewrite_row.argtypes = [ctypes.c_void_p, _i64, _i64, _i32p, _f32p]
        lib.ref_csr_arrays.argtypes = [ctypes.c_void_p, _f32p, _i32p, _i32p,
                                       ctypes.POINTER(ctypes.c_int64)]
        lib.ref_csr_values_ptr.restype = _f32p
        lib.ref_csr_values_ptr.argtypes = [ctypes.c_void_p]
        _ref = lib
    return _ref


class RefCsr:
    """A reference sparselab::PaddedCSR built from host arrays (ref_shim.cpp)."""

    def __init__(self, p: Csr):
        self.p = p
        lib = _ref_lib()
        self.h = lib.ref_csr_new(p.nrows, p.ncols, p.total_capacity, _ptr(p.values, _f32p),
                                 _ptr(p.col_indices, _i32p), _ptr(p.row_start, _i32p),
                                 _ptr(p.row_nnz, _i32p), _ptr(p.row_capacity, _i32p))
        if not self.h:
            raise RuntimeError(lib.ref_last_error().decode())

    def __del__(self):
        if getattr(self, "h", None):
            _ref_lib().ref_csr_free(self.h)
            self.h = None

    def _check(self, rc):
        if rc != 0:
            raise ValueError(_ref_lib().ref_last_error().decode())

    def check_invariants(self) -> str:
        buf = ctypes.create_string_buffer(4096)
        _ref_lib().ref_check_invariants(self.h, buf, 4096)
        return buf.value.decode()

    def spmm(self, X, kernel: str = "simd") -> np.ndarray:
        X = np.ascontiguousarray(X, dtype=np.float32)
        K, N = X.shape
        Y = np.empty((self.p.nrows, N), dtype=np.float32)
        fn = _ref_lib().ref_spmm_simd if kernel != "scalar" else _ref_lib().ref_spmm_scalar
        self._check(fn(self.h, _ptr(X, _f32p), K, N, _ptr(Y, _f32p)))
        return Y

    def sddmm(self, dY, X, kernel: str = "simd") -> np.ndarray:
        dY = np.ascontiguousarray(dY, dtype=np.float32)
        X = np.ascontiguousarray(X, dtype=np.float32)
        K, N = X.shape
        dW = np.empty(self.p.total_capacity, dtype=np.float32)
        fn = (_ref_lib().ref_spmm_grad_w_simd if kernel != "scalar"
              else _ref_lib().ref_spmm_grad_w)
        self._check(fn(self.h, _ptr(dY, _f32p), N, _ptr(X, _f32p), K, _ptr(dW, _f32p)))
        return dW

    def rewrite_row(self, row, cols, vals):
        cols = np.ascontiguousarray(cols, dtype=np.int32)
        vals = np.ascontiguousarray(vals, dtype=np.float32)
        self._check(_ref_lib().ref_rewrite_row(self.h, row, cols.shape[0], _ptr(cols, _i32p),
                                               _ptr(vals, _f32p)))

    def values_view(self) -> np.ndarray:
        """Writable numpy view of the reference object's own values buffer."""
        ptr = _ref_lib().ref_csr_values_ptr(self.h)
        return np.ctypeslib.as_array(ptr, shape=(self.p.total_capacity,))

    def spmm_into(self, X: np.ndarray, Y: np.ndarray, kernel: str = "simd") -> None:
        K, N = X.shape
        fn = _ref_lib().ref_spmm_simd if kernel != "scalar" else _ref_lib().ref_spmm_scalar
        self._check(fn(self.h, _ptr(X, _f32p), K, N, _ptr(Y, _f32p)))

    def sddmm_into(self, dY: np.ndarray, X: np.ndarray, dW: np.ndarray,
                   kernel: str = "simd") -> None:
        K, N = X.shape
        fn = (_ref_lib().ref_spmm_grad_w_simd if kernel != "scalar"
              else _ref_lib().ref_spmm_grad_w)
        self._check(fn(self.h, _ptr(dY, _f32p), N, _ptr(X, _f32p), K, _ptr(dW, _f32p)))

    def arrays(self):
        p = self.p
        values = np.empty(p.total_capacity, dtype=np.float32)
        col = np.empty(p.total_capacity, dtype=np.int32)
        nnz = np.empty(p.nrows, dtype=np.int32)
        ver = ctypes.c_int64(0)
        _ref_lib().ref_csr_arrays(self.h, _ptr(values, _f32p), _ptr(col, _i32p),
                                  _ptr(nnz, _i32p), ctypes.byref(ver))
        return values, col, nnz, int(ver.value)


def ref_dense_grad(dY, X) -> np.ndarray:
    dY = np.ascontiguousarray(dY, dtype=np.float32)
    X = np.ascontiguousarray(X, dtype=np.float32)
    M, N = dY.shape
    K = X.shape[0]
    G = np.empty((M, K), dtype=np.float32)
    if _ref_lib().ref_dense_grad(M, K, N, _ptr(dY, _f32p), _ptr(X, _f32p), _ptr(G, _f32p)):
        raise ValueError(_ref_lib().ref_last_error().decode())
    return G


# ───────────────────────── synthetic workloads ─────────────────────────


def uniform_rows(M, K, nnz_per_row, seed, sigma=0.02, padding_ratio=0.2) -> Csr:
    """Each row gets `nnz_per_row` distinct uniform columns (BASELINE config 1 shape)."""
    rng = np.random.default_rng(seed)
    cols = [np.sort(rng.choice(K, size=nnz_per_row, replace=False)).astype(np.int32)
            for _ in range(M)]
    vals = [rng.normal(0.0, sigma, size=nnz_per_row).astype(np.float32) for _ in range(M)]
    return from_row_lists(M, K, cols, vals, padding_ratio)


def bernoulli(M, K, sparsity, seed, padding_ratio=0.2, scale=1.0) -> Csr:
    """Bernoulli(1 - sparsity) mask with N(0, scale) values (SparseLinear-style)."""
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((M, K)) * scale).astype(np.float32)
    W[rng.random((M, K)) < sparsity] = 0.0
    return from_dense(W, padding_ratio=padding_ratio)


def zipf_rows(M, K, density, s, seed, sigma=0.01, padding_ratio=0.2) -> Csr:
    """Row nnz ~ c * rank^-s capped at K, total ~ density*M*K."""
    rng = np.random.default_rng(seed)
    target = int(round(density * M * K))
    ranks = np.arange(1, M + 1, dtype=np.float64) ** (-s)
    lo, hi = 0.0, float(K) * M
    for _ in range(100):  # water-filling: find c with sum(min(K, c*r^-s)) = target
        mid = 0.5 * (lo + hi)
        if np.minimum(K, mid * ranks).sum() < target:
            lo = mid
        else:
            hi = mid
    counts = np.minimum(K, np.floor(hi * ranks)).astype(np.int64)
    counts[0] += target - counts.sum()
    counts = np.minimum(counts, K)
    counts = counts[rng.permutation(M)]
    cols = [np.sort(rng.choice(K, size=int(n), replace=False)).astype(np.int32)
            for n in counts]
    vals = [rng.normal(0.0, sigma, size=int(n)).astype(np.float32) for n in counts]
    return from_row_lists(M, K, cols, vals, padding_ratio)


def dense_from_csr64(p: Csr) -> np.ndarray:
    return to_dense(p).astype(np.float64)


def allclose_ref(a, b, rtol=1e-5, atol=1e-5) -> bool:
    return bool(np.allclose(a, b, rtol=rtol, atol=atol))


def max_rel_err(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    denom = np.maximum(np.abs(b), 1e-30)
    return float(np.max(np.abs(a - b) / denom)) if a.size else 0.0


__all__ = [
    "Csr", "build", "row_capacity", "from_row_lists", "from_dense", "to_dense", "live_slots",
    "padding_slots", "transpose_with_perm", "refresh", "check_invariants", "rewrite_row",
    "spmm", "sddmm", "dense_grad", "ref_available", "RefCsr", "ref_dense_grad",
    "uniform_rows", "bernoulli", "zipf_rows", "dense_from_csr64", "allclose_ref",
    "max_rel_err", "math",
]
