"""sparsecore_amd.layout — the padded-CSR matrix, its factories and its transpose.

Drop-in for the reference's C++ ``PaddedCSR`` class (csrc/kernels/padded_csr.hpp:47-143,
exposed by csrc/bindings.cpp:596-743) together with the Python factories of
``sparselab/layout.py``. The arrays live in torch tensors, normally on the HIP
device (HBM); a matrix built on the CPU can be moved with ``.cuda()`` /
``.to(device)``. Host-side work here is setup and validation only; the
transpose used by the backward pass runs on the GPU
(``transpose_with_perm`` → the ``slk_transpose_*`` kernels).

Layout (unchanged from the reference, padded_csr.hpp:30-45):

    values[total_capacity]        float32; live slots hold weights, padding 0.0
    col_indices[total_capacity]   int32;   live slots hold their column, padding -1
    row_start[nrows]              int32;   first slot of each row
    row_nnz[nrows]                int32;   live slots per row (<= capacity)
    row_capacity[nrows]           int32;   slots reserved per row
    topology_version              int;     bumped by every rewrite_row

Within a row the first ``row_nnz`` slots are live with strictly ascending
columns and the rest are padding; rows tile ``[0, total_capacity)`` in order.
"""

from __future__ import annotations

import math
import weakref  # noqa: F401  (PaddedCSR objects are weak-referenceable)

import numpy as np
import torch

from . import _lib

__all__ = [
    "PaddedCSR",
    "from_coo",
    "from_dense",
    "from_torch_sparse_csr",
    "random",
    "to_dense",
    "transpose",
    "transpose_with_perm",
    "transposes_with_perm",
]

_I32 = torch.int32
_F32 = torch.float32
_NONE = (1 << 63) - 1  # "no violation" word of the device checker


# ─────────────────────────────────────────────────────────────────────
#  Row-capacity rule
# ─────────────────────────────────────────────────────────────────────

def _compute_row_capacity(row_nnz: np.ndarray, padding_ratio: float) -> np.ndarray:
    """capacity[i] = max(1, ceil(nnz[i] * (1 + padding_ratio))), in float64.

    Same rule as sparselab/layout.py:46-68; the device transpose applies it in
    the same float64 arithmetic (slk_transpose_count).
    """
    if padding_ratio < 0:
        raise ValueError(f"padding_ratio must be >= 0, got {padding_ratio}")
    scaled = np.ceil(np.asarray(row_nnz).astype(np.float64) * (1.0 + padding_ratio))
    return np.maximum(1, scaled).astype(np.int32)


def _as_tensor(x, dtype, device) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        t = x.detach()
        if device is not None:
            t = t.to(device)
        return t.to(dtype).contiguous()
    arr = np.asarray(x)
    if arr.dtype == object:
        arr = np.asarray(list(x))
    t = torch.from_numpy(np.ascontiguousarray(arr).astype(
        np.float32 if dtype == _F32 else np.int32))
    return t.to(device) if device is not None else t


def _wrap_i32(v: int) -> int:
    return ((v + (1 << 31)) % (1 << 32)) - (1 << 31)


# ─────────────────────────────────────────────────────────────────────
#  Invariant messages (text of csrc/kernels/padded_csr.cpp:79-196; the
#  reference tests match these substrings, so the wording is kept)
# ─────────────────────────────────────────────────────────────────────

def _msg_inv3_first(got: int) -> str:
    return f"Invariant 3 violated: row_start[0] must be 0, got {got}."


def _msg_inv3(i: int, got: int, expected: int) -> str:
    return (f"Invariant 3 violated: row_start[{i}]={got} should equal row_start[{i - 1}] + "
            f"row_capacity[{i - 1}] = {expected}.")


def _msg_inv4(i: int, nnz: int, cap: int) -> str:
    return f"Invariant 4 violated at row {i}: row_nnz={nnz} must be in [0, {cap}]."


def _msg_inv6_range(i: int, k: int, c: int, ncols: int) -> str:
    return (f"Invariant 6 violated at row {i}, slot {k}: col_indices={c} must be in "
            f"[0, {ncols}).")


def _msg_inv6_order(i: int, k: int, c: int, prev: int) -> str:
    return (f"Invariant 6 violated at row {i}, slot {k}: col_indices={c} must be strictly "
            f"greater than previous={prev} (live columns must be sorted ascending and "
            f"distinct).")


def _msg_inv57(i: int, k: int, c: int) -> str:
    return (f"Invariants 5+7 violated at row {i}, slot {k}: padding col_indices={c} "
            f"must be -1.")


def _check_shape_and_lengths(nrows, ncols, n_values, n_col, n_rs, n_nnz, n_cap) -> str:
    if nrows < 0 or ncols < 0:
        return f"Invariant 1 violated: shape must be non-negative, got ({nrows}, {ncols})."
    if not (n_rs == n_nnz == n_cap == nrows):
        return (f"Metadata array length mismatch: row_start={n_rs}, row_nnz={n_nnz}, "
                f"row_capacity={n_cap}, expected nrows={nrows}.")
    if n_values != n_col:
        return (f"Invariant 2 violated: values ({n_values}) and col_indices ({n_col}) must "
                f"have the same length.")
    return ""


def _check_host(nrows, ncols, values, col, rs, nnz, cap) -> str:
    """Vectorized host check of invariants 1-7 with the reference's first-violation order."""
    msg = _check_shape_and_lengths(nrows, ncols, values.shape[0], col.shape[0], rs.shape[0],
                                   nnz.shape[0], cap.shape[0])
    if msg:
        return msg
    rs64, nnz64, cap64 = rs.astype(np.int64), nnz.astype(np.int64), cap.astype(np.int64)
    total = int(cap64.sum())
    if values.shape[0] != total:
        return (f"Invariant 2 violated: values.size()={values.shape[0]} does not match "
                f"total_capacity={total} (sum of row_capacity).")
    if nrows == 0:
        return ""
    if rs64[0] != 0:
        return _msg_inv3_first(int(rs64[0]))
    if nrows > 1:
        expected = (rs.astype(np.int32)[:-1].astype(np.int64) + cap64[:-1])
        expected = ((expected + (1 << 31)) % (1 << 32)) - (1 << 31)
        bad = np.flatnonzero(rs64[1:] != expected)
        if bad.size:
            i = int(bad[0]) + 1
            return _msg_inv3(i, int(rs64[i]), int(expected[i - 1]))
    bad = np.flatnonzero((nnz64 < 0) | (nnz64 > cap64))
    if bad.size:
        i = int(bad[0])
        return _msg_inv4(i, int(nnz64[i]), int(cap64[i]))
    # Rows tile [0, total) now; classify every slot.
    row_of = np.repeat(np.arange(nrows, dtype=np.int64), cap64)
    pos = np.arange(total, dtype=np.int64) - rs64[row_of]
    live = pos < nnz64[row_of]
    c = col.astype(np.int64)
    prev = np.empty_like(c)
    prev[0:1] = -1
    prev[1:] = c[:-1]
    prev[pos == 0] = -1
    live_bad = live & ((c < 0) | (c >= ncols) | (c <= prev))
    pad_bad = (~live) & (c != -1)
    lb = np.flatnonzero(live_bad)
    pb = np.flatnonzero(pad_bad)
    if not lb.size and not pb.size:
        return ""
    lrow = int(row_of[lb[0]]) if lb.size else None
    prow = int(row_of[pb[0]]) if pb.size else None
    if lrow is not None and (prow is None or lrow <= prow):
        s = int(lb[0])
        i, k, cc = lrow, int(pos[s]), int(c[s])
        if cc < 0 or cc >= ncols:
            return _msg_inv6_range(i, k, cc, ncols)
        return _msg_inv6_order(i, k, cc, int(prev[s]))
    s = int(pb[0])
    return _msg_inv57(prow, int(pos[s]), int(c[s]))


# ─────────────────────────────────────────────────────────────────────
#  PaddedCSR
# ─────────────────────────────────────────────────────────────────────

# A row is "heavy" for slk_spmm's LDS-staged kernel when it holds more than
# this many times the mean row's slots (slk_csr.n_heavy_rows). Measured on the
# 16384^2 Zipf(1.1) layer at 95% sparsity, with heavy rows at 8 columns per
# lane: a bar of 1, 1.5, 2, 3, 4 and 6 x the mean gave 7.37, 7.16, 7.08, 7.11,
# 7.36 and 7.29 ms (12.6 ms unsplit); uniform layers have none.
HEAVY_ROW_FACTOR = 2.0


# A row is "dense" for slk_spmm when its live slots cover at least this share
# of the columns (slk_csr.n_dense_rows): it then runs as a dense row on the
# matrix cores (an fp32 K=1 MFMA per column, bit-equal to the slot chain),
# whose time grows with the columns, not the slots. Only matrices with at least
# DENSE_MIN_COLS columns and DENSE_MIN_ROWS such rows take it.
DENSE_ROW_FRACTION = 0.25
DENSE_MIN_COLS = 4096
DENSE_MIN_ROWS = 32


def dense_row_count(row_nnz: np.ndarray, ncols: int) -> int:
    """Rows with at least DENSE_ROW_FRACTION x ncols live slots (the head of
    the longest-rows-first order) when there are DENSE_MIN_ROWS of them and
    ncols >= DENSE_MIN_COLS, else 0."""
    if ncols < DENSE_MIN_COLS or len(row_nnz) == 0:
        return 0
    n = int(np.count_nonzero(np.asarray(row_nnz, dtype=np.float64) >= DENSE_ROW_FRACTION * ncols))
    return n if n >= DENSE_MIN_ROWS else 0


def heavy_row_count(row_nnz: np.ndarray) -> int:
    """Rows with more than HEAVY_ROW_FACTOR x the mean row_nnz: the head of the
    longest-rows-first order that slk_spmm runs as a launch of its own."""
    n = len(row_nnz)
    if n == 0:
        return 0
    mean = float(np.asarray(row_nnz, dtype=np.float64).sum()) / n
    return int(np.count_nonzero(np.asarray(row_nnz) > HEAVY_ROW_FACTOR * mean))


class PaddedCSR:
    """Sparse matrix with padded-row CSR storage (reference padded_csr.hpp:47-143).

    ``PaddedCSR(nrows, ncols)`` builds an empty zero-capacity matrix;
    ``PaddedCSR(nrows, ncols, values, col_indices, row_start, row_nnz,
    row_capacity)`` takes the five arrays (lists, numpy arrays or tensors),
    validates all invariants and raises ``ValueError`` on the first violation,
    as the reference constructor does (csrc/bindings.cpp:608-627).
    ``device=`` places the arrays (default: where tensor inputs live, else CPU).
    """

    def __init__(self, nrows, ncols, values=None, col_indices=None, row_start=None,
                 row_nnz=None, row_capacity=None, *, device=None):
        nrows = int(nrows)
        ncols = int(ncols)
        parts = (values, col_indices, row_start, row_nnz, row_capacity)
        if all(p is None for p in parts):
            if nrows < 0 or ncols < 0:
                raise ValueError(f"PaddedCSR: shape must be non-negative, got ({nrows}, {ncols})")
            dev = torch.device(device) if device is not None else torch.device("cpu")
            self._init(nrows, ncols, torch.zeros(0, dtype=_F32, device=dev),
                       torch.zeros(0, dtype=_I32, device=dev),
                       torch.zeros(nrows, dtype=_I32, device=dev),
                       torch.zeros(nrows, dtype=_I32, device=dev),
                       torch.zeros(nrows, dtype=_I32, device=dev), nnz=0)
            return
        if any(p is None for p in parts):
            raise TypeError("PaddedCSR() takes either (nrows, ncols) or all of values, "
                            "col_indices, row_start, row_nnz, row_capacity")
        if device is None:
            devs = {p.device for p in parts if isinstance(p, torch.Tensor)}
            device = devs.pop() if len(devs) == 1 else None
        v = _as_tensor(values, _F32, device)
        c = _as_tensor(col_indices, _I32, device)
        rs = _as_tensor(row_start, _I32, device)
        nz = _as_tensor(row_nnz, _I32, device)
        cp = _as_tensor(row_capacity, _I32, device)
        for t in (v, c, rs, nz, cp):
            if t.dim() != 1:
                raise ValueError("PaddedCSR arrays must be 1-D")
        self._init(nrows, ncols, v, c, rs, nz, cp, nnz=None)
        msg = self._check()
        if msg:
            raise ValueError("PaddedCSR invariant check failed: " + msg)
        self._nnz = int(nz.to(torch.int64).sum().item()) if nrows else 0

    # internal constructor: trusted arrays (kernel outputs), no validation
    @classmethod
    def _from_parts(cls, nrows, ncols, values, col, rs, nnz_t, cap_t, nnz: int,
                    topology_version: int = 0) -> "PaddedCSR":
        self = cls.__new__(cls)
        self._init(nrows, ncols, values, col, rs, nnz_t, cap_t, nnz=nnz)
        self._topology_version = int(topology_version)
        return self

    def _init(self, nrows, ncols, values, col, rs, nnz_t, cap_t, nnz):
        self._nrows = nrows
        self._ncols = ncols
        self._values = values
        self._col = col
        self._rs = rs
        self._row_nnz = nnz_t
        self._row_cap = cap_t
        self._nnz = nnz
        self._topology_version = 0
        self._cview = None
        self._order = None      # (topology_version, device row schedule, heavy rows)
        # derived views: (key, the base view they copy, view, schedule arrays)
        self._seglist = None    # key (topology_version, block_cols, seg_slots)
        self._phased = None     # key (topology_version, n_phases)
        self._binned = None     # key (topology_version, first, rw, h)
        # True when a few columns hold many of the slots (a transpose of a
        # matrix with heavy rows): its gathers already stay in cache
        self._cols_skewed = False
        self._host_rows = None  # cached numpy (row_start, row_nnz, row_capacity)
        self._heavy_hint = None  # heavy_row_count(row_nnz) when a builder counted it
        self._dense_hint = None  # dense_row_count(row_nnz, ncols) likewise

    # ─── shape and aggregates (bindings.cpp:631-660) ────────────────
    @property
    def shape(self) -> tuple[int, int]:
        return (self._nrows, self._ncols)

    @property
    def nrows(self) -> int:
        return self._nrows

    @property
    def ncols(self) -> int:
        return self._ncols

    @property
    def nnz(self) -> int:
        return self._nnz

    @property
    def total_capacity(self) -> int:
        return int(self._values.numel())

    @property
    def padding_slots(self) -> int:
        return self.total_capacity - self._nnz

    @property
    def sparsity(self) -> float:
        if self._nrows == 0 or self._ncols == 0:
            return 1.0
        return 1.0 - self._nnz / float(self._nrows * self._ncols)

    @property
    def topology_version(self) -> int:
        return self._topology_version

    @property
    def device(self) -> torch.device:
        return self._values.device

    # ─── arrays (bindings.cpp:665-687) ──────────────────────────────
    # `values` is the live weight buffer (an optimizer may update it in
    # place); the structure arrays must only change through rewrite_row.
    @property
    def values(self) -> torch.Tensor:
        return self._values

    @property
    def col_indices(self) -> torch.Tensor:
        return self._col

    @property
    def row_start(self) -> torch.Tensor:
        return self._rs

    @property
    def row_nnz(self) -> torch.Tensor:
        return self._row_nnz

    @property
    def row_capacity(self) -> torch.Tensor:
        return self._row_cap

    def _bind_values(self, t: torch.Tensor) -> None:
        """Point the matrix at another float32 buffer of the same size (aliasing)."""
        if t.dtype != _F32 or t.numel() != self._values.numel() or not t.is_contiguous():
            raise ValueError("values buffer must be a contiguous float32 tensor of "
                             "total_capacity elements")
        self._values = t
        self._cview = None

    def _on_device(self) -> bool:
        return self._values.device.type == "cuda"

    def _require_device(self, who: str) -> None:
        if not self._on_device():
            raise RuntimeError(
                f"{who}: the PaddedCSR lives on {self._values.device}; the padded-CSR kernels run "
                f"on the HIP device only — move it with .cuda() / .to('cuda')")

    # Matrices with at least this many rows get a longest-rows-first schedule
    # (slk_csr.row_order) so that skewed rows do not straggle in slk_spmm.
    _ORDER_MIN_ROWS = 2048

    def _view(self) -> _lib.CsrView:
        v = self._cview
        if v is None:
            order, n_heavy, n_dense, dws = None, 0, 0, None
            if self._nrows >= self._ORDER_MIN_ROWS and self._on_device():
                if self._order is None or self._order[0] != self._topology_version:
                    # stable: equal-length rows keep their natural order
                    heavy, dense = self._heavy_hint, self._dense_hint
                    if heavy is None or dense is None:
                        nz = self._rows_host()[1]
                        if heavy is None:
                            heavy = heavy_row_count(nz)
                        if dense is None:
                            dense = dense_row_count(nz, self._ncols)
                    ws = None
                    if dense:
                        ws = torch.empty(_lib.dense_rows_workspace_bytes(dense, self._ncols),
                                         dtype=torch.uint8, device=self._values.device)
                    self._order = (self._topology_version,
                                   torch.argsort(self._row_nnz, descending=True,
                                                 stable=True).to(_I32), heavy, dense, ws)
                order, n_heavy, n_dense, dws = self._order[1:5]
            v = _lib.CsrView(self._nrows, self._ncols, self._values.numel(),
                             _lib.ptr(self._values), _lib.ptr(self._col), _lib.ptr(self._rs),
                             _lib.ptr(self._row_nnz), _lib.ptr(self._row_cap), _lib.ptr(order),
                             n_heavy_rows=n_heavy, n_dense_rows=n_dense,
                             dense_ws=_lib.ptr(dws))
            self._cview = v
        return v

    @staticmethod
    def _derived(base: _lib.CsrView, **changes) -> _lib.CsrView:
        fields = {f: getattr(base, f) for f, _ in _lib.CsrView._fields_}
        fields.update(changes)
        return _lib.CsrView(**fields)

    def _view_segmented(self, block_cols: int, seg_slots: int,
                        skip_dense: bool = False) -> _lib.CsrView:
        """The view plus W's live slots cut into segments of at most seg_slots
        consecutive slots of one row inside one column block (slk_csr.seg_start):
        a schedule for slk_sddmm that keeps each segment's dY row in registers.
        With skip_dense (and dense rows in the view) the list leaves the dense
        rows out (slk_csr.seg_dense_rows) and slk_sddmm runs them on the
        matrix cores. Built on the device (slk_seg_list_build, six launches, no
        host read) once per topology. The cached view is rebuilt whenever the
        base view is (a values rebind, a row-schedule change), so it never
        carries a stale pointer; the segment arrays survive that as long as the
        topology does."""
        base = self._view()
        skip = int(base.n_dense_rows) if skip_dense else 0
        key = (self._topology_version, int(block_cols), int(seg_slots), skip)
        c = self._seglist
        if c is None or c[0] != key:
            arrays = _lib.seg_list_build(self._derived(base, seg_dense_rows=skip), int(block_cols),
                                         int(seg_slots), self.device)
            c = (key, None, None, arrays)
        if c[1] is not base:
            start, row, count, groups = c[3]
            view = self._derived(base, seg_start=_lib.ptr(start), seg_row=_lib.ptr(row),
                                 seg_count=_lib.ptr(count), seg_groups=_lib.ptr(groups),
                                 n_seg=int(start.numel()), seg_block=int(block_cols),
                                 seg_slots=int(seg_slots), seg_dense_rows=skip)
            c = (key, base, view, c[3])
        self._seglist = c
        return c[2]

    def _view_phased(self, n_phases: int) -> _lib.CsrView:
        """The view plus phase bounds for slk_spmm's gather kernel
        (slk_csr.phase_lo): the columns swept in n_phases launches, each row's
        chain resumed from Y, so the X rows one phase gathers fit the L2s.
        Built on the device (slk_phase_bounds_build, one launch) once per
        topology; the cached view follows the base view as above."""
        base = self._view()
        key = (self._topology_version, int(n_phases))
        c = self._phased
        if c is None or c[0] != key:
            c = (key, None, None, _lib.phase_bounds_build(base, int(n_phases), self.device))
        if c[1] is not base:
            view = self._derived(base, phase_lo=_lib.ptr(c[3]), n_phases=int(n_phases))
            c = (key, base, view, c[3])
        self._phased = c
        return c[2]

    def _bin_coverage(self) -> tuple[int, int]:
        """(first, slots): the positions a binned stream covers start at
        `first` (after the heavy rows, which the LDS kernel runs; 0 without
        them), and `slots` bounds their live slots (exact where the host row
        mirror is at hand, else nnz)."""
        base = self._view()
        first = int(base.n_heavy_rows)
        if first == 0:
            return 0, self._nnz
        if self._host_rows is None:
            return first, self._nnz
        nz = np.sort(self._host_rows[1])[::-1]
        return first, self._nnz - int(nz[:first].sum())

    def _view_binned(self, rw: int, h: int) -> _lib.CsrView:
        """The view plus the binned slot stream of slk_spmm's LDS-staged kernel
        (slk_csr.bin_*) for rw rows per wave and h column halves: the rows after
        the heavy ones (all rows without heavy ones), each wave's slots listed
        chunk by chunk and row by row. Built on the device (slk_bin_build, two
        launches, no host read) once per topology; the cached view follows the
        base view as the other schedules do."""
        base = self._view()
        first, n_bin = self._bin_coverage()
        key = (self._topology_version, first, int(rw), int(h))
        c = self._binned
        if c is None or c[0] != key:
            c = (key, None, None,
                 _lib.bin_build(base, first, int(rw), int(h), n_bin, self.device), n_bin)
        if c[1] is not base:
            off, slot, cnt, start = c[3]
            view = self._derived(base, bin_off=_lib.ptr(off), bin_slot=_lib.ptr(slot),
                                 bin_cnt=_lib.ptr(cnt), bin_start=_lib.ptr(start),
                                 bin_first=first, bin_rw=int(rw), bin_h=int(h), n_bin=c[4])
            c = (key, base, view, c[3], c[4])
        self._binned = c
        return c[2]

    def _rows_host(self):
        h = self._host_rows
        if h is None:
            h = (self._rs.cpu().numpy().copy(), self._row_nnz.cpu().numpy().copy(),
                 self._row_cap.cpu().numpy().copy())
            self._host_rows = h
        return h

    # ─── invariants (padded_csr.cpp:79-196) ─────────────────────────
    def _check(self) -> str:
        if not self._on_device():
            return _check_host(self._nrows, self._ncols, self._values.detach().numpy(),
                               self._col.numpy(), self._rs.numpy(), self._row_nnz.numpy(),
                               self._row_cap.numpy())
        return self._check_device()

    def _check_device(self) -> str:
        M, K = self._nrows, self._ncols
        msg = _check_shape_and_lengths(M, K, self._values.numel(), self._col.numel(),
                                       self._rs.numel(), self._row_nnz.numel(),
                                       self._row_cap.numel())
        if msg:
            return msg
        res = torch.empty(_lib.SLK_CHECK_WORDS, dtype=torch.int64, device=self._values.device)
        _lib.check_invariants(self._view(), self._col.numel(), res)
        w = res.cpu().tolist()
        total = w[0]
        if self._values.numel() != total:
            return (f"Invariant 2 violated: values.size()={self._values.numel()} does not "
                    f"match total_capacity={total} (sum of row_capacity).")

        def at(t, i):
            return int(t[i].item())

        if w[1] != _NONE:
            i = w[1]
            if i == 0:
                return _msg_inv3_first(at(self._rs, 0))
            return _msg_inv3(i, at(self._rs, i),
                             _wrap_i32(at(self._rs, i - 1) + at(self._row_cap, i - 1)))
        if w[2] != _NONE:
            i = w[2]
            return _msg_inv4(i, at(self._row_nnz, i), at(self._row_cap, i))
        live, pad = w[3], w[4]
        if live == _NONE and pad == _NONE:
            return ""
        if live != _NONE and (pad == _NONE or (live >> 32) <= (pad >> 32)):
            i, k = live >> 32, live & 0xFFFFFFFF
            s = at(self._rs, i) + k
            c = at(self._col, s)
            if c < 0 or c >= K:
                return _msg_inv6_range(i, k, c, K)
            return _msg_inv6_order(i, k, c, at(self._col, s - 1) if k > 0 else -1)
        i, k = pad >> 32, pad & 0xFFFFFFFF
        return _msg_inv57(i, k, at(self._col, at(self._rs, i) + k))

    def assert_invariants(self) -> None:
        """Raise ValueError describing the first violated invariant, if any."""
        msg = self._check()
        if msg:
            raise ValueError("PaddedCSR invariant check failed: " + msg)

    # ─── mutation (padded_csr.cpp:219-296, bindings.cpp:703-734) ────
    def rewrite_row(self, row_idx, new_cols, new_values) -> None:
        """Replace row ``row_idx``'s live set; trailing slots become padding.

        ``new_cols`` must be strictly ascending, distinct, inside [0, ncols) and
        no longer than the row's capacity. Bumps ``topology_version``.
        """
        cols = np.asarray(new_cols.detach().cpu() if isinstance(new_cols, torch.Tensor)
                          else new_cols)
        vals = np.asarray(new_values.detach().cpu() if isinstance(new_values, torch.Tensor)
                          else new_values)
        if cols.ndim != 1 or vals.ndim != 1:
            raise ValueError("rewrite_row: new_cols and new_values must be 1-D arrays")
        cols = cols.astype(np.int32)
        vals = vals.astype(np.float32)
        row_idx = int(row_idx)
        if row_idx < 0 or row_idx >= self._nrows:
            raise ValueError(f"rewrite_row: row_idx={row_idx} out of range [0, {self._nrows}).")
        if cols.shape[0] != vals.shape[0]:
            raise ValueError(f"rewrite_row: new_cols.size()={cols.shape[0]} must equal "
                             f"new_values.size()={vals.shape[0]}")
        rs, nz, cp = self._rows_host()
        cap = int(cp[row_idx])
        n = int(cols.shape[0])
        if n > cap:
            raise ValueError(f"rewrite_row: row {row_idx} has capacity {cap} but got {n} new "
                             f"entries.")
        prev = -1
        for k in range(n):
            c = int(cols[k])
            if c < 0 or c >= self._ncols:
                raise ValueError(f"rewrite_row: new_cols[{k}]={c} out of range "
                                 f"[0, {self._ncols}).")
            if c <= prev:
                raise ValueError(f"rewrite_row: new_cols must be strictly ascending, got {prev} "
                                 f"followed by {c} at position {k}.")
            prev = c
        full_c = np.full(cap, -1, dtype=np.int32)
        full_v = np.zeros(cap, dtype=np.float32)
        full_c[:n] = cols
        full_v[:n] = vals
        base = int(rs[row_idx])
        with torch.no_grad():
            self._col[base:base + cap].copy_(torch.from_numpy(full_c))
            self._values[base:base + cap].copy_(torch.from_numpy(full_v))
            self._row_nnz[row_idx:row_idx + 1].fill_(n)
        self._nnz += n - int(nz[row_idx])
        nz[row_idx] = n
        self._topology_version += 1
        self._cview = None  # the row schedule depends on row_nnz
        self._heavy_hint = None
        self._dense_hint = None

    def _drop_grow(self, k_drop: int, rule: int, G: torch.Tensor | None = None,
                   seed: int = 0) -> None:
        """One SET / RigL drop-and-grow pass over every row, on the device.

        Drops the live slots with |v| <= the k_drop-th smallest live |v| (each
        row keeps at least its largest slot), regrows as many columns per row
        (RigL: largest |G| first, never a column whose |G| is NaN; SET: a
        uniform random subset keyed by ``seed``), zero-initialised, rows
        rewritten sorted by column. Capacities do not change; row nnz changes
        only where a RigL row runs out of non-NaN columns to grow into, which
        costs one device read. Bumps ``topology_version``.
        """
        self._require_device("drop_grow")
        if not 1 <= k_drop <= self._nnz:
            raise ValueError(f"drop_grow: k_drop={k_drop} outside [1, nnz={self._nnz}]")
        dev = self._values.device
        view = self._view()
        ws = torch.empty(_lib.SLK_KTH_WORKSPACE_BYTES, dtype=torch.uint8, device=dev)
        thr = torch.empty(1, dtype=_F32, device=dev)
        _lib.live_abs_kth(view, k_drop, ws, thr)
        stage = torch.empty(_lib.drop_grow_workspace_bytes(view), dtype=torch.uint8, device=dev)
        removed = torch.empty(1, dtype=torch.int64, device=dev)
        _lib.drop_grow(view, thr, rule, G, seed, stage, removed)
        self._after_topology_pass(int(removed.item()) if rule == _lib.SLK_GROW_GRADIENT else 0)

    # Above this many undecided columns per empty column, the exact dense
    # gradient (every element recomputed in one GEMM-shaped pass) is cheaper
    # than recomputing the undecided ones one by one.
    _RIGL_EXACT_SHARE = 0.125

    def _rigl_update(self, k_drop: int, dY: torch.Tensor, X: torch.Tensor,
                     then=None) -> None:
        """One RigL drop-and-grow pass, grows ranked by |G|, G = dY·Xᵀ with the
        reference's dense_grad arithmetic, without computing G everywhere.

        dY (nrows x N) and X (ncols x N) are row-major float32 on the device.
        G' = dY·Xᵀ runs on the matrix cores; its certified error bound decides
        most empty columns, and only the undecided ones are computed exactly
        (slk_rigl_norms, slk_dense_grad_approx, slk_rigl_count,
        slk_rigl_finish). The rows come out exactly as
        ``_drop_grow(k_drop, SLK_GROW_GRADIENT, dense_grad(dY, X))`` writes
        them. One device read: the undecided count with the removed slots.

        ``then`` (optional) is called once the rewrite is queued, before that
        read, to queue more device work on the rewritten rows: it returns
        (device int64 tensor, finish); the tensor is read together with the
        RigL counts, and finish(host values) runs after the bookkeeping if the
        certified path rewrote the rows, else (the exact path taken instead)
        finish(None).
        """
        self._require_device("rigl")
        if not 1 <= k_drop <= self._nnz:
            raise ValueError(f"drop_grow: k_drop={k_drop} outside [1, nnz={self._nnz}]")
        M, K = self._nrows, self._ncols
        if dY.shape[0] != M or X.shape[0] != K or dY.shape[1] != X.shape[1]:
            raise ValueError(f"rigl: dY {tuple(dY.shape)} and X {tuple(X.shape)} do not match "
                             f"W ({M}, {K})")
        dev = self._values.device
        dY = dY.to(_F32).contiguous()
        X = X.to(_F32).contiguous()
        view = self._view()
        ws = torch.empty(_lib.SLK_KTH_WORKSPACE_BYTES, dtype=torch.uint8, device=dev)
        thr = torch.empty(1, dtype=_F32, device=dev)
        _lib.live_abs_kth(view, k_drop, ws, thr)
        nrm_dY = torch.empty(M, dtype=_F32, device=dev)
        nrm_X = torch.empty(K, dtype=_F32, device=dev)
        _lib.rigl_norms(dY, X, nrm_dY, nrm_X)
        Gp = torch.empty(M, K, dtype=_F32, device=dev)
        Gc = torch.empty(M, K, dtype=torch.uint8, device=dev)
        _lib.dense_grad_approx(dY, X, Gp, Gc)
        info = torch.empty(M * _lib.RIGL_INFO_BYTES, dtype=torch.uint8, device=dev)
        amb_off = torch.empty(2 * M + 1, dtype=torch.int64, device=dev)
        counts = torch.empty(2, dtype=torch.int64, device=dev)  # undecided, removed
        total, removed = counts[0:1], counts[1:2]
        # the undecided-column lists, sized for the most the certified path
        # takes (the count writes them where it holds rows in registers)
        cap = max(1, int(self._RIGL_EXACT_SHARE * max(1, M * K - self._nnz)))
        amb = torch.empty(8 * cap, dtype=torch.uint8, device=dev)
        stage = torch.empty(_lib.drop_grow_workspace_bytes(view), dtype=torch.uint8, device=dev)
        _lib.rigl_count(view, thr, Gp, Gc, nrm_dY, nrm_X, dY.shape[1], info, amb_off, total,
                        amb, stage)
        # queued right behind the count: its exact step covers the lists'
        # capacity and reads the count on the device, and its row rewrite
        # leaves every row alone when the count exceeds that capacity, so the
        # undecided count and the removed slots are read together afterwards
        _lib.rigl_finish(view, thr, Gp, Gc, nrm_dY, nrm_X, dY, X, info, amb_off, amb, stage,
                         removed)
        more, finish = then() if then is not None else (None, None)
        host = (torch.cat([counts, more]) if more is not None else counts).tolist()
        n_amb, lost = host[0], host[1]
        if n_amb > cap:
            del Gp, Gc, amb, stage
            from .ops import dense_grad
            self._drop_grow(k_drop, _lib.SLK_GROW_GRADIENT, dense_grad(dY, X))
            if finish is not None:
                finish(None)
            return
        self._after_topology_pass(int(lost))
        if finish is not None:
            finish(host[2:])

    def _after_topology_pass(self, lost: int) -> None:
        """Bookkeeping after a drop/grow pass: the version bump, and where rows
        shrank (RigL rows short of non-NaN columns), the host nnz and the row
        schedule."""
        self._topology_version += 1
        if lost:
            self._nnz -= lost
            self._host_rows = None
            self._heavy_hint = None
            self._dense_hint = None
            self._cview = None
            self._order = None
        elif self._order is not None:
            # row_nnz is unchanged, so the cached row schedule stays valid
            self._order = (self._topology_version,) + self._order[1:]

    # ─── device movement ───────────────────────────────────────────
    def to(self, device) -> "PaddedCSR":
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        if device == self._values.device:
            return self
        out = PaddedCSR._from_parts(self._nrows, self._ncols, self._values.to(device),
                                    self._col.to(device), self._rs.to(device),
                                    self._row_nnz.to(device), self._row_cap.to(device),
                                    self._nnz, self._topology_version)
        out._host_rows = self._host_rows
        return out

    def cuda(self, device=None) -> "PaddedCSR":
        if device is None:
            device = torch.device("cuda")
        elif isinstance(device, int):
            device = torch.device("cuda", device)
        return self.to(device)

    def cpu(self) -> "PaddedCSR":
        return self.to("cpu")

    def __repr__(self) -> str:
        return (f"PaddedCSR(nrows={self._nrows}, ncols={self._ncols}, nnz={self._nnz}, "
                f"capacity={self.total_capacity})")

    # factories and conversions are attached below (as the reference attaches
    # them in sparselab/__init__.py:56-60)


# ─────────────────────────────────────────────────────────────────────
#  Factories (sparselab/layout.py:75-255)
# ─────────────────────────────────────────────────────────────────────

def _build_from_rows(nrows, ncols, crow, col, vals, padding_ratio, device) -> PaddedCSR:
    row_nnz = np.diff(crow).astype(np.int32)
    cap = _compute_row_capacity(row_nnz, padding_ratio) if nrows else np.zeros(0, np.int32)
    start = np.zeros(nrows, dtype=np.int64)
    if nrows > 1:
        start[1:] = np.cumsum(cap[:-1].astype(np.int64))
    total = int(cap.astype(np.int64).sum())
    values = np.zeros(total, dtype=np.float32)
    cols = np.full(total, -1, dtype=np.int32)
    n = int(crow[-1]) if nrows else 0
    if n:
        row_of = np.repeat(np.arange(nrows, dtype=np.int64), row_nnz.astype(np.int64))
        dest = start[row_of] + (np.arange(n, dtype=np.int64) - crow[:-1].astype(np.int64)[row_of])
        values[dest] = vals[:n]
        cols[dest] = col[:n]
    p = PaddedCSR(nrows, ncols, torch.from_numpy(values), torch.from_numpy(cols),
                  torch.from_numpy(start.astype(np.int32)), torch.from_numpy(row_nnz),
                  torch.from_numpy(cap))
    return p.to(device) if device is not None else p


def _build_from_rows_device(nrows, ncols, crow, col, vals, padding_ratio, dev) -> PaddedCSR:
    """_build_from_rows with torch ops on the HIP device: the padded arrays are
    laid out where the input lives and validated by the device checker, so a
    matrix built from GPU tensors never passes through host memory."""
    crow = crow.to(dev, torch.int64)
    n = int(crow[-1]) if nrows else 0
    row_nnz = crow[1:] - crow[:-1]
    cap = torch.clamp(torch.ceil(row_nnz.to(torch.float64) * (1.0 + padding_ratio)),
                      min=1.0).to(torch.int64)
    start = torch.cumsum(cap, 0) - cap
    total = int(cap.sum()) if nrows else 0
    v = torch.zeros(total, dtype=_F32, device=dev)
    c = torch.full((total,), -1, dtype=_I32, device=dev)
    if n:
        rows = torch.repeat_interleave(torch.arange(nrows, device=dev), row_nnz, output_size=n)
        dest = start[rows] + (torch.arange(n, device=dev) - crow[:-1][rows])
        v[dest] = vals[:n].to(dev, _F32)
        c[dest] = col[:n].to(dev, _I32)
    return PaddedCSR(nrows, ncols, v, c, start.to(_I32), row_nnz.to(_I32), cap.to(_I32))


def from_torch_sparse_csr(csr: torch.Tensor, *, padding_ratio: float = 0.2,
                          device=None) -> PaddedCSR:
    """PaddedCSR from a ``torch.sparse_csr`` tensor (layout.py:75-165).

    Each row's entries are copied in the order given and the constructor's
    invariant check rejects unsorted or repeated columns, as the reference
    does. The result lives on ``device`` (default: the input's device); a
    HIP-resident input is converted on the device.
    """
    if csr.layout != torch.sparse_csr:
        raise ValueError(f"from_torch_sparse_csr expected layout=torch.sparse_csr, "
                         f"got layout={csr.layout}")
    if csr.dim() != 2:
        raise ValueError(f"from_torch_sparse_csr expected 2-D tensor, got {csr.dim()}-D")
    if padding_ratio < 0:
        raise ValueError(f"padding_ratio must be >= 0, got {padding_ratio}")
    nrows, ncols = csr.size()
    target = torch.device(device) if device is not None else csr.device
    if csr.device.type == "cuda" and target.type == "cuda":
        return _build_from_rows_device(int(nrows), int(ncols), csr.crow_indices(),
                                       csr.col_indices(), csr.values().detach(), padding_ratio,
                                       target)
    crow = csr.crow_indices().contiguous().cpu().numpy().astype(np.int64)
    col = csr.col_indices().contiguous().cpu().numpy().astype(np.int32)
    vals = csr.values().detach().contiguous().cpu().numpy().astype(np.float32)
    return _build_from_rows(int(nrows), int(ncols), crow, col, vals, padding_ratio, target)


def from_dense(W: torch.Tensor, *, threshold: float = 0.0, padding_ratio: float = 0.2,
               device=None) -> PaddedCSR:
    """PaddedCSR holding the entries of ``W`` with |W| > threshold (layout.py:172-208).

    Built on the device when ``W`` and the target device are HIP devices."""
    if W.dim() != 2:
        raise ValueError(f"from_dense expected 2-D tensor, got {W.dim()}-D")
    if padding_ratio < 0:
        raise ValueError(f"padding_ratio must be >= 0, got {padding_ratio}")
    target = torch.device(device) if device is not None else W.device
    if W.device.type == "cuda" and target.type == "cuda":
        # on the device: row-major nonzeros, the entries W.to_sparse_csr() keeps
        Wf = W.detach().to(device=target, dtype=_F32)
        if threshold > 0:
            Wf = torch.where(Wf.abs() > threshold, Wf, torch.zeros_like(Wf))
        nrows, ncols = Wf.shape
        rows, cols = torch.nonzero(Wf != 0, as_tuple=True)
        crow = torch.zeros(nrows + 1, dtype=torch.int64, device=target)
        if nrows:
            crow[1:] = torch.cumsum(torch.bincount(rows, minlength=nrows), 0)
        return _build_from_rows_device(nrows, ncols, crow, cols, Wf[rows, cols], padding_ratio,
                                       target)
    W_np = W.detach().to(dtype=_F32).cpu().contiguous().numpy()
    if threshold > 0:
        W_np = np.where(np.abs(W_np) > threshold, W_np, np.float32(0.0))
    nrows, ncols = W_np.shape
    # Row-major nonzeros, i.e. what W.to_sparse_csr() stores (entries != 0).
    rows, cols = np.nonzero(W_np != 0)
    crow = np.zeros(nrows + 1, dtype=np.int64)
    if nrows:
        crow[1:] = np.cumsum(np.bincount(rows, minlength=nrows))
    return _build_from_rows(nrows, ncols, crow, cols.astype(np.int32), W_np[rows, cols],
                            padding_ratio, target)


def random(nrows: int, ncols: int, *, sparsity: float, padding_ratio: float = 0.2,
           seed: int | None = None, device=None) -> PaddedCSR:
    """Random pattern at the given sparsity with N(0, 1) values (layout.py:215-255).

    Draws from a CPU torch.Generator in the reference's order (randn values,
    then the rand keep-mask), so a seed selects the same matrix as there.
    """
    if not 0.0 <= sparsity < 1.0:
        raise ValueError(f"sparsity must be in [0, 1), got {sparsity}")
    gen = torch.Generator()
    if seed is not None:
        gen.manual_seed(seed)
    W = torch.randn(nrows, ncols, generator=gen, dtype=_F32)
    keep = torch.rand(nrows, ncols, generator=gen) < (1.0 - sparsity)
    W = W * keep.float()
    return from_dense(W, threshold=0.0, padding_ratio=padding_ratio, device=device)


def from_coo(rows: torch.Tensor, cols: torch.Tensor, values: torch.Tensor, shape,
             *, padding_ratio: float = 0.2, device=None) -> PaddedCSR:
    """PaddedCSR from coordinate triples, built where the inputs live (GPU or CPU).

    Entries are ordered by (row, column); a repeated (row, column) raises
    ValueError. Capacities follow the float64 rule of layout.py:46-68. The
    arrays are validated with the same invariant checker as the constructor
    (on the device for device inputs), so a GPU-built matrix never leaves HBM.
    """
    if padding_ratio < 0:
        raise ValueError(f"padding_ratio must be >= 0, got {padding_ratio}")
    M, K = (int(s) for s in shape)
    dev = torch.device(device) if device is not None else values.device
    rows = rows.to(dev, torch.int64).reshape(-1)
    cols = cols.to(dev, torch.int64).reshape(-1)
    values = values.detach().to(dev, _F32).reshape(-1)
    n = rows.numel()
    if cols.numel() != n or values.numel() != n:
        raise ValueError("from_coo: rows, cols and values must have the same length")
    if n and (int(rows.min()) < 0 or int(rows.max()) >= M or int(cols.min()) < 0
              or int(cols.max()) >= K):
        raise ValueError(f"from_coo: coordinates out of range for shape ({M}, {K})")
    key = rows * max(K, 1) + cols
    order = torch.argsort(key)
    key, rows, cols, values = key[order], rows[order], cols[order], values[order]
    if n > 1 and bool((key[1:] == key[:-1]).any()):
        raise ValueError("from_coo: repeated (row, column) entry")
    row_nnz = torch.bincount(rows, minlength=M) if M else torch.zeros(0, dtype=torch.int64,
                                                                      device=dev)
    cap = torch.clamp(torch.ceil(row_nnz.to(torch.float64) * (1.0 + padding_ratio)),
                      min=1.0).to(torch.int64)
    start = torch.cumsum(cap, 0) - cap
    total = int(cap.sum()) if M else 0
    first = torch.cumsum(row_nnz, 0) - row_nnz
    dest = start[rows] + (torch.arange(n, device=dev) - first[rows])
    v = torch.zeros(total, dtype=_F32, device=dev)
    c = torch.full((total,), -1, dtype=_I32, device=dev)
    v[dest] = values
    c[dest] = cols.to(_I32)
    p = PaddedCSR(M, K, v, c, start.to(_I32), row_nnz.to(_I32), cap.to(_I32))
    return p


def _live_slots(p: PaddedCSR):
    """(rows, slots) of every live entry, in row-major order, on p's device."""
    dev = p.device
    n = p.nnz
    nnz64 = p.row_nnz.to(torch.int64)
    rows = torch.repeat_interleave(torch.arange(p.nrows, device=dev), nnz64, output_size=n)
    first = torch.cumsum(nnz64, 0) - nnz64
    offs = torch.arange(n, device=dev) - first[rows]
    slots = p.row_start.to(torch.int64)[rows] + offs
    return rows, slots


def to_dense(p: PaddedCSR) -> torch.Tensor:
    """Dense float32 copy of p on p's device (layout.py:262-292)."""
    dense = torch.zeros(p.nrows, p.ncols, dtype=_F32, device=p.device)
    if p.nnz:
        rows, slots = _live_slots(p)
        dense[rows, p.col_indices[slots].to(torch.int64)] = p.values[slots]
    return dense


# ─────────────────────────────────────────────────────────────────────
#  Transpose (layout.py:307-536) — on the HIP device
# ─────────────────────────────────────────────────────────────────────

def _capacity_bound(nnz: int, rows: int, padding_ratio: float) -> int:
    """An upper bound of the total capacity of `rows` rows holding `nnz` live
    slots under the capacity rule max(1, ceil(n * fl(1 + padding_ratio)))
    (float64): each row's capacity is at most n·(1 + padding_ratio)·(1 +
    2^-53) + 2, so the arrays can be sized before the exact total is read."""
    scaled = float(nnz) * (1.0 + padding_ratio) * (1.0 + 1e-15)
    return int(np.ceil(scaled)) + 2 * int(rows)


def transpose_with_perm(p: PaddedCSR, *, padding_ratio: float = 0.2):
    """(WT, perm): the transpose of p and, for each WT slot, the W slot it copies.

    WT is ncols x nrows with capacities max(1, ceil(nnz*(1+padding_ratio))),
    each row listing its source rows in ascending order; perm is int64 with -1
    on padding (layout.py:460-536). Built on the GPU by a counting sort
    (slk_transpose_count / slk_transpose_fill). The slot arrays are sized by
    a bound of the WT capacity, so the fill is queued right behind the count;
    the one device->host read of the exact capacity comes after it, and the
    arrays are trimmed to it (views, no copy).
    """
    staged = _transpose_queue(p, padding_ratio, p.nnz)
    return _transpose_take(p, staged, staged["counts"].tolist(), p.nnz)


def _transpose_queue(p: PaddedCSR, padding_ratio: float, nnz_bound: int) -> dict:
    """Queues transpose_with_perm's device work for p: the count, the fill
    (into arrays sized by a capacity bound from nnz_bound, at least p's live
    slots, when the bound fits int32) and the row hints. `counts` (int64
    capacity, heavy rows, dense rows) is for the caller to read, alone or
    with other device values, and to hand to _transpose_take."""
    if padding_ratio < 0:
        raise ValueError(f"padding_ratio must be >= 0, got {padding_ratio}")
    p._require_device("transpose")
    dev = p.device
    M, K = p.nrows, p.ncols
    view = p._view()
    ws = torch.empty(_lib.transpose_workspace_bytes(view), dtype=torch.uint8, device=dev)
    rs_t = torch.empty(K, dtype=_I32, device=dev)
    nnz_t = torch.empty(K, dtype=_I32, device=dev)
    cap_t = torch.empty(K, dtype=_I32, device=dev)
    counts = torch.empty(3, dtype=torch.int64, device=dev)  # capacity, heavy, dense rows
    _lib.transpose_count(view, padding_ratio, ws, rs_t, nnz_t, cap_t, counts[0:1])
    bound = _capacity_bound(nnz_bound, K, padding_ratio)
    filled = None
    if bound <= np.iinfo(np.int32).max:  # fill first, read the exact capacity after it
        filled = (torch.empty(bound, dtype=_F32, device=dev),
                  torch.empty(bound, dtype=_I32, device=dev),
                  torch.empty(bound, dtype=torch.int64, device=dev))
        _lib.transpose_fill(view, ws, rs_t, nnz_t, cap_t, bound, *filled)
    _count_rows(nnz_t, nnz_bound, M, counts[1:3])
    return {"view": view, "ws": ws, "rs_t": rs_t, "nnz_t": nnz_t, "cap_t": cap_t,
            "counts": counts, "filled": filled, "nnz_bound": nnz_bound}


def _transpose_take(p: PaddedCSR, staged: dict, host_counts, nnz: int):
    """(WT, perm) from _transpose_queue's work and its counts read on the host;
    nnz = p's live slots. Hints counted against another bound than nnz are
    dropped (WT recounts them from its rows when it needs them)."""
    capT, heavy, dense = (int(x) for x in host_counts)
    if capT > np.iinfo(np.int32).max:
        raise ValueError(f"transpose: capacity {capT} exceeds the int32 slot range")
    dev = p.device
    if staged["filled"] is not None:
        val_t, col_t, perm = (a[:capT] for a in staged["filled"])
    else:
        val_t = torch.empty(capT, dtype=_F32, device=dev)
        col_t = torch.empty(capT, dtype=_I32, device=dev)
        perm = torch.empty(capT, dtype=torch.int64, device=dev)
        _lib.transpose_fill(staged["view"], staged["ws"], staged["rs_t"], staged["nnz_t"],
                            staged["cap_t"], capT, val_t, col_t, perm)
    WT = PaddedCSR._from_parts(p.ncols, p.nrows, val_t, col_t, staged["rs_t"],
                               staged["nnz_t"], staged["cap_t"], nnz)
    exact = staged["nnz_bound"] == nnz
    WT._heavy_hint = heavy if exact else None
    WT._dense_hint = dense if exact else None
    WT._cols_skewed = staged["view"].n_heavy_rows > 0  # WT's columns are p's rows
    return WT, perm


def _count_rows(nnz_t: torch.Tensor, nnz: int, ncols: int, out: torch.Tensor) -> None:
    """out[0] = heavy_row_count and out[1] = dense_row_count of a WT whose
    row_nnz is nnz_t (total nnz, ncols columns), counted on the device (read
    with the capacity, no extra host sync)."""
    n = nnz_t.numel()
    bar = HEAVY_ROW_FACTOR * (float(nnz) / n) if n else 0.0  # heavy_row_count's float64 bar
    dense_bar = DENSE_ROW_FRACTION * ncols if ncols >= DENSE_MIN_COLS else float("inf")
    _lib.row_hints(nnz_t, bar, dense_bar, DENSE_MIN_ROWS, out)


def transposes_with_perm(ps, *, padding_ratio: float = 0.2):
    """[(WT, perm)] for several matrices, as transpose_with_perm gives them one
    by one, with a single device->host read: every counting pass is queued
    first, then the WT capacities are read together, then every fill."""
    if padding_ratio < 0:
        raise ValueError(f"padding_ratio must be >= 0, got {padding_ratio}")
    ps = list(ps)
    if not ps:
        return []
    for p in ps:
        p._require_device("transpose")
    dev = ps[0].device
    if any(p.device != dev for p in ps):
        raise ValueError("transposes_with_perm: all matrices must be on one device")
    n = len(ps)
    caps = torch.empty(3 * n, dtype=torch.int64, device=dev)  # capacities, heavy, dense counts
    staged = []
    for i, p in enumerate(ps):
        view = p._view()
        K = p.ncols
        ws = torch.empty(_lib.transpose_workspace_bytes(view), dtype=torch.uint8, device=dev)
        rs_t = torch.empty(K, dtype=_I32, device=dev)
        nnz_t = torch.empty(K, dtype=_I32, device=dev)
        cap_t = torch.empty(K, dtype=_I32, device=dev)
        _lib.transpose_count(view, padding_ratio, ws, rs_t, nnz_t, cap_t, caps[i:i + 1])
        if K >= PaddedCSR._ORDER_MIN_ROWS:  # only scheduled views use the counts
            _count_rows(nnz_t, p.nnz, p.nrows, caps[n + 2 * i:n + 2 * i + 2])
        else:
            caps[n + 2 * i:n + 2 * i + 2].zero_()
        # the fill right behind the count, into arrays sized by a bound of
        # the capacity (as transpose_with_perm)
        bound = _capacity_bound(p.nnz, K, padding_ratio)
        filled = None
        if bound <= np.iinfo(np.int32).max:
            filled = (torch.empty(bound, dtype=_F32, device=dev),
                      torch.empty(bound, dtype=_I32, device=dev),
                      torch.empty(bound, dtype=torch.int64, device=dev))
            _lib.transpose_fill(view, ws, rs_t, nnz_t, cap_t, bound, *filled)
        staged.append((view, ws, rs_t, nnz_t, cap_t, filled))
    host = caps.tolist()
    out = []
    for p, capT, heavy, dense, (view, ws, rs_t, nnz_t, cap_t, filled) in zip(
            ps, host[:n], host[n::2], host[n + 1::2], staged):
        if capT > np.iinfo(np.int32).max:
            raise ValueError(f"transpose: capacity {capT} exceeds the int32 slot range")
        if filled is not None:
            val_t, col_t, perm = (a[:capT] for a in filled)
        else:
            val_t = torch.empty(capT, dtype=_F32, device=dev)
            col_t = torch.empty(capT, dtype=_I32, device=dev)
            perm = torch.empty(capT, dtype=torch.int64, device=dev)
            _lib.transpose_fill(view, ws, rs_t, nnz_t, cap_t, capT, val_t, col_t, perm)
        WT = PaddedCSR._from_parts(p.ncols, p.nrows, val_t, col_t, rs_t, nnz_t, cap_t, p.nnz)
        WT._heavy_hint = heavy
        WT._dense_hint = dense
        WT._cols_skewed = view.n_heavy_rows > 0  # WT's columns are p's rows
        out.append((WT, perm))
    return out


def transpose(p: PaddedCSR, *, padding_ratio: float = 0.2) -> PaddedCSR:
    """The transpose of p as a new PaddedCSR (layout.py:307-434)."""
    return transpose_with_perm(p, padding_ratio=padding_ratio)[0]


PaddedCSR.from_coo = staticmethod(from_coo)
PaddedCSR.from_dense = staticmethod(from_dense)
PaddedCSR.from_torch_sparse_csr = staticmethod(from_torch_sparse_csr)
PaddedCSR.random = staticmethod(random)
PaddedCSR.to_dense = to_dense
PaddedCSR.transpose = transpose

del math
