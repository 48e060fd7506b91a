"""ctypes binding of ``libsparsecore_amd.so`` (C-ABI: include/sparsecore_amd.h).

This module is the only place that talks to the native library. It replaces
the reference's pybind11 module ``sparselab._core`` (csrc/bindings.cpp) for
the hot path. Every wrapper takes torch tensors that already live on a HIP
device, passes their raw device pointers plus torch's current stream, and
maps a non-zero status to ``ValueError`` (bad arguments, as the reference
raises) or ``RuntimeError`` (HIP failure).

There is no CPU fallback: if the library is missing, importing the package
still works (so the host-side API and its error paths stay usable), but every
kernel call raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libsparsecore_amd.so"
ABI_VERSION = 16

SLK_OK, SLK_EINVAL, SLK_EDEVICE = 0, 1, 2
SLK_DW_SIMD, SLK_DW_SCALAR = 0, 1
SLK_CHECK_WORDS = 5
SLK_KTH_WORKSPACE_BYTES = 8448
SLK_GROW_RANDOM, SLK_GROW_GRADIENT = 0, 1

# Every symbol include/sparsecore_amd.h declares.
EXPORTS = (
    "slk_last_error",
    "slk_abi_version",
    "slk_spmm",
    "slk_spmm_bias",
    "slk_sddmm",
    "slk_sddmm_bias",
    "slk_transpose_workspace_bytes",
    "slk_transpose_count",
    "slk_transpose_fill",
    "slk_transpose_refresh",
    "slk_row_hints",
    "slk_check_invariants",
    "slk_live_abs_kth",
    "slk_drop_grow_workspace_bytes",
    "slk_drop_grow",
    "slk_dense_grad",
    "slk_transpose_dense",
    "slk_spmm_t",
    "slk_backward_narrow",
    "slk_backward_fused",
    "slk_seg_list_capacity",
    "slk_seg_list_workspace_bytes",
    "slk_seg_list_build",
    "slk_phase_bounds_build",
    "slk_set_tuning",
    "slk_drop_grow_noalloc",
    "slk_rigl_norms",
    "slk_dense_grad_approx_workspace_bytes",
    "slk_dense_grad_approx",
    "slk_rigl_bound_factor",
    "slk_rigl_partial_factor",
    "slk_rigl_count",
    "slk_rigl_finish",
    "slk_bin_sizes",
    "slk_bin_build",
    "slk_rigl_mfma_probe",
    "slk_dense_rows_workspace_bytes",
    "slk_dense_mfma_probe",
)

RIGL_INFO_BYTES = 32  # per row, slk_rigl_count's info

DROP_GROW_NOALLOC_MAX_SLOTS = 1 << 21  # SLK_DROP_GROW_NOALLOC_MAX_SLOTS

# Kernel-choice overrides (slk_set_tuning): knob numbers of enum slk_tune_knob.
TUNE_KNOBS = {"spmm_kernel": 0, "spmm_h": 1, "spmm_rw": 2, "spmm_split": 3, "spmm_vec": 4,
              "sddmm_g": 5, "seg_lean": 6, "seg_group": 7, "transpose_tile": 8, "spmm_bin": 9,
              "spmm_g": 10, "rigl_tile": 11, "dense_rows": 12, "transpose_radix": 13}

BIN_MAX_CHUNKS = 960  # SLK_BIN_MAX_CHUNKS

SEG_GROUP = 128  # SLK_SEG_GROUP

NARROW_MAX_ROWS = 64        # SLK_NARROW_MAX_ROWS
NARROW_MAX_CAPACITY = 8192  # SLK_NARROW_MAX_CAPACITY


class CsrView(ctypes.Structure):
    """Mirror of ``slk_csr`` (include/sparsecore_amd.h)."""

    _fields_ = [
        ("nrows", ctypes.c_int64),
        ("ncols", ctypes.c_int64),
        ("total_capacity", ctypes.c_int64),
        ("values", ctypes.c_void_p),
        ("col_indices", ctypes.c_void_p),
        ("row_start", ctypes.c_void_p),
        ("row_nnz", ctypes.c_void_p),
        ("row_capacity", ctypes.c_void_p),
        ("row_order", ctypes.c_void_p),
        ("n_heavy_rows", ctypes.c_int64),
        ("seg_start", ctypes.c_void_p),
        ("seg_row", ctypes.c_void_p),
        ("seg_count", ctypes.c_void_p),
        ("seg_groups", ctypes.c_void_p),
        ("n_seg", ctypes.c_int64),
        ("seg_block", ctypes.c_int64),
        ("seg_slots", ctypes.c_int64),
        ("phase_lo", ctypes.c_void_p),
        ("n_phases", ctypes.c_int64),
        ("bin_off", ctypes.c_void_p),
        ("bin_slot", ctypes.c_void_p),
        ("bin_cnt", ctypes.c_void_p),
        ("bin_start", ctypes.c_void_p),
        ("bin_first", ctypes.c_int64),
        ("bin_rw", ctypes.c_int64),
        ("bin_h", ctypes.c_int64),
        ("n_bin", ctypes.c_int64),
        ("n_dense_rows", ctypes.c_int64),
        ("dense_ws", ctypes.c_void_p),
        ("seg_dense_rows", ctypes.c_int64),
    ]


_lib = None
_load_error: str | None = None

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_csrp = ctypes.POINTER(CsrView)


def _declare(lib) -> None:
    lib.slk_last_error.restype = ctypes.c_char_p
    lib.slk_last_error.argtypes = []
    lib.slk_abi_version.restype = ctypes.c_int
    lib.slk_spmm.argtypes = [_csrp, _vp, _i64, _i64, _vp, _vp]
    lib.slk_spmm_bias.argtypes = [_csrp, _vp, _i64, _i64, _vp, _vp, _vp]
    lib.slk_sddmm.argtypes = [_csrp, _vp, _i64, _vp, _i64, _i64, _vp, ctypes.c_int, _vp]
    lib.slk_sddmm_bias.argtypes = [_csrp, _vp, _i64, _vp, _i64, _i64, _vp, _vp, ctypes.c_int, _vp]
    lib.slk_transpose_workspace_bytes.restype = _i64
    lib.slk_transpose_workspace_bytes.argtypes = [_csrp]
    lib.slk_transpose_count.argtypes = [_csrp, ctypes.c_double, _vp, _i64, _vp, _vp, _vp, _vp,
                                        _vp]
    lib.slk_transpose_fill.argtypes = [_csrp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp]
    lib.slk_transpose_refresh.argtypes = [_vp, _i64, _vp, _i64, _vp, _vp]
    lib.slk_row_hints.argtypes = [_vp, _i64, ctypes.c_double, ctypes.c_double, _i64, _vp, _vp]
    lib.slk_check_invariants.argtypes = [_csrp, _i64, _vp, _vp]
    lib.slk_live_abs_kth.argtypes = [_csrp, _i64, _vp, _i64, _vp, _vp]
    lib.slk_drop_grow_workspace_bytes.restype = _i64
    lib.slk_drop_grow_workspace_bytes.argtypes = [_csrp]
    lib.slk_drop_grow.argtypes = [_csrp, _vp, _vp, _vp, _vp, ctypes.c_int, _vp, _i64,
                                  ctypes.c_uint64, _vp, _i64, _vp, _vp]
    lib.slk_dense_grad.argtypes = [_vp, _vp, _i64, _i64, _i64, ctypes.c_int, _vp, _vp]
    lib.slk_transpose_dense.argtypes = [_vp, _i64, _i64, _i64, _vp, _vp]
    lib.slk_spmm_t.argtypes = [_csrp, _vp, _i64, _i64, _vp, _vp, _vp]
    lib.slk_backward_fused.argtypes = [_csrp, _csrp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp]
    lib.slk_backward_narrow.argtypes = [_csrp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, ctypes.c_int,
                                        _vp]
    lib.slk_dense_mfma_probe.argtypes = [_vp, _vp, _vp, _vp, _i64, _vp]
    lib.slk_dense_rows_workspace_bytes.restype = _i64
    lib.slk_dense_rows_workspace_bytes.argtypes = [_i64, _i64]
    lib.slk_seg_list_capacity.restype = _i64
    lib.slk_seg_list_capacity.argtypes = [_csrp, _i64, _i64]
    lib.slk_seg_list_workspace_bytes.restype = _i64
    lib.slk_seg_list_workspace_bytes.argtypes = [_csrp, _i64]
    lib.slk_seg_list_build.argtypes = [_csrp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp,
                                       _vp]
    lib.slk_phase_bounds_build.argtypes = [_csrp, _i64, _vp, _vp]
    lib.slk_set_tuning.argtypes = [ctypes.c_int, _i64]
    lib.slk_rigl_norms.argtypes = [_vp, _i64, _vp, _i64, _i64, _vp, _vp, _vp]
    lib.slk_dense_grad_approx_workspace_bytes.restype = _i64
    lib.slk_dense_grad_approx_workspace_bytes.argtypes = [_i64, _i64, _i64]
    lib.slk_dense_grad_approx.argtypes = [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp]
    lib.slk_rigl_bound_factor.restype = ctypes.c_double
    lib.slk_rigl_bound_factor.argtypes = [_i64]
    lib.slk_rigl_partial_factor.restype = ctypes.c_double
    lib.slk_rigl_partial_factor.argtypes = [_i64]
    lib.slk_rigl_count.argtypes = [_csrp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp,
                                   _vp, _i64, _vp, _i64, _vp]
    lib.slk_rigl_finish.argtypes = [_csrp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp,
                                    _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp]
    lib.slk_drop_grow_noalloc.argtypes = [_csrp, _vp, _vp, _vp, _vp, ctypes.c_int, _vp, _i64,
                                          ctypes.c_uint64, _vp, _vp]
    lib.slk_bin_sizes.argtypes = [_csrp, _i64, _i64, _i64, ctypes.POINTER(_i64),
                                  ctypes.POINTER(_i64)]
    lib.slk_bin_build.argtypes = [_csrp, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp]
    lib.slk_rigl_mfma_probe.argtypes = [_vp, _vp, _vp, _vp, _i64, _vp]
    sized = ("slk_last_error", "slk_abi_version", "slk_transpose_workspace_bytes",
             "slk_drop_grow_workspace_bytes", "slk_rigl_bound_factor", "slk_rigl_partial_factor",
             "slk_dense_grad_approx_workspace_bytes",
             "slk_seg_list_capacity", "slk_seg_list_workspace_bytes")
    for name in EXPORTS:
        if name not in sized:
            getattr(lib, name).restype = ctypes.c_int


def load(path: str | os.PathLike | None = None):
    """Load (once) and return the native library; raises RuntimeError if absent."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        _load_error = (f"sparsecore_amd: native library {p} is not built. Build it with "
                       f"`python -m sparsecore_amd.build` (hipcc, gfx950). There is no CPU "
                       f"fallback for the padded-CSR kernels.")
        raise RuntimeError(_load_error)
    # torch is imported first (module import above), so the HIP runtime torch
    # loaded is the one this library binds to (same soname).
    lib = ctypes.CDLL(str(p))
    _declare(lib)
    ver = lib.slk_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"sparsecore_amd: library ABI {ver} != expected {ABI_VERSION}; "
                           f"rebuild with `python -m sparsecore_amd.build`")
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


def _raise(rc: int) -> None:
    msg = _lib.slk_last_error().decode(errors="replace")
    if rc == SLK_EINVAL:
        raise ValueError(msg)
    raise RuntimeError(msg or f"sparsecore_amd: native call failed with status {rc}")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None or t.numel() == 0 else t.data_ptr()


def spmm(view: CsrView, X: torch.Tensor, Y: torch.Tensor,
         bias: torch.Tensor | None = None) -> None:
    """Y = W·X, plus bias[i] on row i when a (float32, contiguous) bias is given."""
    lib = load()
    if bias is None:
        rc = lib.slk_spmm(ctypes.byref(view), ptr(X), X.shape[0], X.shape[1], ptr(Y),
                          stream_of(Y))
    else:
        rc = lib.slk_spmm_bias(ctypes.byref(view), ptr(X), X.shape[0], X.shape[1], ptr(bias),
                               ptr(Y), stream_of(Y))
    if rc:
        _raise(rc)


def sddmm(view: CsrView, dY: torch.Tensor, X: torch.Tensor, dW: torch.Tensor,
          order: int, dbias: torch.Tensor | None = None) -> None:
    """dW on the live slots; with ``dbias`` also its row sums of dY (same launch)."""
    lib = load()
    if dbias is None:
        rc = lib.slk_sddmm(ctypes.byref(view), ptr(dY), dY.shape[0], ptr(X), X.shape[0],
                           X.shape[1], ptr(dW), order, stream_of(dW))
    else:
        rc = lib.slk_sddmm_bias(ctypes.byref(view), ptr(dY), dY.shape[0], ptr(X), X.shape[0],
                                X.shape[1], ptr(dW), ptr(dbias), order, stream_of(dbias))
    if rc:
        _raise(rc)


def transpose_workspace_bytes(view: CsrView) -> int:
    return int(load().slk_transpose_workspace_bytes(ctypes.byref(view)))


def transpose_count(view: CsrView, padding_ratio: float, ws: torch.Tensor,
                    rs_t: torch.Tensor, nnz_t: torch.Tensor, cap_t: torch.Tensor,
                    capT_dev: torch.Tensor) -> None:
    lib = load()
    rc = lib.slk_transpose_count(ctypes.byref(view), float(padding_ratio), ptr(ws), ws.numel(),
                                 ptr(rs_t), ptr(nnz_t), ptr(cap_t), capT_dev.data_ptr(),
                                 stream_of(capT_dev))
    if rc:
        _raise(rc)


def transpose_fill(view: CsrView, ws: torch.Tensor, rs_t: torch.Tensor, nnz_t: torch.Tensor,
                   cap_t: torch.Tensor, capT: int, val_t: torch.Tensor, col_t: torch.Tensor,
                   perm: torch.Tensor) -> None:
    lib = load()
    rc = lib.slk_transpose_fill(ctypes.byref(view), ptr(ws), ws.numel(), ptr(rs_t), ptr(nnz_t),
                                ptr(cap_t), capT, ptr(val_t), ptr(col_t), ptr(perm),
                                stream_of(perm))
    if rc:
        _raise(rc)


def transpose_refresh(W_values: torch.Tensor, perm: torch.Tensor, WT_values: torch.Tensor) -> None:
    lib = load()
    rc = lib.slk_transpose_refresh(ptr(W_values), W_values.numel(), ptr(perm), perm.numel(),
                                   ptr(WT_values), stream_of(WT_values))
    if rc:
        _raise(rc)


def row_hints(row_nnz: torch.Tensor, heavy_bar: float, dense_bar: float, dense_min_rows: int,
              out: torch.Tensor) -> None:
    """out[0] = rows with row_nnz > heavy_bar, out[1] = rows with row_nnz >=
    dense_bar (0 if fewer than dense_min_rows); float64 compares, on the
    device (slk_row_hints)."""
    lib = load()
    rc = lib.slk_row_hints(ptr(row_nnz), row_nnz.numel(), float(heavy_bar), float(dense_bar),
                           int(dense_min_rows), out.data_ptr(), stream_of(out))
    if rc:
        _raise(rc)


def check_invariants(view: CsrView, col_len: int, result: torch.Tensor) -> None:
    lib = load()
    rc = lib.slk_check_invariants(ctypes.byref(view), col_len, result.data_ptr(),
                                  stream_of(result))
    if rc:
        _raise(rc)


def live_abs_kth(view: CsrView, k: int, ws: torch.Tensor, thr: torch.Tensor) -> None:
    lib = load()
    rc = lib.slk_live_abs_kth(ctypes.byref(view), k, ws.data_ptr(), ws.numel(), thr.data_ptr(),
                              stream_of(thr))
    if rc:
        _raise(rc)


def drop_grow_workspace_bytes(view: CsrView) -> int:
    return int(load().slk_drop_grow_workspace_bytes(ctypes.byref(view)))


def drop_grow(view: CsrView, thr: torch.Tensor, rule: int, G: torch.Tensor | None, seed: int,
              ws: torch.Tensor, removed: torch.Tensor) -> None:
    """One SET / RigL pass over every row of the view's matrix, in place;
    ``removed`` (int64, 1 element) receives the live slots removed in total."""
    lib = load()
    ldg = G.stride(0) if G is not None else 0
    rc = lib.slk_drop_grow(ctypes.byref(view), view.values, view.col_indices, view.row_nnz,
                           thr.data_ptr(), rule, ptr(G), ldg, seed & (2**64 - 1), ptr(ws),
                           ws.numel(), removed.data_ptr(), stream_of(thr))
    if rc:
        _raise(rc)


def dense_grad(dY: torch.Tensor, X: torch.Tensor, M: int, K: int, N: int, token_major: bool,
               G: torch.Tensor) -> None:
    lib = load()
    rc = lib.slk_dense_grad(ptr(dY), ptr(X), M, K, N, int(token_major), ptr(G), stream_of(G))
    if rc:
        _raise(rc)


def spmm_t(view: CsrView, X: torch.Tensor, Yt: torch.Tensor,
           bias: torch.Tensor | None = None) -> None:
    """Yt (N x M, contiguous) = (W·X)ᵀ (+ bias per row of W) (slk_spmm_t)."""
    lib = load()
    rc = lib.slk_spmm_t(ctypes.byref(view), ptr(X), X.shape[0], X.shape[1], ptr(bias), ptr(Yt),
                        stream_of(Yt))
    if rc:
        _raise(rc)


def backward_narrow(view: CsrView, dYt: torch.Tensor, X: torch.Tensor,
                    dW: torch.Tensor | None, dbias: torch.Tensor | None,
                    dX: torch.Tensor | None, order: int) -> None:
    """dW / dbias / dX of a narrow layer from the token-major gradient dYt
    (N x M, contiguous); X is the K x N layer input (slk_backward_narrow)."""
    lib = load()
    rc = lib.slk_backward_narrow(ctypes.byref(view), ptr(dYt), dYt.shape[0], ptr(X), X.shape[0],
                                 ptr(dW), ptr(dbias), ptr(dX), int(order), stream_of(dYt))
    if rc:
        _raise(rc)


def backward_fused(view: CsrView, viewT: CsrView, perm: torch.Tensor, dY: torch.Tensor,
                   X: torch.Tensor, dW: torch.Tensor, dbias: torch.Tensor | None,
                   dX: torch.Tensor) -> None:
    """dW (SIMD order), dbias and dX = Wᵀ·dY of a small layer in one launch;
    viewT is the transpose's structure and perm its slot map, W's values read
    through it (slk_backward_fused)."""
    lib = load()
    rc = lib.slk_backward_fused(ctypes.byref(view), ctypes.byref(viewT), ptr(perm), ptr(dY),
                                ptr(X), dY.shape[1], ptr(dW), ptr(dbias), ptr(dX),
                                stream_of(dY))
    if rc:
        _raise(rc)


def seg_list_build(view: CsrView, block_cols: int, seg_slots: int, device):
    """(seg_start, seg_row, seg_count, seg_groups) int32 tensors: W's live slots
    cut into segments of at most seg_slots slots of one row inside one column
    block, block by block and row by row, each block padded with empty
    segments to whole groups of SEG_GROUP; seg_groups[0] = groups in use
    (slk_seg_list_build). The arrays have slk_seg_list_capacity entries."""
    lib = load()
    n = int(lib.slk_seg_list_capacity(ctypes.byref(view), int(block_cols), int(seg_slots)))
    n = max(n, SEG_GROUP)
    start = torch.empty(n, dtype=torch.int32, device=device)
    row = torch.empty(n, dtype=torch.int32, device=device)
    count = torch.empty(n, dtype=torch.int32, device=device)
    groups = torch.empty(1, dtype=torch.int32, device=device)
    nbytes = int(lib.slk_seg_list_workspace_bytes(ctypes.byref(view), int(block_cols)))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    rc = lib.slk_seg_list_build(ctypes.byref(view), int(block_cols), int(seg_slots), ptr(ws),
                                nbytes, ptr(start), ptr(row), ptr(count), n, ptr(groups),
                                stream_of(start))
    if rc:
        _raise(rc)
    return start, row, count, groups


def dense_rows_workspace_bytes(n_dense_rows: int, ncols: int) -> int:
    """Bytes of slk_csr.dense_ws (slk_dense_rows_workspace_bytes)."""
    return int(load().slk_dense_rows_workspace_bytes(int(n_dense_rows), int(ncols)))


def phase_bounds_build(view: CsrView, n_phases: int, device) -> torch.Tensor:
    """int32 tensor of nrows * (n_phases + 1) entries: for each row the first
    live slot whose column is >= p * ceil(ncols / n_phases), p = 0..n_phases
    (slk_phase_bounds_build)."""
    lib = load()
    lo = torch.empty(max(1, view.nrows * (int(n_phases) + 1)), dtype=torch.int32, device=device)
    rc = lib.slk_phase_bounds_build(ctypes.byref(view), int(n_phases), ptr(lo), stream_of(lo))
    if rc:
        _raise(rc)
    return lo


def bin_sizes(view: CsrView, first: int, rw: int, h: int) -> tuple[int, int]:
    """(units, chunks) of the binned slot stream (slk_bin_sizes); ValueError
    where the stream is not supported (e.g. more than BIN_MAX_CHUNKS chunks)."""
    units, nch = ctypes.c_int64(0), ctypes.c_int64(0)
    rc = load().slk_bin_sizes(ctypes.byref(view), int(first), int(rw), int(h),
                              ctypes.byref(units), ctypes.byref(nch))
    if rc:
        _raise(rc)
    return units.value, nch.value


def bin_build(view: CsrView, first: int, rw: int, h: int, n_bin: int, device):
    """(bin_off, bin_slot, bin_cnt, bin_start) device arrays of the binned slot
    stream of view's positions [first, nrows) (slk_bin_build); n_bin >= the
    covered live slots."""
    lib = load()
    units, nch = bin_sizes(view, first, rw, h)
    n = max(1, int(n_bin))
    off = torch.empty(n, dtype=torch.int32, device=device)
    slot = torch.empty(n, dtype=torch.int32, device=device)
    cnt = torch.empty(max(1, 2 * units * nch), dtype=torch.int32, device=device)
    start = torch.empty(units + 1, dtype=torch.int32, device=device)
    rc = lib.slk_bin_build(ctypes.byref(view), int(first), int(rw), int(h), ptr(off), ptr(slot),
                           int(n_bin), ptr(cnt), ptr(start), stream_of(start))
    if rc:
        _raise(rc)
    return off, slot, cnt, start


def dense_mfma_probe(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, D: torch.Tensor) -> None:
    """One fp32 32x32x1 two-block MFMA per case (slk_dense_mfma_probe): A, B
    float32 n x 64 (lane operands), C, D float32 n x 64 x 32 (lane registers)."""
    n = A.shape[0]
    if A.shape != (n, 64) or B.shape != (n, 64) or C.shape != (n, 64, 32) or D.shape != (n, 64, 32):
        raise ValueError("dense_mfma_probe: A, B must be n x 64 and C, D n x 64 x 32")
    for t in (A, B, C, D):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("dense_mfma_probe: float32 contiguous tensors expected")
    rc = load().slk_dense_mfma_probe(ptr(A), ptr(B), ptr(C), ptr(D), n, stream_of(D))
    if rc:
        _raise(rc)


def rigl_mfma_probe(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, D: torch.Tensor) -> None:
    """D[t] = C[t] + A[t]·B[t]ᵀ on the matrix cores, one 32x32x16 bf16 MFMA per
    t (slk_rigl_mfma_probe): A, B int16 (bf16 bits) n x 32 x 16, C, D float32
    n x 32 x 32, all contiguous."""
    n = A.shape[0]
    if (A.shape != (n, 32, 16) or B.shape != (n, 32, 16) or C.shape != (n, 32, 32)
            or D.shape != (n, 32, 32)):
        raise ValueError("rigl_mfma_probe: A, B must be n x 32 x 16 and C, D n x 32 x 32")
    rc = load().slk_rigl_mfma_probe(ptr(A), ptr(B), ptr(C), ptr(D), n, stream_of(D))
    if rc:
        _raise(rc)


def transpose_dense(src: torch.Tensor, dst: torch.Tensor) -> None:
    """dst (cols x rows, contiguous) = srcᵀ for a float32 src (rows x cols) whose
    rows are contiguous (stride(1) == 1)."""
    lib = load()
    rows, cols = src.shape
    rc = lib.slk_transpose_dense(ptr(src), rows, cols, src.stride(0) if rows > 1 else cols,
                                 ptr(dst), stream_of(dst))
    if rc:
        _raise(rc)


def set_tuning(knob: str, value: int | None) -> None:
    """Override one kernel choice process-wide (slk_set_tuning); None restores
    the launcher's own choice. For tests and measurement: results keep their
    bits under every setting."""
    rc = load().slk_set_tuning(TUNE_KNOBS[knob], -1 if value is None else int(value))
    if rc:
        _raise(rc)


def rigl_norms(dY: torch.Tensor, X: torch.Tensor, nrm_dY: torch.Tensor,
               nrm_X: torch.Tensor) -> None:
    """Row norms (upper bounds) of dY (M x N) and X (K x N) (slk_rigl_norms)."""
    rc = load().slk_rigl_norms(ptr(dY), dY.shape[0], ptr(X), X.shape[0], dY.shape[1],
                               ptr(nrm_dY), ptr(nrm_X), stream_of(nrm_dY))
    if rc:
        _raise(rc)


def dense_grad_approx(dY: torch.Tensor, X: torch.Tensor, G: torch.Tensor,
                      G_code: torch.Tensor) -> None:
    """G' = dY·Xᵀ on the matrix cores within the certified bound, and its
    partial-sum codes (uint8, M x K) (slk_dense_grad_approx); dY (M x N),
    X (K x N) row-major."""
    lib = load()
    M, N = dY.shape
    K = X.shape[0]
    if G_code.dtype != torch.uint8 or G_code.numel() != M * K or not G_code.is_contiguous():
        raise ValueError("dense_grad_approx: G_code must be a contiguous uint8 M x K tensor")
    nbytes = int(lib.slk_dense_grad_approx_workspace_bytes(M, K, N))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=G.device)
    rc = lib.slk_dense_grad_approx(ptr(dY), ptr(X), M, K, N, ptr(G), ptr(G_code), ptr(ws),
                                   nbytes, stream_of(G))
    if rc:
        _raise(rc)


def rigl_bound_factor(N: int) -> float:
    return float(load().slk_rigl_bound_factor(int(N)))


def rigl_partial_factor(N: int) -> float:
    return float(load().slk_rigl_partial_factor(int(N)))


def rigl_count(view: CsrView, thr: torch.Tensor, G: torch.Tensor, G_code: torch.Tensor,
               nrm_dY: torch.Tensor, nrm_X: torch.Tensor, N: int, info: torch.Tensor,
               amb_off: torch.Tensor, amb_total: torch.Tensor, amb_ws: torch.Tensor,
               ws: torch.Tensor) -> None:
    """Per-row survivors and undecided columns (slk_rigl_count); the lists go
    to amb_ws (8 bytes per undecided column) and ws (slk_drop_grow's
    workspace), which slk_rigl_finish then receives."""
    rc = load().slk_rigl_count(ctypes.byref(view), thr.data_ptr(), ptr(G), G.stride(0),
                               ptr(G_code), ptr(nrm_dY), ptr(nrm_X), int(N), ptr(info),
                               amb_off.data_ptr(), amb_total.data_ptr(), ptr(amb_ws),
                               amb_ws.numel(), ptr(ws), ws.numel(), stream_of(amb_total))
    if rc:
        _raise(rc)


def rigl_finish(view: CsrView, thr: torch.Tensor, G: torch.Tensor, G_code: torch.Tensor,
                nrm_dY: torch.Tensor, nrm_X: torch.Tensor, dY: torch.Tensor, X: torch.Tensor,
                info: torch.Tensor, amb_off: torch.Tensor, amb_ws: torch.Tensor,
                ws: torch.Tensor, removed: torch.Tensor) -> None:
    rc = load().slk_rigl_finish(ctypes.byref(view), view.values, view.col_indices, view.row_nnz,
                                thr.data_ptr(), ptr(G), G.stride(0), ptr(G_code), ptr(nrm_dY),
                                ptr(nrm_X),
                                ptr(dY), ptr(X), dY.shape[1], ptr(info), amb_off.data_ptr(),
                                ptr(amb_ws), amb_ws.numel(), ptr(ws), ws.numel(),
                                removed.data_ptr(), stream_of(removed))
    if rc:
        _raise(rc)


# HIP graph node types (hip_runtime_api.h, enum hipGraphNodeType)
GRAPH_NODE_TYPES = {0: "kernel", 1: "memcpy", 2: "memset", 3: "host", 4: "graph", 5: "empty",
                    6: "wait_event", 7: "event_record", 8: "ext_semaphore_signal",
                    9: "ext_semaphore_wait", 10: "mem_alloc", 11: "mem_free",
                    12: "memcpy_from_symbol", 13: "memcpy_to_symbol", 14: "batch_mem_op"}


def graph_node_types(graph: "torch.cuda.CUDAGraph") -> dict[str, int]:
    """Counts of each node type in a captured graph (made with keep_graph=True,
    read before replay). A memset node is what a captured hipMemsetAsync
    becomes: this library's entry points record none (their outputs are written
    by kernels), but library code captured beside them may, e.g. rocprim's
    partition and radix sort, which zero their counters that way."""
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch loaded (same soname)
    g = ctypes.c_void_p(graph.raw_cuda_graph())
    n = ctypes.c_size_t(0)
    if hip.hipGraphGetNodes(g, None, ctypes.byref(n)) != 0:
        raise RuntimeError("hipGraphGetNodes failed")
    nodes = (ctypes.c_void_p * max(1, n.value))()
    if n.value and hip.hipGraphGetNodes(g, nodes, ctypes.byref(n)) != 0:
        raise RuntimeError("hipGraphGetNodes failed")
    out: dict[str, int] = {}
    t = ctypes.c_int(0)
    for i in range(n.value):
        if hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(t)) != 0:
            raise RuntimeError("hipGraphNodeGetType failed")
        name = GRAPH_NODE_TYPES.get(t.value, f"type{t.value}")
        out[name] = out.get(name, 0) + 1
    return out
