"""The C-ABI library: it loads, exports every entry point include/*.h declares,
and its host-side argument checks answer without touching a device.

No kernel is launched here (no GPU is needed): every call below returns from
argument validation before any HIP call.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from sparsecore_amd import _lib

ROOT = Path(__file__).resolve().parent.parent


def _declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        names |= set(re.findall(r"SLK_API\s+[\w\s\*]+?\b(slk_\w+)\s*\(", h.read_text()))
    return names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_symbols()
    assert declared == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.slk_abi_version() == _lib.ABI_VERSION


def test_exported_symbols_are_exactly_the_api():
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], check=True,
                         capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert exported == _declared_symbols()


def _view(M=4, K=6, cap=0):
    return _lib.CsrView(M, K, cap, None, None, 1, 1, 1)


def test_shape_checks_answer_on_the_host():
    lib = _lib.load()
    v = _view()
    rc = lib.slk_spmm(ctypes.byref(v), None, 7, 3, None, None)
    assert rc == _lib.SLK_EINVAL
    msg = lib.slk_last_error().decode()
    assert "shape mismatch" in msg and "ncols=6" in msg
    rc = lib.slk_sddmm(ctypes.byref(v), None, 5, None, 6, 3, None, _lib.SLK_DW_SIMD, None)
    assert rc == _lib.SLK_EINVAL and "dY.shape" in lib.slk_last_error().decode()
    rc = lib.slk_sddmm(ctypes.byref(v), None, 4, None, 9, 3, None, _lib.SLK_DW_SIMD, None)
    assert rc == _lib.SLK_EINVAL and "X.shape" in lib.slk_last_error().decode()
    rc = lib.slk_sddmm(ctypes.byref(v), None, 4, None, 6, 3, None, 7, None)
    assert rc == _lib.SLK_EINVAL and "order" in lib.slk_last_error().decode()
    bad = _lib.CsrView(-1, 3, 0, None, None, None, None, None)
    assert lib.slk_spmm(ctypes.byref(bad), None, 3, 1, None, None) == _lib.SLK_EINVAL
    rc = lib.slk_transpose_count(ctypes.byref(v), -0.5, None, 0, None, None, None, None, None)
    assert rc == _lib.SLK_EINVAL and "padding_ratio" in lib.slk_last_error().decode()


def test_heavy_row_count_needs_an_order_and_a_valid_range():
    """slk_csr.n_heavy_rows is checked before any device work: it must lie in
    [0, nrows] and needs row_order."""
    lib = _lib.load()
    for n_heavy, order in ((1, None), (-1, 8), (5, 8)):
        v = _lib.CsrView(4, 6, 0, None, None, 1, 1, 1, order, n_heavy_rows=n_heavy)
        assert lib.slk_spmm(ctypes.byref(v), None, 6, 3, None, None) == _lib.SLK_EINVAL
        assert "n_heavy_rows" in lib.slk_last_error().decode()


def test_heavy_rows_are_those_far_above_the_mean():
    from sparsecore_amd.layout import HEAVY_ROW_FACTOR, heavy_row_count

    assert HEAVY_ROW_FACTOR == 2.0
    assert heavy_row_count(np.zeros(0, np.int32)) == 0
    assert heavy_row_count(np.full(100, 7, np.int32)) == 0  # uniform: none
    nnz = np.full(100, 10, np.int32)
    nnz[[3, 50]] = 200  # mean 13.8: heavy above 27.6
    assert heavy_row_count(nnz) == 2
    nnz[7] = 27  # mean 13.97, bar 27.94: still two
    assert heavy_row_count(nnz) == 2
    nnz[7] = 29  # mean 13.99, bar 27.98
    assert heavy_row_count(nnz) == 3
    import bench

    counts = bench.zipf_row_counts(16384, 16384, 0.05, 1.1, 0)
    assert heavy_row_count(counts) == int((counts > 2 * counts.mean()).sum()) > 0


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["zipf", "ties", "uniform", "empty-rows", "none", "dense",
                                  "dense-few", "dense-at-bar"])
@pytest.mark.parametrize("ncols", [4000, 8192])
def test_transpose_builders_count_rows_like_the_host_rules(dev, case, ncols):
    """The transpose builders count a WT's heavy and dense rows on the device
    (slk_row_hints, read with its capacity); the counts equal heavy_row_count
    and dense_row_count on the host arrays."""
    import torch

    from sparsecore_amd import layout

    rng = np.random.default_rng(3)
    bar = int(np.ceil(layout.DENSE_ROW_FRACTION * ncols))
    nnz = {"zipf": np.minimum(4000, (3000 * np.arange(1, 2501) ** -1.1).astype(np.int32)),
           "ties": np.array([10] * 99 + [4 * 10 + 30], np.int32),
           "uniform": np.full(3000, 17, np.int32),
           "empty-rows": np.concatenate([np.zeros(500, np.int32), rng.integers(0, 50, 2000)]),
           "none": np.zeros(0, np.int32),
           "dense": np.concatenate([rng.integers(bar, ncols, 40), rng.integers(0, 80, 3000)]),
           "dense-few": np.concatenate([rng.integers(bar, ncols, 31), rng.integers(0, 80, 3000)]),
           "dense-at-bar": np.concatenate([np.full(32, bar), np.full(32, bar - 1),
                                           rng.integers(0, 80, 3000)]),
           }[case].astype(np.int32)
    rng.shuffle(nnz)
    out = torch.full((2,), -1, dtype=torch.int64, device=dev)
    layout._count_rows(torch.from_numpy(nnz).to(dev), int(nnz.sum()), ncols, out)
    assert int(out[0]) == layout.heavy_row_count(nnz)
    assert int(out[1]) == layout.dense_row_count(nnz, ncols)
    if case == "dense" and ncols >= layout.DENSE_MIN_COLS:
        assert int(out[1]) == 40
    if case in ("dense-few", "uniform"):
        assert int(out[1]) == 0


def test_empty_problems_are_no_ops():
    lib = _lib.load()
    v = _lib.CsrView(0, 6, 0, None, None, None, None, None)
    assert lib.slk_spmm(ctypes.byref(v), None, 6, 3, None, None) == _lib.SLK_OK
    assert lib.slk_last_error().decode() == ""
    v = _view(cap=0)
    assert lib.slk_sddmm(ctypes.byref(v), None, 4, None, 6, 3, None, 0, None) == _lib.SLK_OK
    assert lib.slk_transpose_refresh(None, 0, None, 0, None, None) == _lib.SLK_OK


@pytest.mark.parametrize("M,K,expect_rows_per_block", [(512, 784, 4), (16384, 16384, 16)])
def test_transpose_workspace_is_bounded(M, K, expect_rows_per_block):
    lib = _lib.load()
    v = _lib.CsrView(M, K, 0, None, None, None, None, None)
    nbytes = lib.slk_transpose_workspace_bytes(ctypes.byref(v))
    nblk = -(-M // expect_rows_per_block)
    assert nbytes == nblk * K * 4
    assert nbytes <= (1 << 24) * 4


def test_topology_entry_points_check_arguments_on_the_host():
    lib = _lib.load()
    # fake, never dereferenced slot pointers: every call fails validation first
    v = _lib.CsrView(4, 6, 10, 8, 8, 1, 1, 1)
    rc = lib.slk_live_abs_kth(ctypes.byref(v), 3, None, 0, None, None)
    assert rc == _lib.SLK_EINVAL and "workspace" in lib.slk_last_error().decode()
    rc = lib.slk_live_abs_kth(ctypes.byref(v), 0, 1, _lib.SLK_KTH_WORKSPACE_BYTES, 1, None)
    assert rc == _lib.SLK_EINVAL and "k=0" in lib.slk_last_error().decode()
    # (W, values, col_indices, row_nnz, thr, rule, G, ldg, seed, ws, ws_bytes, removed, stream)
    rc = lib.slk_drop_grow(ctypes.byref(v), 16, 8, 1, 1, 0, None, 0, 0, None, 0, 1, None)
    assert rc == _lib.SLK_EINVAL and "own arrays" in lib.slk_last_error().decode()
    rc = lib.slk_drop_grow(ctypes.byref(v), 8, 8, 2, 1, 0, None, 0, 0, None, 0, 1, None)
    assert rc == _lib.SLK_EINVAL and "own arrays" in lib.slk_last_error().decode()
    rc = lib.slk_drop_grow(ctypes.byref(v), 8, 8, 1, 1, 5, None, 0, 0, None, 0, 1, None)
    assert rc == _lib.SLK_EINVAL and "rule" in lib.slk_last_error().decode()
    wide = _lib.CsrView(4, 200000, 10, 8, 8, 1, 1, 1)
    rc = lib.slk_drop_grow(ctypes.byref(wide), 8, 8, 1, 1, 0, None, 0, 0, None, 0, 1, None)
    assert rc == _lib.SLK_EINVAL and "ncols" in lib.slk_last_error().decode()
    rc = lib.slk_drop_grow(ctypes.byref(v), 8, 8, 1, 1, 0, None, 0, 0, None, 0, None, None)
    assert rc == _lib.SLK_EINVAL and "removed" in lib.slk_last_error().decode()
    rc = lib.slk_drop_grow(ctypes.byref(v), 8, 8, 1, 1, _lib.SLK_GROW_GRADIENT, None, 0, 0,
                           None, 0, 1, None)
    assert rc == _lib.SLK_EINVAL and "ldg" in lib.slk_last_error().decode()
    rc = lib.slk_drop_grow(ctypes.byref(v), 8, 8, 1, 1, _lib.SLK_GROW_RANDOM, None, 0, 0,
                           None, 79, 1, None)
    assert rc == _lib.SLK_EINVAL and "workspace" in lib.slk_last_error().decode()
    assert lib.slk_drop_grow_workspace_bytes(ctypes.byref(v)) == 80
    rc = lib.slk_dense_grad(None, None, -1, 2, 2, 0, None, None)
    assert rc == _lib.SLK_EINVAL and "non-negative" in lib.slk_last_error().decode()
    assert lib.slk_dense_grad(None, None, 0, 5, 4, 0, None, None) == _lib.SLK_OK


def test_spmm_bias_rejects_null_bias_on_the_host():
    lib = _lib.load()
    v = _view()
    rc = lib.slk_spmm_bias(ctypes.byref(v), None, 6, 3, None, None, None)
    assert rc == _lib.SLK_EINVAL and "bias" in lib.slk_last_error().decode()


def test_transpose_dense_rejects_bad_stride_on_the_host():
    lib = _lib.load()
    rc = lib.slk_transpose_dense(None, 4, 8, 5, None, None)
    assert rc == _lib.SLK_EINVAL and "ld_src" in lib.slk_last_error().decode()


def test_sddmm_bias_rejects_null_dbias_on_the_host():
    lib = _lib.load()
    v = _view()
    rc = lib.slk_sddmm_bias(ctypes.byref(v), None, 4, None, 6, 3, None, None, _lib.SLK_DW_SIMD,
                            None)
    assert rc == _lib.SLK_EINVAL and "dbias" in lib.slk_last_error().decode()


def test_segment_list_fields_are_checked_on_the_host():
    """A view that carries a segment list must carry all of it, with a block
    width of 64 or 128 and 4 or 8 slots per segment; slk_seg_list_build checks
    its block width, segment size and output length before any device work."""
    lib = _lib.load()
    one = ctypes.c_int32(0)
    p = ctypes.addressof(one)
    good = dict(seg_start=p, seg_row=p, seg_count=p, seg_groups=p, n_seg=64, seg_block=64,
                seg_slots=4)
    for bad in ({"seg_row": None}, {"seg_groups": None}, {"seg_block": 32}, {"seg_slots": 6},
                {"n_seg": -1}):
        f = dict(good, **bad)
        v = _lib.CsrView(4, 6, 0, None, None, 1, 1, 1, **f)
        rc = lib.slk_sddmm(ctypes.byref(v), None, 4, None, 6, 3, None, _lib.SLK_DW_SIMD, None)
        assert rc == _lib.SLK_EINVAL and "segment list" in lib.slk_last_error().decode(), bad
    v = _view()
    for cols, slots, word in ((32, 4, "block_cols"), (64, 5, "seg_slots")):
        rc = lib.slk_seg_list_build(ctypes.byref(v), cols, slots, None, 0, p, p, p, 64, p, None)
        assert rc == _lib.SLK_EINVAL and word in lib.slk_last_error().decode()
    need = lib.slk_seg_list_capacity(ctypes.byref(_lib.CsrView(4, 6, 40, None, None, 1, 1, 1)),
                                     64, 4)
    G = _lib.SEG_GROUP  # every run's segments, plus each block's padding (< G) and one group
    assert need == 40 // 4 + min(40, 4 * 1) + (G - 1) + G
    vc = _lib.CsrView(4, 6, 40, 1, 1, 1, 1, 1)
    rc = lib.slk_seg_list_build(ctypes.byref(vc), 64, 4, None, 0, p, p, p, need - 1, p, None)
    assert rc == _lib.SLK_EINVAL and "n_seg" in lib.slk_last_error().decode()


def test_phase_bounds_are_checked_on_the_host():
    """A view with phase bounds needs n_phases >= 1; slk_phase_bounds_build
    rejects fewer than one phase before any device work."""
    lib = _lib.load()
    one = ctypes.c_int32(0)
    v = _lib.CsrView(4, 6, 0, None, None, 1, 1, 1, phase_lo=ctypes.addressof(one), n_phases=0)
    rc = lib.slk_spmm(ctypes.byref(v), None, 6, 3, None, None)
    assert rc == _lib.SLK_EINVAL and "n_phases" in lib.slk_last_error().decode()
    rc = lib.slk_phase_bounds_build(ctypes.byref(_view()), 0, ctypes.addressof(one), None)
    assert rc == _lib.SLK_EINVAL and "n_phases" in lib.slk_last_error().decode()
