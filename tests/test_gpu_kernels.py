"""GPU parity of the HIP kernels against the oracle and the golden fixtures.

Bar: bit-exact. Forward and dX reproduce the reference's fma chains, dW the
reference's summation orders, and the transpose is pure integer/data movement
whose layout the PaddedCSR invariants fix uniquely.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from helpers import (assert_bits_equal, c1_inputs, csr_arrays_equal, from_oracle, golden_cases,
                     golden_csr, to_oracle)
from sparsecore_amd import _lib, layout, ops

pytestmark = pytest.mark.gpu

N_SWEEP = [1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 255, 256, 257, 1000]


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _spmm(W, X):
    return ops._launch_spmm(W, X)


def _sddmm(W, dY, X, kernel="simd"):
    return ops._launch_sddmm(W, dY, X, kernel)


def _with_fields(v, **changes):
    """A copy of a CsrView with some fields replaced."""
    fields = {f: getattr(v, f) for f, _ in _lib.CsrView._fields_}
    fields.update(changes)
    return _lib.CsrView(**fields)


# ───────────────────────── golden fixtures ─────────────────────────────

@pytest.mark.parametrize("name", sorted(golden_cases()))
def test_golden_fixture_bit_exact(dev, name):
    print(f"[golden] {name}", flush=True)
    case = golden_cases()[name]
    c = golden_csr(case)
    W = from_oracle(c, dev)
    X, dY = _t(case["X"], dev), _t(case["dY"], dev)
    assert_bits_equal(_spmm(W, X).cpu().numpy(), case["Y"], "Y")
    assert_bits_equal(_sddmm(W, dY, X, "simd").cpu().numpy(), case["dW"], "dW")
    assert_bits_equal(_sddmm(W, dY, X, "scalar").cpu().numpy(), case["dW_scalar"], "dW_scalar")
    WT = ops._cached_transpose(W)
    assert_bits_equal(_spmm(WT, dY).cpu().numpy(), case["dX"], "dX")


def test_c1_config_matches_reference_digests(dev):
    import gen

    print("[golden] c1 512x784 N=256", flush=True)
    meta, c, X_np, dY_np = c1_inputs()
    W = from_oracle(c, dev)
    X, dY = _t(X_np, dev), _t(dY_np, dev)
    WT, _ = layout.transpose_with_perm(W)
    outs = {"Y": _spmm(W, X), "dW": _sddmm(W, dY, X, "simd"),
            "dW_scalar": _sddmm(W, dY, X, "scalar"), "dX": _spmm(WT, dY)}
    for k, v in outs.items():
        got = v.cpu().numpy()
        s = meta["samples"][k]
        flat = got.reshape(-1)
        assert flat[s["index"]].view(np.uint32).tolist() == s["value_bits"], k
        assert gen.digest(got) == meta["outputs_sha256"][k], k


# ───────────────────────── forward / dW sweeps ─────────────────────────

def _case(M, K, N, per_row, seed, pr=0.2):
    c = oracle.uniform_rows(M, K, per_row, seed=seed, sigma=1.0, padding_ratio=pr)
    rng = np.random.default_rng(seed + 1)
    X = rng.standard_normal((K, N)).astype(np.float32)
    dY = rng.standard_normal((M, N)).astype(np.float32)
    return c, X, dY


@pytest.mark.parametrize("N", N_SWEEP)
def test_spmm_and_sddmm_bit_exact_over_N(dev, N):
    print(f"[sweep] N={N}", flush=True)
    c, X_np, dY_np = _case(48, 70, N, 11, seed=N)
    W = from_oracle(c, dev)
    X, dY = _t(X_np, dev), _t(dY_np, dev)
    assert_bits_equal(_spmm(W, X).cpu().numpy(), oracle.spmm(c, X_np), "Y")
    assert_bits_equal(_sddmm(W, dY, X).cpu().numpy(), oracle.sddmm(c, dY_np, X_np), "dW")
    assert_bits_equal(_sddmm(W, dY, X, "scalar").cpu().numpy(),
                      oracle.sddmm(c, dY_np, X_np, "scalar"), "dW scalar")


@pytest.mark.parametrize("N", [8, 64, 256])
def test_unaligned_inputs_take_the_scalar_load_path(dev, N):
    """X / dY starting 4 bytes past a 16-byte boundary (views with an offset)."""
    c, X_np, dY_np = _case(33, 41, N, 7, seed=5)
    W = from_oracle(c, dev)
    Xbuf = torch.empty(X_np.size + 1, device=dev)
    Xbuf[1:] = _t(X_np.reshape(-1), dev)
    dYbuf = torch.empty(dY_np.size + 1, device=dev)
    dYbuf[1:] = _t(dY_np.reshape(-1), dev)
    X = Xbuf[1:].view(X_np.shape)
    dY = dYbuf[1:].view(dY_np.shape)
    assert X.data_ptr() % 16 != 0
    assert_bits_equal(_spmm(W, X).cpu().numpy(), oracle.spmm(c, X_np), "Y")
    assert_bits_equal(_sddmm(W, dY, X).cpu().numpy(), oracle.sddmm(c, dY_np, X_np), "dW")


@pytest.mark.parametrize("vec", [1, 2, 4])
@pytest.mark.parametrize("N,per_row", [(300, 9), (1024, 150), (4100, 3)])
def test_spmm_every_vector_width(dev, tune, vec, N, per_row):
    """Each lane width of the one-row-per-wave kernel (the launcher picks it by
    problem size; tune(spmm_vec=...) forces it), including rows longer than one
    64-slot metadata chunk and partial last batches."""
    tune(spmm_vec=vec)
    c, X_np, _ = _case(40, 200, N, per_row, seed=vec * 7 + N)
    W = from_oracle(c, dev)
    assert_bits_equal(_spmm(W, _t(X_np, dev)).cpu().numpy(), oracle.spmm(c, X_np), "Y")


@pytest.mark.parametrize("h,rw", [(1, 2), (1, 3), (1, 4), (1, 6), (1, 8), (2, 2), (2, 3), (2, 4), (2, 6), (2, 8)])
@pytest.mark.parametrize("M,K,N,per_row", [
    (1, 1, 4, 1), (63, 127, 64, 40), (64, 128, 256, 128), (65, 129, 260, 100),
    (200, 300, 1000, 37), (130, 1000, 200, 700), (70, 5000, 96, 3000), (33, 260, 132, 0),
    (9, 64, 256, 64), (300, 64, 512, 64), (40, 100, 520, 50)])
def test_spmm_lds_kernel_bit_exact(dev, tune, h, rw, M, K, N, per_row):
    """The LDS-staged kernel (forced, each columns-per-lane and rows-per-wave
    variant): partial row blocks and column tiles (one half of a two-half tile
    past N), K not a multiple of the chunk, rows with more slots in one chunk
    than the chunk's rows (fully dense rows), empty rows."""
    tune(spmm_kernel=1)
    tune(spmm_h=h)
    tune(spmm_rw=rw)
    print(f"[lds h={h} rw={rw}] M={M} K={K} N={N} per_row={per_row}", flush=True)
    c, X_np, _ = _case(M, K, N, per_row, seed=M + K + N)
    W = from_oracle(c, dev)
    assert_bits_equal(_spmm(W, _t(X_np, dev)).cpu().numpy(), oracle.spmm(c, X_np), "Y")


@pytest.mark.parametrize("env,N", [
    ({"spmm_vec": 1}, 300), ({"spmm_vec": 2}, 300), ({"spmm_vec": 4}, 1024),
    ({}, 5), ({}, 40), ({"spmm_kernel": 1}, 132),
    ({"spmm_kernel": 1, "spmm_rw": 2}, 1024),
    ({"spmm_kernel": 1, "spmm_h": 2, "spmm_rw": 4}, 1032)])
def test_spmm_bias_epilogue_bit_exact(dev, tune, env, N):
    """slk_spmm_bias = slk_spmm followed by one float32 add of bias[i] per row,
    in every kernel (wave kernel at each lane width, packed narrow-N kernel,
    LDS-staged kernel), including rows with no live slot (Y = 0 + bias)."""
    tune(**env)
    print(f"[bias] env={env} N={N}", flush=True)
    c, X_np, _ = _case(45, 150, N, 20, seed=N + len(env))
    c.row_nnz[3] = 0
    c.col_indices[c.row_start[3]:c.row_start[3] + c.row_capacity[3]] = -1
    c.values[c.row_start[3]:c.row_start[3] + c.row_capacity[3]] = 0.0
    b_np = np.random.default_rng(N).standard_normal(45).astype(np.float32)
    W = from_oracle(c, dev)
    Y = torch.empty(45, N, device=dev)
    _lib.spmm(W._view(), _t(X_np, dev), Y, _t(b_np, dev))
    ref = oracle.spmm(c, X_np) + b_np[:, None]
    assert ref.dtype == np.float32
    assert_bits_equal(Y.cpu().numpy(), ref, "Y+bias")


def test_spmm_lds_kernel_skewed_rows(dev, tune):
    tune(spmm_kernel=1)
    c = oracle.zipf_rows(300, 700, 0.08, 1.1, seed=5, sigma=0.5)
    X_np = np.random.default_rng(5).standard_normal((700, 192)).astype(np.float32)
    W = from_oracle(c, dev)
    assert_bits_equal(_spmm(W, _t(X_np, dev)).cpu().numpy(), oracle.spmm(c, X_np), "Y")
    WT, _ = layout.transpose_with_perm(W)
    dY_np = np.random.default_rng(6).standard_normal((300, 192)).astype(np.float32)
    WT_o, _ = oracle.transpose_with_perm(c)
    assert_bits_equal(_spmm(WT, _t(dY_np, dev)).cpu().numpy(), oracle.spmm(WT_o, dY_np), "dX")


@pytest.mark.parametrize("pr", [0.0, 0.2, 0.5, 1.0])
def test_padding_slots_of_dW_are_exactly_zero(dev, pr):
    c, X_np, dY_np = _case(20, 30, 9, 6, seed=11, pr=pr)
    W = from_oracle(c, dev)
    dW = _sddmm(W, _t(dY_np, dev), _t(X_np, dev)).cpu().numpy()
    pads = oracle.padding_slots(c)
    assert np.all(dW[pads].view(np.uint32) == 0)  # +0.0 exactly


def test_skewed_rows_bit_exact(dev):
    c = oracle.zipf_rows(256, 512, 0.05, 1.1, seed=3, sigma=0.5)
    rng = np.random.default_rng(3)
    X_np = rng.standard_normal((512, 96)).astype(np.float32)
    dY_np = rng.standard_normal((256, 96)).astype(np.float32)
    W = from_oracle(c, dev)
    X, dY = _t(X_np, dev), _t(dY_np, dev)
    assert int(c.row_nnz.max()) == 512  # a fully dense row
    assert_bits_equal(_spmm(W, X).cpu().numpy(), oracle.spmm(c, X_np), "Y")
    assert_bits_equal(_sddmm(W, dY, X).cpu().numpy(), oracle.sddmm(c, dY_np, X_np), "dW")
    WT, perm = layout.transpose_with_perm(W)
    WT_o, perm_o = oracle.transpose_with_perm(c)
    csr_arrays_equal(to_oracle(WT), WT_o, "WT")
    assert_bits_equal(perm.cpu().numpy(), perm_o, "perm")


@pytest.mark.parametrize("G", [1, 2, 4])
@pytest.mark.parametrize("N", [16, 24, 256, 260, 264, 271, 512, 1000, 1031, 2048])
def test_sddmm_windowed_groups_bit_exact(dev, tune, G, N):
    """dW with G groups of 16 slots per wave swept through N one window at a
    time (the launcher's choice for 16-byte-aligned large N; tune(sddmm_g=...) forces
    G, 1 = the one-group kernel). Cases: groups inside one row, across rows,
    rows of 1..3 live slots, empty rows, a fully dense row, padding ratios 0
    and 1, an 8-wide tail step, a scalar tail, partial windows, and a capacity
    that is not a multiple of the wave."""
    tune(sddmm_g=G)
    kernel = f"G={G}"
    print(f"[sddmm {kernel}] N={N}", flush=True)
    rng = np.random.default_rng(N + G)
    cases = [oracle.uniform_rows(97, 50, 3, seed=N, sigma=1.0, padding_ratio=0.2),
             oracle.uniform_rows(64, 40, 1, seed=N + 1, sigma=1.0, padding_ratio=0.0),
             oracle.zipf_rows(120, 300, 0.05, 1.1, seed=N + 2, sigma=0.5),
             oracle.uniform_rows(33, 64, 20, seed=N + 3, sigma=1.0, padding_ratio=1.0),
             oracle.uniform_rows(7, 500, 300, seed=N + 4, sigma=1.0, padding_ratio=0.2)]
    c = cases[3]
    c.row_nnz[5] = 0
    c.col_indices[c.row_start[5]:c.row_start[5] + c.row_capacity[5]] = -1
    c.values[c.row_start[5]:c.row_start[5] + c.row_capacity[5]] = 0.0
    for i, c in enumerate(cases):
        X_np = rng.standard_normal((c.ncols, N)).astype(np.float32)
        dY_np = rng.standard_normal((c.nrows, N)).astype(np.float32)
        W = from_oracle(c, dev)
        got = _sddmm(W, _t(dY_np, dev), _t(X_np, dev)).cpu().numpy()
        assert_bits_equal(got, oracle.sddmm(c, dY_np, X_np), f"dW case {i}")


@pytest.mark.parametrize("N", [1, 5, 40, 256, 1028])
def test_row_order_schedule_bit_exact(dev, N):
    """Tall skewed matrices get a longest-rows-first schedule (slk_csr.row_order).
    The schedule moves rows between waves only: results stay bit-exact, for the
    one-row-per-wave kernel and for the several-rows-per-wave kernel (N < 64)."""
    print(f"[row_order] N={N}", flush=True)
    c = oracle.zipf_rows(3000, 400, 0.03, 1.1, seed=N, sigma=0.5)
    rng = np.random.default_rng(N)
    X_np = rng.standard_normal((400, N)).astype(np.float32)
    W = from_oracle(c, dev)
    v = W._view()
    assert v.row_order is not None
    order = W._order[1].cpu().numpy()
    assert sorted(order.tolist()) == list(range(3000))
    assert np.all(np.diff(c.row_nnz[order]) <= 0)
    want = oracle.spmm(c, X_np)
    X = _t(X_np, dev)
    assert_bits_equal(_spmm(W, X).cpu().numpy(), want, "Y (row_order)")
    # any permutation is a valid schedule: a random one through the C view
    perm = torch.from_numpy(rng.permutation(3000).astype(np.int32)).to(dev)
    v2 = _with_fields(v, row_order=perm.data_ptr())
    Y = torch.empty(3000, N, device=dev)
    _lib.spmm(v2, X, Y)
    assert_bits_equal(Y.cpu().numpy(), want, "Y (random order)")
    # and no schedule at all
    v3 = _with_fields(v, row_order=None, n_heavy_rows=0)
    _lib.spmm(v3, X, Y)
    assert_bits_equal(Y.cpu().numpy(), want, "Y (natural order)")


def test_gather_path_skewed_rows_wide_N_bit_exact(dev):
    """A skewed matrix too sparse for the LDS kernel, at N >= 1024 (the 16-byte
    gather kernel over the longest-first order): rows from fully dense to
    empty give the reference's bits, with and without bias."""
    print("[gather skewed wide N]", flush=True)
    c = oracle.zipf_rows(2500, 600, 0.01, 1.1, seed=17, sigma=0.5)
    assert c.row_nnz.max() == 600 and c.row_nnz.min() == 0
    rng = np.random.default_rng(17)
    N = 1040
    X_np = rng.standard_normal((600, N)).astype(np.float32)
    b_np = rng.standard_normal(2500).astype(np.float32)
    W = from_oracle(c, dev)
    v = W._view()
    assert v.row_order is not None and v.n_heavy_rows > 0
    X = _t(X_np, dev)
    want = oracle.spmm(c, X_np)
    Y = torch.full((2500, N), float("nan"), device=dev)
    _lib.spmm(v, X, Y)
    assert_bits_equal(Y.cpu().numpy(), want, "Y")
    _lib.spmm(v, X, Y, _t(b_np, dev))
    assert_bits_equal(Y.cpu().numpy(), want + b_np[:, None], "Y+bias")


@pytest.mark.parametrize("h,rw", [(1, 2), (1, 3), (1, 4), (1, 6), (1, 8), (2, 2), (2, 3), (2, 4), (2, 6), (2, 8)])
def test_row_order_lds_kernel_bit_exact(dev, tune, h, rw):
    """Every LDS-staged kernel variant gives the natural order's bits whatever
    row schedule the view carries (the longest-first one, a random
    permutation, none): a tall skewed matrix with a partial last row block
    (3000 rows) and a partial column tile, with and without bias."""
    tune(spmm_kernel=1)
    tune(spmm_h=h)
    tune(spmm_rw=rw)
    print(f"[row_order lds h={h} rw={rw}]", flush=True)
    c = oracle.zipf_rows(3000, 400, 0.03, 1.1, seed=rw + h, sigma=0.5)
    rng = np.random.default_rng(rw * h)
    N = 260
    X_np = rng.standard_normal((400, N)).astype(np.float32)
    b_np = rng.standard_normal(3000).astype(np.float32)
    W = from_oracle(c, dev)
    v = W._view()
    assert v.row_order is not None
    X, b = _t(X_np, dev), _t(b_np, dev)
    want = oracle.spmm(c, X_np)
    perm = torch.from_numpy(rng.permutation(3000).astype(np.int32)).to(dev)
    for name, view in (("sorted", v), ("random", _with_fields(v, row_order=perm.data_ptr())),
                       ("natural", _with_fields(v, row_order=None, n_heavy_rows=0))):
        Y = torch.full((3000, N), float("nan"), device=dev)
        _lib.spmm(view, X, Y)
        assert_bits_equal(Y.cpu().numpy(), want, f"Y ({name} order)")
        _lib.spmm(view, X, Y, b)
        assert_bits_equal(Y.cpu().numpy(), want + b_np[:, None], f"Y+bias ({name} order)")


@pytest.mark.parametrize("h,rw", [(1, 2), (1, 3), (1, 4), (1, 6), (1, 8), (2, 2), (2, 3), (2, 4), (2, 6), (2, 8)])
def test_lds_heavy_row_split_bit_exact(dev, tune, h, rw):
    """A skewed matrix's heavy rows (the head of the longest-first order) run
    as their own LDS launch and the rest as a second one: the bits are the
    oracle's for every split point (none, one row, a partial row block, the
    view's own count, all but one row, all rows), every variant of the second
    launch, with and without bias."""
    tune(spmm_kernel=1)
    tune(spmm_h=h)
    tune(spmm_rw=rw)
    print(f"[heavy split h={h} rw={rw}]", flush=True)
    c = oracle.zipf_rows(3000, 700, 0.03, 1.1, seed=h * 10 + rw, sigma=0.5)
    rng = np.random.default_rng(rw + h)
    N = 520
    X_np = rng.standard_normal((700, N)).astype(np.float32)
    b_np = rng.standard_normal(3000).astype(np.float32)
    W = from_oracle(c, dev)
    v = W._view()
    assert v.row_order is not None and 0 < v.n_heavy_rows < 300
    assert v.n_heavy_rows == layout.heavy_row_count(c.row_nnz)
    X, b = _t(X_np, dev), _t(b_np, dev)
    want = oracle.spmm(c, X_np)
    for T in (0, 1, 45, v.n_heavy_rows, 2999, 3000):
        view = _with_fields(v, n_heavy_rows=T)
        Y = torch.full((3000, N), float("nan"), device=dev)
        _lib.spmm(view, X, Y)
        assert_bits_equal(Y.cpu().numpy(), want, f"Y (T={T})")
        _lib.spmm(view, X, Y, b)
        assert_bits_equal(Y.cpu().numpy(), want + b_np[:, None], f"Y+bias (T={T})")


@pytest.mark.parametrize("split", [None, 1])
def test_lds_heavy_rows_with_phase_bounds_on_two_streams_bit_exact(dev, tune, split):
    """With phase bounds in the view, the rows after the heavy ones run on the
    phased gather kernel on the library's second stream, concurrently with the
    heavy rows' LDS launch (split=None, the default), or as the one-grid LDS
    split (split=1): the oracle's bits either way, for several split points,
    with and without bias, and again on later calls (the side stream reused)."""
    tune(spmm_kernel=1)
    if split is not None:
        tune(spmm_split=split)
    print(f"[heavy two streams split={split}]", flush=True)
    c = oracle.zipf_rows(3000, 700, 0.03, 1.1, seed=91, sigma=0.5)
    rng = np.random.default_rng(91)
    N = 520
    X_np = rng.standard_normal((700, N)).astype(np.float32)
    b_np = rng.standard_normal(3000).astype(np.float32)
    W = from_oracle(c, dev)
    v = W._view_phased(3)
    assert v.row_order is not None and v.n_heavy_rows > 0 and v.n_phases == 3
    X, b = _t(X_np, dev), _t(b_np, dev)
    want = oracle.spmm(c, X_np)
    for rep in range(2):
        for T in (1, v.n_heavy_rows, 2999):
            view = _with_fields(v, n_heavy_rows=T)
            Y = torch.full((3000, N), float("nan"), device=dev)
            _lib.spmm(view, X, Y)
            torch.cuda.synchronize()
            assert_bits_equal(Y.cpu().numpy(), want, f"Y (T={T}, call {rep})")
            _lib.spmm(view, X, Y, b)
            torch.cuda.synchronize()
            assert_bits_equal(Y.cpu().numpy(), want + b_np[:, None], f"Y+bias (T={T}, call {rep})")


def test_transpose_builders_hint_the_heavy_row_count(dev):
    """A transpose's heavy-row count is counted on the device with its capacity
    (no host read of its rows), by both builders; it equals the host rule on
    the built WT, and rewrite_row drops the hint."""
    print("[heavy hint]", flush=True)
    cT = oracle.zipf_rows(3000, 400, 0.03, 1.1, seed=9, sigma=0.5)
    c, _ = oracle.transpose_with_perm(cT)  # 400 x 3000, skewed columns
    W = from_oracle(c, dev)
    WT1, _ = layout.transpose_with_perm(W)
    (WT2, _), = layout.transposes_with_perm([W])
    want = layout.heavy_row_count(cT.row_nnz)
    assert want > 0
    for WT in (WT1, WT2):
        assert WT._heavy_hint == want
        assert WT._view().n_heavy_rows == want
        assert WT._host_rows is None  # nothing was read back for it
    r = int(np.argmax(to_oracle(WT1).row_capacity))
    WT1.rewrite_row(r, np.arange(3), np.ones(3, np.float32))
    assert WT1._heavy_hint is None
    assert WT1._view().n_heavy_rows == layout.heavy_row_count(to_oracle(WT1).row_nnz)


def test_row_order_follows_rewrite_row(dev):
    """rewrite_row changes row_nnz, so the cached schedule is rebuilt."""
    c = oracle.uniform_rows(2048, 64, 4, seed=2, sigma=1.0, padding_ratio=3.0)
    W = from_oracle(c, dev)
    W._view()
    W.rewrite_row(1500, np.arange(16, dtype=np.int32), np.ones(16, np.float32))
    W._view()
    assert int(W._order[1][0]) == 1500
    X_np = np.random.default_rng(1).standard_normal((64, 70)).astype(np.float32)
    assert_bits_equal(_spmm(W, _t(X_np, dev)).cpu().numpy(),
                      oracle.spmm(to_oracle(W), X_np), "Y after rewrite_row")


def test_empty_shapes(dev):
    empty = layout.PaddedCSR(8, 16, device=dev)
    Y = _spmm(empty, torch.randn(16, 4, device=dev))
    assert Y.shape == (8, 4) and torch.count_nonzero(Y).item() == 0
    dW = _sddmm(empty, torch.randn(8, 4, device=dev), torch.randn(16, 4, device=dev))
    assert dW.shape == (0,)
    zero_rows = layout.PaddedCSR(0, 5, device=dev)
    assert _spmm(zero_rows, torch.randn(5, 3, device=dev)).shape == (0, 3)
    c, X_np, _ = _case(6, 9, 3, 2, seed=1)
    W = from_oracle(c, dev)
    assert _spmm(W, _t(X_np[:, :0], dev)).shape == (6, 0)
    zeros = from_oracle(oracle.from_dense(np.zeros((5, 7), np.float32)), dev)
    assert torch.count_nonzero(_spmm(zeros, torch.randn(7, 3, device=dev))).item() == 0
    no_cols = layout.PaddedCSR(4, 0, device=dev)
    Y = _spmm(no_cols, torch.empty(0, 6, device=dev))
    assert Y.shape == (4, 6) and torch.count_nonzero(Y).item() == 0


def test_shape_errors_raise_value_error(dev):
    c, X_np, dY_np = _case(8, 16, 4, 3, seed=2)
    W = from_oracle(c, dev)
    with pytest.raises(ValueError, match="shape mismatch"):
        _spmm(W, torch.randn(17, 4, device=dev))
    with pytest.raises(ValueError, match="dY.shape"):
        _sddmm(W, torch.randn(9, 4, device=dev), _t(X_np, dev))
    with pytest.raises(ValueError, match="X.shape"):
        _sddmm(W, _t(dY_np, dev), torch.randn(15, 4, device=dev))


def test_repeated_calls_are_bit_identical(dev):
    c, X_np, dY_np = _case(64, 128, 96, 20, seed=9)
    W = from_oracle(c, dev)
    X, dY = _t(X_np, dev), _t(dY_np, dev)
    y0, g0 = _spmm(W, X), _sddmm(W, dY, X)
    t0 = layout.transpose_with_perm(W)
    for _ in range(3):
        assert torch.equal(_spmm(W, X), y0)
        assert torch.equal(_sddmm(W, dY, X), g0)
        t = layout.transpose_with_perm(W)
        assert torch.equal(t[1], t0[1]) and torch.equal(t[0].col_indices, t0[0].col_indices)


# ─────────────────────────── transpose ─────────────────────────────────

@pytest.mark.parametrize("M,K,sparsity,pr", [
    (3, 4, 0.5, 0.2), (8, 8, 0.0, 0.2), (8, 8, 0.9, 0.2), (16, 32, 0.8, 0.0), (32, 16, 0.8, 1.0),
    (1, 1, 0.0, 0.2), (1, 16, 0.5, 0.2), (16, 1, 0.5, 0.2), (64, 64, 0.99, 0.2),
    (512, 784, 0.9, 0.2), (1536, 384, 0.9, 0.2), (300, 7, 0.3, 0.3)])
def test_transpose_bit_exact(dev, M, K, sparsity, pr):
    print(f"[transpose] {M}x{K} s={sparsity} pr={pr}", flush=True)
    c = oracle.bernoulli(M, K, sparsity, seed=M + K)
    W = from_oracle(c, dev)
    WT, perm = layout.transpose_with_perm(W, padding_ratio=pr)
    WT_o, perm_o = oracle.transpose_with_perm(c, pr)
    csr_arrays_equal(to_oracle(WT), WT_o, "WT")
    assert_bits_equal(perm.cpu().numpy(), perm_o, "perm")
    assert WT.nnz == c.nnz and WT.shape == (K, M)
    WT.assert_invariants()


@pytest.mark.parametrize("M,K,kind", [
    (2000, 1000, "uniform"), (1300, 3000, "zipf"), (777, 5000, "uniform"), (4100, 700, "zipf"),
    (70, 20000, "uniform")])
def test_transpose_tiles_bit_exact(dev, tune, M, K, kind):
    """The row x column tiled scatter (the default where a row block is at most
    32 rows and ncols >= 512) gives the oracle's WT and perm, as does the
    one-workgroup-per-row-block scatter it replaces: partial row and column
    tiles, skewed rows."""
    print(f"[transpose tiles] {M}x{K} {kind}", flush=True)
    c = (oracle.zipf_rows(M, K, 0.03, 1.1, seed=M, sigma=1.0) if kind == "zipf"
         else oracle.uniform_rows(M, K, max(1, K // 40), seed=M))
    W = from_oracle(c, dev)
    WT_o, perm_o = oracle.transpose_with_perm(c)
    for tile in (None, 0):
        tune(transpose_tile=tile)
        WT, perm = layout.transpose_with_perm(W)
        csr_arrays_equal(to_oracle(WT), WT_o, f"WT tile={tile}")
        assert_bits_equal(perm.cpu().numpy(), perm_o, f"perm tile={tile}")


@pytest.mark.parametrize("M,K,kind", [
    (300, 200, "uniform"), (5000, 256, "zipf"), (2000, 257, "uniform"), (1300, 3000, "zipf"),
    (4100, 700, "zipf"), (70, 20000, "uniform"), (40, 40000, "uniform"), (9, 65535, "uniform"),
    (3000, 5000, "empty-rows"), (64, 3000, "none-live")])
def test_transpose_radix_bit_exact(dev, tune, M, K, kind):
    """The radix path (a stable sort by column: one 8-bit pass for ncols <=
    256, two up to 65535) gives the oracle's WT and perm, and so does the
    counting sort: one-pass and two-pass column counts, skewed rows, column
    chunks of the count (ncols > 16384), rows and matrices without live
    slots, partial tiles."""
    print(f"[transpose radix] {M}x{K} {kind}", flush=True)
    if kind == "zipf":
        c = oracle.zipf_rows(M, K, 0.03, 1.1, seed=M, sigma=1.0)
    elif kind == "empty-rows":
        c = oracle.uniform_rows(M, K, 40, seed=M)
        dense = oracle.to_dense(c)
        dense[::3] = 0.0  # every third row empty
        c = oracle.from_dense(dense)
    elif kind == "none-live":
        c = oracle.from_dense(np.zeros((M, K), np.float32))
    else:
        c = oracle.uniform_rows(M, K, max(1, K // 40), seed=M)
    W = from_oracle(c, dev)
    WT_o, perm_o = oracle.transpose_with_perm(c)
    for radix in (1, 0):
        tune(transpose_radix=radix)
        WT, perm = layout.transpose_with_perm(W)
        csr_arrays_equal(to_oracle(WT), WT_o, f"WT radix={radix}")
        assert_bits_equal(perm.cpu().numpy(), perm_o, f"perm radix={radix}")


def test_transpose_wide_matrix_uses_column_chunks(dev):
    """ncols > 16384 exercises the multi-pass (column-chunked) LDS counters."""
    c = oracle.uniform_rows(40, 40000, 300, seed=4)
    W = from_oracle(c, dev)
    WT, perm = layout.transpose_with_perm(W)
    WT_o, perm_o = oracle.transpose_with_perm(c)
    csr_arrays_equal(to_oracle(WT), WT_o, "WT")
    assert_bits_equal(perm.cpu().numpy(), perm_o, "perm")


def test_transpose_of_empty_and_empty_ctor(dev):
    W = layout.PaddedCSR(5, 8, device=dev)
    WT = W.transpose()
    assert WT.shape == (8, 5) and WT.nnz == 0
    assert WT.row_capacity.tolist() == [1] * 8
    WT.assert_invariants()
    W0 = layout.PaddedCSR(0, 3, device=dev)
    assert W0.transpose().row_capacity.tolist() == [1, 1, 1]


def test_transpose_refresh_matches_oracle(dev):
    c = oracle.bernoulli(64, 48, 0.8, seed=6)
    W = from_oracle(c, dev)
    WT, perm = layout.transpose_with_perm(W)
    with torch.no_grad():
        W.values.mul_(-3.0).add_(0.25)
    before = WT.values.clone()
    _lib.transpose_refresh(W.values, perm, WT.values)
    expect = oracle.refresh(before.cpu().numpy(), W.values.cpu().numpy(), perm.cpu().numpy())
    assert_bits_equal(WT.values.cpu().numpy(), expect, "refreshed values")


def test_transpose_negative_padding_ratio(dev):
    W = from_oracle(oracle.bernoulli(4, 4, 0.5, seed=1), dev)
    with pytest.raises(ValueError, match="padding_ratio"):
        W.transpose(padding_ratio=-0.1)


@pytest.mark.parametrize("rows,cols,ld", [(1, 1, 1), (1, 7, 9), (31, 33, 33), (256, 784, 784),
                                          (100, 40, 64), (2048, 96, 96), (65, 1, 3)])
def test_transpose_dense_is_a_bitwise_copy(dev, rows, cols, ld):
    """slk_transpose_dense: dst = srcᵀ for row-strided sources, partial tiles."""
    buf = torch.randn(rows * ld + 3, device=dev)
    src = buf[:rows * ld].view(rows, ld)[:, :cols]
    dst = torch.empty(cols, rows, device=dev)
    _lib.transpose_dense(src, dst)
    assert torch.equal(dst.view(torch.int32), src.t().contiguous().view(torch.int32))



@pytest.mark.parametrize("env,N,order", [
    ({}, 256, "simd"), ({}, 255, "simd"), ({"sddmm_g": 2}, 1040, "simd"),
    ({"sddmm_g": 4}, 1024, "simd"), ({}, 37, "scalar"), ({}, 0, "simd")])
def test_sddmm_bias_fuses_the_bias_gradient(dev, tune, env, N, order):
    """slk_sddmm_bias: dW bit-identical to slk_sddmm, dbias = Σ_j dY[i, j] within
    float32 rounding of the float64 sum, repeatable, for every dW kernel
    (including rows with no live slot and the scalar order)."""
    tune(**env)
    c, X_np, dY_np = _case(70, 90, N, 12, seed=N + 3)
    c.row_nnz[4] = 0
    c.col_indices[c.row_start[4]:c.row_start[4] + c.row_capacity[4]] = -1
    c.values[c.row_start[4]:c.row_start[4] + c.row_capacity[4]] = 0.0
    W = from_oracle(c, dev)
    X, dY = _t(X_np, dev), _t(dY_np, dev)
    ordv = _lib.SLK_DW_SCALAR if order == "scalar" else _lib.SLK_DW_SIMD
    dW0 = torch.empty(W.total_capacity, device=dev)
    _lib.sddmm(W._view(), dY, X, dW0, ordv)
    runs = []
    for _ in range(2):
        dW = torch.empty(W.total_capacity, device=dev)
        db = torch.full((70,), float("nan"), device=dev)
        _lib.sddmm(W._view(), dY, X, dW, ordv, db)
        runs.append((dW.cpu().numpy(), db.cpu().numpy()))
    assert_bits_equal(runs[0][0], dW0.cpu().numpy(), "dW")
    assert_bits_equal(runs[1][1], runs[0][1], "dbias repeat")
    ref = dY_np.astype(np.float64).sum(axis=1)
    bound = 1e-6 * np.abs(dY_np).astype(np.float64).sum(axis=1) + 1e-30
    assert np.all(np.abs(runs[0][1] - ref) <= bound), "dbias"


def _zero_capacity_rows(M, K, per_row, empty, seed):
    """A padded CSR whose rows in `empty` have capacity 0 (no slots at all)."""
    rng = np.random.default_rng(seed)
    cols, vals = [], []
    for i in range(M):
        n = 0 if i in empty else int(rng.integers(0, per_row + 1))
        cols.append(np.sort(rng.choice(K, size=n, replace=False)).astype(np.int32))
        vals.append(rng.standard_normal(n).astype(np.float32))
    cap = np.array([0 if i in empty else max(1, int(np.ceil(len(cols[i]) * 1.2)))
                    for i in range(M)], dtype=np.int32)
    rs = np.zeros(M, dtype=np.int32)
    rs[1:] = np.cumsum(cap)[:-1]
    col = np.full(int(cap.sum()), -1, dtype=np.int32)
    val = np.zeros(int(cap.sum()), dtype=np.float32)
    for i in range(M):
        col[rs[i]:rs[i] + len(cols[i])] = cols[i]
        val[rs[i]:rs[i] + len(cols[i])] = vals[i]
    return oracle.Csr(M, K, val, col, rs, np.array([len(x) for x in cols], np.int32), cap)


@pytest.mark.parametrize("N", [16, 20, 64, 100, 128, 200, 256, 264, 268, 384, 520])
@pytest.mark.parametrize("layout", ["dense-rows", "zero-capacity-runs", "short-zero-runs"])
def test_sddmm_rows_without_slots_bit_exact(dev, N, layout):
    """dW at every N shape of the one-group kernel (pairs of 128-float blocks,
    a lone block, 16-wide steps, the 8-wide step, the scalar tail), including
    runs of rows with capacity 0 between the slots of one wave: long ones
    (more than 63 rows: the fallback search) and runs of 1, 2, 30, 61, 62, 63
    and 64 rows (the ballot over the next 64 rows' starts, at its edge)."""
    print(f"[dW rows] N={N} {layout}", flush=True)
    if layout == "dense-rows":
        c = oracle.uniform_rows(300, 90, 30, seed=N, sigma=1.0)
    elif layout == "zero-capacity-runs":
        empty = set(range(5, 150)) | set(range(151, 240))
        c = _zero_capacity_rows(400, 90, 12, empty, seed=N)
    else:
        empty, r = set(), 3
        for run in (1, 2, 30, 61, 62, 63, 64, 1, 63):
            empty |= set(range(r, r + run))
            r += run + 2
        c = _zero_capacity_rows(r + 20, 90, 12, empty, seed=N)
    rng = np.random.default_rng(N)
    X_np = rng.standard_normal((90, N)).astype(np.float32)
    dY_np = rng.standard_normal((c.nrows, N)).astype(np.float32)
    W = from_oracle(c, dev)
    got = _sddmm(W, _t(dY_np, dev), _t(X_np, dev)).cpu().numpy()
    assert_bits_equal(got, oracle.sddmm(c, dY_np, X_np), "dW")


# ───────────────────────── narrow layers ───────────────────────────────

def _narrow_case(M, K, N, per_row, seed, empty=()):
    c = oracle.uniform_rows(M, K, per_row, seed=seed, sigma=1.0)
    for i in empty:
        c.row_nnz[i] = 0
        c.col_indices[c.row_start[i]:c.row_start[i] + c.row_capacity[i]] = -1
        c.values[c.row_start[i]:c.row_start[i] + c.row_capacity[i]] = 0.0
    rng = np.random.default_rng(seed + 7)
    X = rng.standard_normal((K, N)).astype(np.float32)
    dY = rng.standard_normal((M, N)).astype(np.float32)
    b = rng.standard_normal(M).astype(np.float32)
    return c, X, dY, b


@pytest.mark.parametrize("M,K,N,per_row", [
    (10, 512, 256, 51), (1, 40, 7, 13), (64, 100, 1, 20), (33, 70, 130, 70), (5, 3000, 64, 5)])
def test_spmm_t_token_major_bit_exact(dev, M, K, N, per_row):
    """slk_spmm_t stores (W·X)ᵀ token-major with the same fma chain and bias
    rounding as slk_spmm_bias, with and without bias, empty rows included."""
    print(f"[spmm_t] M={M} K={K} N={N}", flush=True)
    c, X_np, _, b_np = _narrow_case(M, K, N, per_row, seed=M + N, empty=(0,))
    W = from_oracle(c, dev)
    X = _t(X_np, dev)
    for bias in (None, _t(b_np, dev)):
        Yt = torch.full((N, M), float("nan"), device=dev)
        _lib.spmm_t(W._view(), X, Yt, bias)
        ref = oracle.spmm(c, X_np) + (b_np[:, None] if bias is not None else np.float32(0))
        assert_bits_equal(Yt.cpu().numpy(), np.ascontiguousarray(ref.T), "Yt")


@pytest.mark.parametrize("M,K,N,per_row", [
    (10, 512, 256, 51), (1, 40, 7, 13), (64, 100, 3, 20), (33, 70, 130, 70), (7, 2000, 24, 9),
    (64, 300, 64, 106)])
@pytest.mark.parametrize("order", ["simd", "scalar"])
def test_backward_narrow_bit_exact(dev, M, K, N, per_row, order):
    """slk_backward_narrow from the token-major gradient: dW is the oracle's
    in each summation order, dbias the same bits as slk_sddmm_bias's, and dX
    the reference's spmm(WT, dY) bit for bit (rows without slots, columns no
    row holds, N not a multiple of 4, a W of 8000 slots)."""
    print(f"[narrow bwd] M={M} K={K} N={N} {order}", flush=True)
    c, X_np, dY_np, _ = _narrow_case(M, K, N, per_row, seed=M * K + N, empty=(M // 2,))
    W = from_oracle(c, dev)
    assert W.total_capacity <= _lib.NARROW_MAX_CAPACITY
    X, dYt = _t(X_np, dev), _t(np.ascontiguousarray(dY_np.T), dev)
    ordv = _lib.SLK_DW_SCALAR if order == "scalar" else _lib.SLK_DW_SIMD
    dW = torch.full((W.total_capacity,), float("nan"), device=dev)
    db = torch.full((M,), float("nan"), device=dev)
    dX = torch.full((K, N), float("nan"), device=dev)
    _lib.backward_narrow(W._view(), dYt, X, dW, db, dX, ordv)
    assert_bits_equal(dW.cpu().numpy(), oracle.sddmm(c, dY_np, X_np, order), "dW")
    WT, _ = oracle.transpose_with_perm(c)
    assert_bits_equal(dX.cpu().numpy(), oracle.spmm(WT, dY_np), "dX")
    db_ref = torch.empty(M, device=dev)
    _lib.sddmm(W._view(), _t(dY_np, dev), X, torch.empty_like(dW), ordv, db_ref)
    assert torch.equal(db, db_ref)
    # each output alone
    for want in ("dW", "dbias", "dX"):
        outs = {"dW": None, "dbias": None, "dX": None}
        outs[want] = {"dW": torch.empty_like(dW), "dbias": torch.empty_like(db),
                      "dX": torch.empty_like(dX)}[want]
        _lib.backward_narrow(W._view(), dYt, X, outs["dW"], outs["dbias"], outs["dX"], ordv)
        assert torch.equal(outs[want], {"dW": dW, "dbias": db, "dX": dX}[want]), want


def test_backward_narrow_rejects_wide_layers(dev):
    c, X_np, dY_np, _ = _narrow_case(65, 20, 8, 3, seed=1)
    W = from_oracle(c, dev)
    dYt = _t(np.ascontiguousarray(dY_np.T), dev)
    with pytest.raises(ValueError, match="at most 64 rows"):
        _lib.backward_narrow(W._view(), dYt, _t(X_np, dev), None, None,
                             torch.empty(20, 8, device=dev), _lib.SLK_DW_SIMD)
    c2, X2, dY2, _ = _narrow_case(8, 3000, 4, 1100, seed=2)
    W2 = from_oracle(c2, dev)
    assert W2.total_capacity > _lib.NARROW_MAX_CAPACITY
    with pytest.raises(ValueError, match="slots"):
        _lib.backward_narrow(W2._view(), _t(np.ascontiguousarray(dY2.T), dev), _t(X2, dev),
                             torch.empty(W2.total_capacity, device=dev), None, None,
                             _lib.SLK_DW_SIMD)


def _expected_seg_list(c, block, S, n):
    """The padded segment list, restated in numpy: for every column block, for
    every row, the row's run of live slots in the block cut into segments of at
    most S slots; each block padded with empty segments (row 0, slot 0, count 0)
    to a multiple of SEG_GROUP; each group of SEG_GROUP segments then stably
    sorted by count, largest first; n entries in all."""
    G = _lib.SEG_GROUP
    start, row, cnt = [], [], []
    nb = -(-c.ncols // block)
    for b in range(nb):
        k0 = len(start)
        for r in range(c.nrows):
            s0 = int(c.row_start[r])
            cols = c.col_indices[s0:s0 + int(c.row_nnz[r])]
            a = s0 + int(np.searchsorted(cols, b * block))
            e = s0 + int(np.searchsorted(cols, (b + 1) * block))
            for s in range(a, e, S):
                start.append(s)
                row.append(r)
                cnt.append(min(S, e - s))
        pad = (-(len(start) - k0)) % G
        start += [0] * pad
        row += [0] * pad
        cnt += [0] * pad
    groups = len(start) // G
    for g in range(groups):
        sl = slice(g * G, (g + 1) * G)
        order = np.argsort(-np.asarray(cnt[sl]), kind="stable")
        start[sl], row[sl], cnt[sl] = ([v[sl][i] for i in order] for v in (start, row, cnt))
    assert len(start) <= n
    fill = n - len(start)
    as32 = lambda v: np.asarray(v + [0] * fill, dtype=np.int32)
    return as32(start), as32(row), as32(cnt), groups


@pytest.mark.parametrize("S", [4, 8])
@pytest.mark.parametrize("shape,density,block", [
    ((150, 300), 0.06, 64),
    ((150, 300), 0.3, 128),
    ((3000, 257), 0.02, 64),      # more rows than the scan's 1024 threads
    ((5, 4100), 0.3, 128),        # 33 blocks, a last block of 4 columns
    ((64, 64), 1.0, 64),          # fully dense: 16 or 8 full segments per row
])
def test_seg_list_build_matches_the_restatement(dev, S, shape, density, block):
    """slk_seg_list_build writes exactly the numpy restatement's padded list
    (segments block by block and row by row, runs cut every S slots, blocks
    padded to whole groups, each group sorted by count, the rest of the arrays
    empty) and the group count, for skewed rows including an empty one."""
    M, K = shape
    print(f"[seg list] S={S} shape={shape} d={density} block={block}", flush=True)
    c = oracle.zipf_rows(M, K, density, 1.1, seed=M + K + block + S, sigma=0.5)
    c.row_nnz[M // 2] = 0
    c.col_indices[c.row_start[M // 2]:c.row_start[M // 2] + c.row_capacity[M // 2]] = -1
    W = from_oracle(c, dev)
    start, row, cnt, groups = _lib.seg_list_build(W._view(), block, S, dev)
    want = _expected_seg_list(c, block, S, start.numel())
    assert np.array_equal(start.cpu().numpy(), want[0])
    assert np.array_equal(row.cpu().numpy(), want[1])
    assert np.array_equal(cnt.cpu().numpy(), want[2])
    assert int(groups.item()) == want[3]


def test_seg_list_build_rejects_bad_arguments(dev):
    c = oracle.zipf_rows(16, 32, 0.2, 1.1, seed=3)
    W = from_oracle(c, dev)
    with pytest.raises(ValueError, match="block_cols"):
        _lib.seg_list_build(W._view(), 32, 4, dev)
    with pytest.raises(ValueError, match="seg_slots"):
        _lib.seg_list_build(W._view(), 64, 6, dev)
    lib = _lib.load()
    view = W._view()
    n = int(lib.slk_seg_list_capacity(ctypes.byref(view), 64, 4))
    out = torch.empty(n, dtype=torch.int32, device=dev)
    rc = lib.slk_seg_list_build(ctypes.byref(view), 64, 4, None, 0, _lib.ptr(out), _lib.ptr(out),
                                _lib.ptr(out), n - 1, _lib.ptr(out), None)
    assert rc != 0 and b"n_seg" in lib.slk_last_error()


@pytest.mark.parametrize("block,S", [(64, 4), (64, 8), (128, 4), (128, 8)])
@pytest.mark.parametrize("M,K,density,N", [
    (200, 256, 0.5, 1024),    # dense rows: several full segments per run
    (3000, 300, 0.02, 1100),  # sparse skewed rows: many short segments, many groups
    (700, 200, 0.1, 1032),    # partial last window, 8-wide step
    (500, 130, 0.2, 1045),    # scalar tail, a last block narrower than the block width
    (90, 150, 0.3, 16),       # one 16-float step: a single, partial window
    (90, 150, 0.3, 60),       # 8-wide step and tail after three steps
])
def test_sddmm_seg_kernel_bit_exact(dev, block, S, M, K, density, N):
    """slk_sddmm on a segment list (X staged in LDS per workgroup, each
    segment's dY row in registers) gives the oracle's bits: full and partial
    windows, the 8-wide step and scalar tail, narrow last blocks, empty rows,
    empty padding segments, zeroed padding slots and the fused bias gradient."""
    print(f"[dW seg] block={block} S={S} M={M} K={K} d={density} N={N}", flush=True)
    c = oracle.zipf_rows(M, K, density, 0.6, seed=M + N + S, sigma=0.5)
    c.row_nnz[M // 3] = 0
    c.col_indices[c.row_start[M // 3]:c.row_start[M // 3] + c.row_capacity[M // 3]] = -1
    rng = np.random.default_rng(N + S)
    X_np = rng.standard_normal((K, N)).astype(np.float32)
    dY_np = rng.standard_normal((M, N)).astype(np.float32)
    W = from_oracle(c, dev)
    X, dY = _t(X_np, dev), _t(dY_np, dev)
    view = W._view_segmented(block, S)
    assert view.seg_block == block and view.seg_slots == S
    dW = torch.full((W.total_capacity,), float("nan"), device=dev)
    db = torch.full((M,), float("nan"), device=dev)
    _lib.sddmm(view, dY, X, dW, _lib.SLK_DW_SIMD, db)
    assert_bits_equal(dW.cpu().numpy(), oracle.sddmm(c, dY_np, X_np), "dW seg")
    db_ref = torch.empty(M, device=dev)
    _lib.sddmm(W._view(), dY, X, torch.empty_like(dW), _lib.SLK_DW_SIMD, db_ref)
    assert torch.equal(db, db_ref)
    dW2 = torch.full((W.total_capacity,), float("nan"), device=dev)
    _lib.sddmm(view, dY, X, dW2, _lib.SLK_DW_SIMD)
    assert_bits_equal(dW2.cpu().numpy(), oracle.sddmm(c, dY_np, X_np), "dW seg, no bias")


@pytest.mark.parametrize("P", [1, 2, 3, 7, 40])
def test_phase_bounds_build_matches_searchsorted(dev, P):
    """slk_phase_bounds_build gives, for every row and phase boundary
    p * ceil(K / P), the first live slot at or past that column (numpy's
    searchsorted over the row's ascending columns), empty rows included."""
    c = oracle.zipf_rows(700, 300, 0.05, 1.1, seed=P, sigma=0.5)
    c.row_nnz[5] = 0
    c.col_indices[c.row_start[5]:c.row_start[5] + c.row_capacity[5]] = -1
    W = from_oracle(c, dev)
    lo = _lib.phase_bounds_build(W._view(), P, dev).cpu().numpy().reshape(700, P + 1)
    C = -(-300 // P)
    for r in range(700):
        s0 = int(c.row_start[r])
        cols = c.col_indices[s0:s0 + int(c.row_nnz[r])]
        want = s0 + np.searchsorted(cols, np.arange(P + 1) * C)
        assert np.array_equal(lo[r], want), r


@pytest.mark.parametrize("P", [2, 3, 7])
@pytest.mark.parametrize("N,order", [(1024, True), (1032, False), (260, True)])
def test_spmm_phased_sweep_bit_exact(dev, tune, P, N, order):
    """The 16-byte gather kernel swept in P column phases, each row's fma chain
    resumed from the partial sums the previous phase left in Y, gives the
    one-pass chain's bits — with and without bias (added once, after the last
    phase), under the longest-first row order and without one, for rows from
    fully dense to empty."""
    tune(spmm_kernel=0)
    tune(spmm_vec=4)
    print(f"[spmm phased] P={P} N={N} order={order}", flush=True)
    c = oracle.zipf_rows(2500, 600, 0.02, 1.1, seed=P + N, sigma=0.5)
    c.row_nnz[11] = 0
    c.col_indices[c.row_start[11]:c.row_start[11] + c.row_capacity[11]] = -1
    rng = np.random.default_rng(P * N)
    X_np = rng.standard_normal((600, N)).astype(np.float32)
    b_np = rng.standard_normal(2500).astype(np.float32)
    W = from_oracle(c, dev)
    v = W._view_phased(P)
    assert v.n_phases == P and v.phase_lo is not None
    if not order:
        v = _with_fields(v, row_order=None, n_heavy_rows=0)
    X = _t(X_np, dev)
    want = oracle.spmm(c, X_np)
    Y = torch.full((2500, N), float("nan"), device=dev)
    _lib.spmm(v, X, Y)
    assert_bits_equal(Y.cpu().numpy(), want, "Y phased")
    _lib.spmm(v, X, Y, _t(b_np, dev))
    assert_bits_equal(Y.cpu().numpy(), want + b_np[:, None], "Y+bias phased")
