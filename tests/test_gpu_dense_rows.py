"""GPU parity of slk_spmm's dense rows (slk_csr.n_dense_rows) and of the
matrix-core instruction they rest on.

* The instruction. slk_dense_mfma_probe runs one fp32 32x32x1 two-block MFMA
  (v_mfma_f32_32x32x1_2b_f32) on given lane operands and accumulator
  registers. Every output register must equal libm's fmaf (oracle.fmaf) of
  the A and B lanes and the C register that the documented layout names, bit
  for bit (NaN as NaN), over random operands, cancelling sums (c = -fl(a·b)
  plus a few ulps: only a fused product gets these right), subnormal operands
  and results, exponents across the whole range, and ±0 / ±inf / NaN mixes.
  The dense-row kernel is correct only if this holds.
* The forward. The densest rows of a tall matrix (the head of its row order)
  run as dense rows on the matrix cores; Y must equal the oracle (the
  reference's slot-order chain) under ==, bit for bit except possibly the
  sign of a zero, on shapes that reach the kernel's edges: dense-row counts
  that are not a multiple of a workgroup's 128 rows, K not a multiple of 4,
  N not a multiple of 64 and below one column tile, fully dense rows, rows
  at the density bar, explicit zero values, bias. The dense rows forced back
  onto the other kernels (SLK_TUNE_DENSE_ROWS = 0) give the same values. X
  with inf and NaN (in columns that dense rows skip) takes the recompute path
  and still equals the oracle.
* The weight gradient. With a segment list that leaves the dense rows out
  (slk_csr.seg_dense_rows), slk_sddmm computes their live slots on the matrix
  cores in the reference's SIMD order; dW (padding included) and dbias must
  equal the oracle's bit for bit, and the list must hold no segment of a
  dense row. A view whose N the dense kernel cannot take (not a multiple of
  64) is refused, and ops then picks a list with the dense rows in it.
Bar: bit-exact (the forward's zeros compared by value).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from helpers import from_oracle
from sparsecore_amd import _lib, layout, ops

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _assert_equal_values(got, want, what):
    """Equal under == with NaN equal to NaN; any bit difference is a zero's sign."""
    got = np.ascontiguousarray(got, dtype=np.float32)
    want = np.ascontiguousarray(want, dtype=np.float32)
    assert got.shape == want.shape, what
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    bad = np.flatnonzero(~same.reshape(-1))
    assert bad.size == 0, (f"{what}: {bad.size} of {got.size} differ, first at {int(bad[0])}: "
                           f"{got.reshape(-1)[bad[0]]!r} vs {want.reshape(-1)[bad[0]]!r}")
    bits = got.view(np.uint32) != want.view(np.uint32)
    fin = ~np.isnan(got)
    assert np.all(got[bits & fin] == 0.0), f"{what}: non-zero values differ in bits"


# ───────────────────────────── the instruction ─────────────────────────────

def _layout_lanes():
    """(A lane, B lane) of lane l's accumulator register r."""
    l = np.arange(64)[:, None]
    r = np.arange(32)[None, :]
    blk, rr = r // 16, r % 16
    a = 32 * blk + 8 * (rr // 4) + 4 * (l // 32) + rr % 4
    b = 32 * blk + l % 32 + 0 * r
    return a, b


def _probe_operands(kind, n, rng):
    def rnd(lo, hi, shape):
        return np.ldexp(rng.standard_normal(shape), rng.integers(lo, hi + 1, shape)).astype(np.float32)

    if kind == "normal":
        A, B = rng.standard_normal((n, 64)), rng.standard_normal((n, 64))
        C = rng.standard_normal((n, 64, 32))
    elif kind == "wide":
        A, B, C = rnd(-60, 60, (n, 64)), rnd(-60, 60, (n, 64)), rnd(-120, 120, (n, 64, 32))
    elif kind == "subnormal":
        A, B = rnd(-75, -55, (n, 64)), rnd(-75, -55, (n, 64))
        C = np.where(rng.random((n, 64, 32)) < 0.5, rnd(-149, -126, (n, 64, 32)), 0.0)
    elif kind == "special":
        sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 1e-45, 3e38], np.float32)
        A, B = sp[rng.integers(0, 9, (n, 64))], sp[rng.integers(0, 9, (n, 64))]
        C = sp[rng.integers(0, 7, (n, 64, 32))]
    else:  # cancel: C = -fl(a*b) moved by up to 3 ulps
        A, B = rng.standard_normal((n, 64)), rng.standard_normal((n, 64))
        C = None
    A, B = A.astype(np.float32), B.astype(np.float32)
    if C is None:
        al, bl = _layout_lanes()
        p = (A[:, al] * B[:, bl]).astype(np.float32)
        C = -((p.view(np.int32) + rng.integers(-3, 4, p.shape).astype(np.int32)).view(np.float32))
    return A, B, np.asarray(C, np.float32)


@pytest.mark.parametrize("kind", ["normal", "cancel", "subnormal", "wide", "special"])
def test_fp32_mfma_outer_product_is_an_fma(dev, kind):
    print(f"[dense mfma probe] {kind}", flush=True)
    rng = np.random.default_rng(["normal", "cancel", "subnormal", "wide", "special"].index(kind))
    n = 512
    A, B, C = _probe_operands(kind, n, rng)
    D = torch.empty((n, 64, 32), dtype=torch.float32, device=dev)
    _lib.dense_mfma_probe(_t(A, dev), _t(B, dev), _t(C, dev), D)
    got = D.cpu().numpy()
    al, bl = _layout_lanes()
    want = oracle.fmaf(A[:, al], B[:, bl], C)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    if kind == "cancel":  # the cases an unfused multiply-add gets wrong are present
        unfused = (A[:, al] * B[:, bl]).astype(np.float32) + C
        assert np.count_nonzero(unfused != want) > 1000


def test_fp32_mfma_chain_of_4096_steps_equals_the_fma_chain(dev):
    """4096 probe calls feeding the accumulator back: one running fma chain."""
    print("[dense mfma probe] chain", flush=True)
    rng = np.random.default_rng(7)
    steps, n = 4096, 4
    A = rng.standard_normal((steps, n, 64)).astype(np.float32)
    B = rng.standard_normal((steps, n, 64)).astype(np.float32)
    acc = torch.zeros((n, 64, 32), dtype=torch.float32, device=dev)
    out = torch.empty_like(acc)
    Ad, Bd = _t(A, dev), _t(B, dev)
    for s in range(steps):
        _lib.dense_mfma_probe(Ad[s], Bd[s], acc, out)
        acc, out = out, acc
    al, bl = _layout_lanes()
    want = np.zeros((n, 64, 32), np.float32)
    for s in range(steps):
        want = oracle.fmaf(A[s][:, al], B[s][:, bl], want)
    np.testing.assert_array_equal(acc.cpu().numpy().view(np.uint32), want.view(np.uint32))


# ───────────────────────────── the forward ─────────────────────────────────

def _matrix(M, K, n_dense, seed, *, full=1, at_bar=2, zeros=True):
    """M x K padded-CSR: n_dense rows between 30% and 100% dense (`full` of
    them completely, `at_bar` exactly at the dense bar and one just below it),
    the rest about 1% dense, in a shuffled row order."""
    rng = np.random.default_rng(seed)
    bar = int(np.ceil(layout.DENSE_ROW_FRACTION * K))
    nnz = rng.integers(max(1, K // 200), max(2, K // 50), M)
    nnz[:n_dense] = rng.integers(int(0.3 * K), K, n_dense)
    nnz[:full] = K
    nnz[full:full + at_bar] = bar
    nnz[n_dense] = bar - 1  # one row just below the bar (not dense)
    perm = rng.permutation(M)
    nnz = nnz[perm]
    cols, vals = [], []
    for i in range(M):
        c = np.sort(rng.choice(K, int(nnz[i]), replace=False)).astype(np.int32)
        v = rng.standard_normal(c.size).astype(np.float32) * 0.05
        if zeros and c.size > 3:
            v[rng.integers(0, c.size, 2)] = 0.0  # explicit zero values are live slots
        cols.append(c)
        vals.append(v)
    return oracle.from_row_lists(M, K, cols, vals)


@pytest.mark.parametrize("M,K,n_dense,N", [(2100, 4099, 150, 300), (2048, 4096, 128, 64),
                                           (2300, 5003, 40, 37), (2200, 4100, 257, 200)])
@pytest.mark.parametrize("bias", [False, True])
def test_dense_rows_forward_equals_the_oracle(dev, M, K, n_dense, N, bias):
    print(f"[dense rows] {M}x{K} dense={n_dense} N={N} bias={bias}", flush=True)
    c = _matrix(M, K, n_dense, seed=M + N)
    W = from_oracle(c, dev)
    v = W._view()
    # the full rows, the rows at the bar and the random dense ones, not the one below it
    assert v.n_dense_rows == n_dense and v.dense_ws is not None
    rng = np.random.default_rng(N)
    X = rng.standard_normal((K, N)).astype(np.float32)
    b = rng.standard_normal(M).astype(np.float32) if bias else None
    want = oracle.spmm(c, X)
    if bias:
        want = (want + b[:, None]).astype(np.float32)
    Xd = _t(X, dev)
    Y = torch.empty((M, N), dtype=torch.float32, device=dev)
    bd = _t(b, dev) if bias else None
    _lib.spmm(v, Xd, Y, bd)
    _assert_equal_values(Y.cpu().numpy(), want, "Y")
    # the same rows through the other kernels
    Y2 = torch.full_like(Y, float("nan"))
    _lib.set_tuning("dense_rows", 0)
    try:
        _lib.spmm(v, Xd, Y2, bd)
    finally:
        _lib.set_tuning("dense_rows", None)
    _assert_equal_values(Y2.cpu().numpy(), want, "Y without dense rows")


@pytest.mark.parametrize("n_heavy", [0, 150, 420])
def test_dense_rows_beside_the_phased_gather(dev, n_heavy):
    """Phase bounds put the light rows on the phased gather of the side
    stream: the dense rows run on the caller's stream beside it, and the
    heavy rows beyond the dense ones (none when n_heavy <= n_dense) on the
    LDS kernel after them."""
    M, K, n_dense, N = 2200, 4100, 300, 1024
    print(f"[dense rows] phased {M}x{K} dense={n_dense} heavy={n_heavy} N={N}", flush=True)
    c = _matrix(M, K, n_dense, seed=11 + n_heavy)
    W = from_oracle(c, dev)
    # the constructor's device check built the row order: rebuild it with the hint
    W._heavy_hint, W._order, W._cview = n_heavy, None, None
    v = W._view_phased(3)
    assert v.n_dense_rows == n_dense and v.n_heavy_rows == n_heavy and v.n_phases == 3
    rng = np.random.default_rng(n_heavy)
    X = rng.standard_normal((K, N)).astype(np.float32)
    b = rng.standard_normal(M).astype(np.float32)
    want = (oracle.spmm(c, X) + b[:, None]).astype(np.float32)
    Y = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    _lib.spmm(v, _t(X, dev), Y, _t(b, dev))
    _assert_equal_values(Y.cpu().numpy(), want, "Y")


@pytest.mark.parametrize("bad", ["inf", "nan", "inf-in-dense-column", "overflow"])
def test_dense_rows_nonfinite_inputs_take_the_recompute(dev, bad):
    print(f"[dense rows] non-finite {bad}", flush=True)
    M, K, N = 2100, 4099, 130
    c = _matrix(M, K, 60, seed=11, full=0)
    W = from_oracle(c, dev)
    v = W._view()
    assert v.n_dense_rows == 60
    rng = np.random.default_rng(5)
    X = rng.standard_normal((K, N)).astype(np.float32)
    order = W._order[1].cpu().numpy()
    d0 = int(order[0])
    live = set(c.col_indices[c.row_start[d0]:c.row_start[d0] + c.row_nnz[d0]].tolist())
    skipped = next(k for k in range(K) if k not in live)
    if bad == "inf":
        X[skipped, 5] = np.inf   # dense row d0 skips column `skipped`: the reference never reads it
    elif bad == "nan":
        X[skipped, 70] = np.nan
        X[skipped + 1 if skipped + 1 not in live else skipped, 71] = -np.inf
    elif bad == "inf-in-dense-column":
        k = sorted(live)[3]
        X[k, 9] = np.inf         # a live column: the reference's chain becomes non-finite too
    else:
        X[:, 3] = 3e38           # finite inputs whose chains overflow
    want = oracle.spmm(c, X)
    Y = torch.empty((M, N), dtype=torch.float32, device=dev)
    _lib.spmm(v, _t(X, dev), Y)
    _assert_equal_values(Y.cpu().numpy(), want, "Y")


def test_dense_rows_follow_the_values_and_the_topology(dev):
    """The dense copy is rebuilt from W's values on every call; a topology
    change rebuilds the row schedule and its dense-row count."""
    print("[dense rows] values and topology", flush=True)
    M, K, N = 2100, 4099, 100
    c = _matrix(M, K, 100, seed=3)
    W = from_oracle(c, dev)
    rng = np.random.default_rng(1)
    X = rng.standard_normal((K, N)).astype(np.float32)
    Xd = _t(X, dev)
    Y = ops.spmm(W, Xd)
    _assert_equal_values(Y.cpu().numpy(), oracle.spmm(c, X), "Y")
    with torch.no_grad():
        W.values.mul_(-1.5)
    c2 = oracle.Csr(c.nrows, c.ncols, W.values.cpu().numpy(), c.col_indices, c.row_start,
                    c.row_nnz, c.row_capacity)
    _assert_equal_values(ops.spmm(W, Xd).cpu().numpy(), oracle.spmm(c2, X), "Y after a values change")
    # a dense row rewritten sparse leaves the dense set
    order = W._order[1].cpu().numpy()
    W.rewrite_row(int(order[0]), np.arange(5), np.ones(5, np.float32))
    assert W._view().n_dense_rows == 99
    c3 = oracle.Csr(W.nrows, W.ncols, W.values.cpu().numpy(), W.col_indices.cpu().numpy(),
                    W.row_start.cpu().numpy(), W.row_nnz.cpu().numpy(), W.row_capacity.cpu().numpy())
    _assert_equal_values(ops.spmm(W, Xd).cpu().numpy(), oracle.spmm(c3, X), "Y after rewrite_row")


# ───────────────────────────── the weight gradient ─────────────────────────

@pytest.mark.parametrize("M,K,n_dense,N,seg", [(2100, 4099, 150, 256, (64, 8)),
                                               (2200, 4100, 257, 192, (128, 8)),
                                               (2048, 4096, 40, 64, (64, 4)),
                                               (2300, 5003, 130, 1024, None)])
@pytest.mark.parametrize("bias", [False, True])
def test_dense_rows_dw_equals_the_oracle(dev, M, K, n_dense, N, seg, bias):
    print(f"[dense dW] {M}x{K} dense={n_dense} N={N} seg={seg} bias={bias}", flush=True)
    c = _matrix(M, K, n_dense, seed=3 * M + N)
    W = from_oracle(c, dev)
    rng = np.random.default_rng(N + 1)
    X = rng.standard_normal((K, N)).astype(np.float32)
    dY = rng.standard_normal((M, N)).astype(np.float32)
    Xd, dYd = _t(X, dev), _t(dY, dev)
    old = dict(ops._overrides)
    try:
        ops._overrides["dense_dw"] = True  # any count of dense rows
        if seg is not None:
            ops._overrides["seg"] = seg
        v = ops._sddmm_view(W, Xd)
        assert v.n_dense_rows == n_dense and v.seg_dense_rows == n_dense
        # the list holds no segment of a dense row
        start, row, count, groups = W._seglist[3]
        used = count.cpu().numpy() > 0
        dense = set(W._order[1][:n_dense].cpu().numpy().tolist())
        assert not dense & set(row.cpu().numpy()[used].tolist())
        dW = torch.full((W.total_capacity,), float("nan"), device=dev)
        db = torch.full((M,), float("nan"), device=dev) if bias else None
        _lib.sddmm(v, dYd, Xd, dW, _lib.SLK_DW_SIMD, db)
        want = oracle.sddmm(c, dY, X, "simd")
        np.testing.assert_array_equal(dW.cpu().numpy().view(np.uint32), want.view(np.uint32))
        if bias:  # the same sums as the view without dense rows gives
            ops._overrides["dense_dw"] = False
            v2 = ops._sddmm_view(W, Xd)
            assert v2.seg_dense_rows == 0
            dW2 = torch.full_like(dW, float("nan"))
            db2 = torch.full_like(db, float("nan"))
            _lib.sddmm(v2, dYd, Xd, dW2, _lib.SLK_DW_SIMD, db2)
            np.testing.assert_array_equal(db.cpu().numpy().view(np.uint32),
                                          db2.cpu().numpy().view(np.uint32))
            np.testing.assert_array_equal(dW2.cpu().numpy().view(np.uint32), want.view(np.uint32))
    finally:
        ops._overrides.clear()
        ops._overrides.update(old)


def test_dense_rows_dw_refuses_an_n_it_cannot_take(dev):
    print("[dense dW] refused N", flush=True)
    M, K, N = 2100, 4099, 256
    c = _matrix(M, K, 40, seed=8)
    W = from_oracle(c, dev)
    rng = np.random.default_rng(2)
    Xd = _t(rng.standard_normal((K, N)).astype(np.float32), dev)
    v = W._view_segmented(64, 8, skip_dense=True)
    assert v.seg_dense_rows == 40
    X2 = _t(rng.standard_normal((K, 200)).astype(np.float32), dev)  # 200 % 64 != 0
    dY2 = _t(rng.standard_normal((M, 200)).astype(np.float32), dev)
    dW = torch.empty(W.total_capacity, device=dev)
    with pytest.raises(ValueError, match="multiple of 64"):
        _lib.sddmm(v, dY2, X2, dW, _lib.SLK_DW_SIMD, None)
    # ops picks a list with the dense rows for such an N, and the oracle's bits
    want = oracle.sddmm(c, dY2.cpu().numpy(), X2.cpu().numpy(), "simd")
    old = dict(ops._overrides)
    try:
        ops._overrides["seg"] = (64, 8)
        v2 = ops._sddmm_view(W, X2)
        assert v2.seg_dense_rows == 0
        _lib.sddmm(v2, dY2, X2, dW, _lib.SLK_DW_SIMD, None)
    finally:
        ops._overrides.clear()
        ops._overrides.update(old)
    np.testing.assert_array_equal(dW.cpu().numpy().view(np.uint32), want.view(np.uint32))
    del Xd
