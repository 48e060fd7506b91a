"""Pins the CPU oracle before it is trusted as the GPU path's checker.

Each oracle function is checked against something it does not share code
with: the reference's own kernels compiled from the reference sources
(oracle/_ref, bit-exact), the committed golden fixtures made from that build,
float64 closed forms (W @ X, dY @ Xᵀ), brute force on small inputs, and the
literal known answers of the reference tests.
"""

from __future__ import annotations

import json

import numpy as np
import pytest

import oracle
from helpers import GOLDEN, assert_bits_equal, c1_inputs, golden_cases, golden_csr

needs_ref = pytest.mark.skipif(not oracle.ref_available(),
                               reason="oracle/_ref (reference build) not present")

N_SWEEP = [0, 1, 2, 3, 4, 5, 7, 8, 9, 12, 15, 16, 17, 20, 23, 24, 31, 32, 33, 47, 64, 65, 100, 255,
           256, 257]


def _inputs(M, K, N, per_row, seed):
    p = oracle.uniform_rows(M, K, per_row, seed=seed, sigma=1.0)
    rng = np.random.default_rng(seed + 7)
    X = rng.standard_normal((K, N)).astype(np.float32)
    dY = rng.standard_normal((M, N)).astype(np.float32)
    return p, X, dY


# ───────────────────── against the reference build ─────────────────────

@needs_ref
@pytest.mark.parametrize("N", N_SWEEP)
def test_kernels_bit_exact_vs_reference_build(N):
    p, X, dY = _inputs(24, 37, N, 9, seed=N)
    ref = oracle.RefCsr(p)
    assert_bits_equal(oracle.spmm(p, X), ref.spmm(X, "simd"), "spmm vs spmm_simd")
    assert_bits_equal(oracle.spmm(p, X), ref.spmm(X, "scalar"), "spmm vs spmm_scalar")
    assert_bits_equal(oracle.sddmm(p, dY, X, "simd"), ref.sddmm(dY, X, "simd"), "dW simd")
    assert_bits_equal(oracle.sddmm(p, dY, X, "scalar"), ref.sddmm(dY, X, "scalar"), "dW scalar")
    assert_bits_equal(oracle.dense_grad(dY, X), oracle.ref_dense_grad(dY, X), "dense_grad")


@needs_ref
def test_kernels_bit_exact_vs_reference_build_threaded_sizes():
    # >= 32 rows takes the OpenMP path in both builds.
    p, X, dY = _inputs(300, 500, 130, 50, seed=3)
    ref = oracle.RefCsr(p)
    assert_bits_equal(oracle.spmm(p, X), ref.spmm(X), "spmm")
    assert_bits_equal(oracle.sddmm(p, dY, X), ref.sddmm(dY, X), "dW")


@needs_ref
def test_invariant_messages_match_reference_checker():
    rng = np.random.default_rng(0)
    base = oracle.uniform_rows(12, 20, 5, seed=1)
    corruptions = []
    for trial in range(60):
        q = base.copy()
        kind = trial % 6
        i = int(rng.integers(0, q.nrows))
        s, n, cap = int(q.row_start[i]), int(q.row_nnz[i]), int(q.row_capacity[i])
        if kind == 0:
            q.col_indices[s + int(rng.integers(0, n))] = int(rng.integers(-3, 25))
        elif kind == 1 and n >= 2:
            q.col_indices[s], q.col_indices[s + 1] = q.col_indices[s + 1], q.col_indices[s]
        elif kind == 2 and cap > n:
            q.col_indices[s + n] = int(rng.integers(0, 20))
        elif kind == 3:
            q.row_nnz[i] = cap + 1
        elif kind == 4 and i > 0:
            q.row_start[i] += 1
        elif kind == 5:
            q.row_nnz[i] = max(0, n - 1)  # leaves a live column in a padding slot
        corruptions.append(q)
    for q in corruptions:
        expect = oracle.RefCsr(q).check_invariants()
        got = oracle.check_invariants(q.nrows, q.ncols, q.values, q.col_indices, q.row_start,
                                      q.row_nnz, q.row_capacity)
        assert got == expect


@needs_ref
def test_rewrite_row_matches_reference():
    p = oracle.uniform_rows(6, 30, 8, seed=4)
    ref = oracle.RefCsr(p)
    q = p
    for row, cols in [(0, [1, 5, 9]), (3, []), (5, list(range(0, 30, 3))[:9]), (3, [29])]:
        vals = np.arange(len(cols), dtype=np.float32) + 0.5
        ref.rewrite_row(row, cols, vals)
        q = oracle.rewrite_row(q, row, cols, vals)
    v, c, nz, ver = ref.arrays()
    assert_bits_equal(q.values, v, "values")
    assert_bits_equal(q.col_indices, c, "cols")
    assert_bits_equal(q.row_nnz, nz, "row_nnz")
    assert ver == 4


# ───────────────────────── golden fixtures ─────────────────────────────

@pytest.mark.parametrize("name", sorted(golden_cases()))
def test_oracle_matches_golden_fixture(name):
    case = golden_cases()[name]
    p = golden_csr(case)
    assert oracle.check_invariants(p.nrows, p.ncols, p.values, p.col_indices, p.row_start,
                                   p.row_nnz, p.row_capacity) == ""
    assert_bits_equal(oracle.spmm(p, case["X"]), case["Y"], "Y")
    assert_bits_equal(oracle.sddmm(p, case["dY"], case["X"], "simd"), case["dW"], "dW")
    assert_bits_equal(oracle.sddmm(p, case["dY"], case["X"], "scalar"), case["dW_scalar"],
                      "dW_scalar")
    WT, _ = oracle.transpose_with_perm(p)
    assert_bits_equal(oracle.spmm(WT, case["dY"]), case["dX"], "dX")


def test_oracle_matches_c1_digests():
    import gen

    meta, p, X, dY = c1_inputs()
    WT, _ = oracle.transpose_with_perm(p)
    outs = {"Y": oracle.spmm(p, X), "dW": oracle.sddmm(p, dY, X, "simd"),
            "dW_scalar": oracle.sddmm(p, dY, X, "scalar"), "dX": oracle.spmm(WT, dY)}
    for k, v in outs.items():
        assert gen.digest(v) == meta["outputs_sha256"][k], k


def test_golden_check_has_teeth():
    """A planted mistake in the oracle (a float64 dot instead of the reference
    order) must fail the bit-exact golden comparison."""
    case = golden_cases()["n33"]
    p = golden_csr(case)
    slots, rows, cols = oracle.live_slots(p)
    wrong = np.zeros(p.total_capacity, np.float32)
    wrong[slots] = np.einsum("ij,ij->i", case["dY"][rows].astype(np.float64),
                             case["X"][cols].astype(np.float64)).astype(np.float32)
    assert not np.array_equal(wrong.view(np.uint32), case["dW"].view(np.uint32))
    assert np.allclose(wrong, case["dW"], rtol=1e-5, atol=1e-5)


# ──────────────────────── closed forms (float64) ───────────────────────

@pytest.mark.parametrize("M,K,N,per_row", [(32, 32, 32, 3), (128, 64, 16, 6), (64, 128, 256, 13),
                                           (7, 13, 5, 4), (1, 1, 1, 1), (50, 40, 3, 40)])
def test_oracle_vs_dense_float64(M, K, N, per_row):
    """|float32 result - exact| <= 1e-5 * sum|terms| (an n-term float32 sum errs by at
    most ~n * 2^-24 * sum|terms|); a dropped, doubled or misplaced term breaks it."""
    p, X, dY = _inputs(M, K, N, per_row, seed=M * 1000 + N)
    X64, dY64 = X.astype(np.float64), dY.astype(np.float64)
    Wd = oracle.dense_from_csr64(p)

    def within(ours, exact, scale):
        assert np.all(np.abs(ours.astype(np.float64) - exact) <= 1e-5 * scale + 1e-30)

    within(oracle.spmm(p, X), Wd @ X64, np.abs(Wd) @ np.abs(X64))
    G = dY64 @ X64.T
    Gabs = np.abs(dY64) @ np.abs(X64).T
    slots, rows, cols = oracle.live_slots(p)
    for order in ("simd", "scalar"):
        dW = oracle.sddmm(p, dY, X, order)
        within(dW[slots], G[rows, cols], Gabs[rows, cols])
        assert np.all(dW[oracle.padding_slots(p)] == 0.0)
    within(oracle.dense_grad(dY, X), G, Gabs)
    WT, _ = oracle.transpose_with_perm(p)
    within(oracle.spmm(WT, dY), Wd.T @ dY64, np.abs(Wd.T) @ np.abs(dY64))


# ─────────────────────────── transpose ─────────────────────────────────

def _transpose_brute(p: oracle.Csr, pr: float):
    """Per column, scan rows in order (O(M*K) python; small inputs only)."""
    dense = oracle.to_dense(p)
    live = np.zeros((p.nrows, p.ncols), dtype=bool)
    slot_of = np.full((p.nrows, p.ncols), -1, dtype=np.int64)
    for s, r, c in zip(*oracle.live_slots(p)):
        live[r, c] = True
        slot_of[r, c] = s
    cols, vals, perm, nnz = [], [], [], []
    for c in range(p.ncols):
        rows = [r for r in range(p.nrows) if live[r, c]]
        nnz.append(len(rows))
        cols.append(rows)
        vals.append([dense[r, c] for r in rows])
        perm.append([slot_of[r, c] for r in rows])
    WT = oracle.from_row_lists(p.ncols, p.nrows, cols, vals, pr)
    perm_arr = np.full(WT.total_capacity, -1, dtype=np.int64)
    for c in range(p.ncols):
        s = int(WT.row_start[c])
        perm_arr[s:s + nnz[c]] = perm[c]
    return WT, perm_arr


@pytest.mark.parametrize("M,K,sparsity,pr", [(3, 4, 0.5, 0.2), (8, 8, 0.0, 0.2), (8, 8, 0.9, 0.2),
                                             (16, 32, 0.8, 0.0), (32, 16, 0.8, 1.0), (1, 1, 0.0, 0.2),
                                             (1, 16, 0.5, 0.5), (16, 1, 0.5, 0.2),
                                             (64, 64, 0.99, 0.2)])
def test_transpose_oracle_vs_brute_force(M, K, sparsity, pr):
    p = oracle.bernoulli(M, K, sparsity, seed=M * 31 + K)
    WT, perm = oracle.transpose_with_perm(p, pr)
    WT_b, perm_b = _transpose_brute(p, pr)
    for name in ("values", "col_indices", "row_start", "row_nnz", "row_capacity"):
        assert_bits_equal(getattr(WT, name), getattr(WT_b, name), name)
    assert_bits_equal(perm, perm_b, "perm")
    assert_bits_equal(oracle.to_dense(WT), oracle.to_dense(p).T.copy(), "dense")
    assert oracle.check_invariants(WT.nrows, WT.ncols, WT.values, WT.col_indices, WT.row_start,
                                   WT.row_nnz, WT.row_capacity) == ""
    live = perm >= 0
    assert_bits_equal(WT.values[live], p.values[perm[live]], "perm gather")


def test_transpose_involution_and_empty():
    p = oracle.bernoulli(15, 20, 0.75, seed=2)
    WTT, _ = oracle.transpose_with_perm(oracle.transpose_with_perm(p)[0])
    assert_bits_equal(oracle.to_dense(WTT), oracle.to_dense(p), "involution")
    empty = oracle.Csr(5, 8, np.zeros(0, np.float32), np.zeros(0, np.int32),
                       np.zeros(5, np.int32), np.zeros(5, np.int32), np.zeros(5, np.int32))
    WT, perm = oracle.transpose_with_perm(empty)
    assert (WT.nrows, WT.ncols, WT.nnz) == (8, 5, 0)
    assert list(WT.row_capacity) == [1] * 8 and np.all(perm == -1)


# ─────────────────────── known answers (reference tests) ───────────────

def test_capacity_known_answer():
    # tests/test_padded_csr.py:61-79: capacities [3, 3, 2], starts [0, 3, 6] at pr 0.5
    W = np.array([[3, 0, 0, 1], [0, 0, 2, 5], [4, 0, 0, 0]], dtype=np.float32)
    p = oracle.from_dense(W, padding_ratio=0.5)
    assert list(p.row_capacity) == [3, 3, 2]
    assert list(p.row_nnz) == [2, 2, 1]
    assert list(p.row_start) == [0, 3, 6]
    assert list(oracle.row_capacity([0, 0, 5], 0.0)) == [1, 1, 5]
    with pytest.raises(ValueError, match="padding_ratio"):
        oracle.row_capacity([1], -0.1)


def test_single_entry_known_answers():
    # tests/test_spmm.py:149-166 (Y[2] = 2.5 * X[3]) and test_spmm_grad.py:221-233
    W = np.zeros((4, 6), np.float32)
    W[2, 3] = 2.5
    p = oracle.from_dense(W)
    X = np.random.default_rng(0).standard_normal((6, 3)).astype(np.float32)
    Y = oracle.spmm(p, X)
    assert np.all(Y[[0, 1, 3]] == 0.0)
    assert_bits_equal(Y[2], (np.float32(2.5) * X[3]).astype(np.float32), "2.5*X[3]")
    dY = np.random.default_rng(1).standard_normal((4, 3)).astype(np.float32)
    dW = oracle.sddmm(p, dY, X)
    slot = int(oracle.live_slots(p)[0][0])
    assert dW[slot] == pytest.approx(float((dY[2].astype(np.float64) * X[3]).sum()), rel=1e-5)
    # transpose single entry: WT[4, 2] of a 5x6 with W[2, 4] = 3.14 (test_padded_csr_transpose.py:126-139)
    W2 = np.zeros((5, 6), np.float32)
    W2[2, 4] = 3.14
    WT, _ = oracle.transpose_with_perm(oracle.from_dense(W2))
    assert oracle.to_dense(WT)[4, 2] == np.float32(3.14)


def test_rewrite_row_known_answer():
    # tests/test_padded_csr_rewrite.py:177-190: a rewritten value 7 times X 2 gives 14
    p = oracle.from_dense(np.eye(3, dtype=np.float32))
    q = oracle.rewrite_row(p, 1, [2], [7.0])
    X = np.full((3, 1), 2.0, np.float32)
    assert oracle.spmm(q, X)[1, 0] == 14.0


def test_c1_fixture_metadata_is_consistent():
    meta = json.loads((GOLDEN / "c1.json").read_text())
    assert set(meta["outputs_sha256"]) == {"Y", "dW", "dW_scalar", "dX"}
    for k, s in meta["samples"].items():
        assert len(s["index"]) == len(s["value_bits"]) == 64, k


def _round_to_f32(q):
    """The float32 nearest the rational q (ties to even), with gradual underflow
    and overflow to infinity — IEEE 754 round-to-nearest, from its definition."""
    from fractions import Fraction

    if q == 0:
        return np.float32(0.0)
    sign = -1.0 if q < 0 else 1.0
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()  # 2^e <= a < 2^(e+2)
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp_exp = max(e, -126) - 23  # 24-bit significand; below 2^-126 the spacing stays 2^-149
    m = a / Fraction(2) ** ulp_exp
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    val = float(n) * 2.0 ** ulp_exp  # exact in float64
    if val >= 2.0 ** 128:
        return np.float32(sign * np.inf)
    return np.float32(sign * val)


def test_oracle_fmaf_is_the_correctly_rounded_fma():
    """oracle.fmaf (libm) equals a·b + c rounded once, computed exactly; and it
    differs from the unfused multiply-add where that rounds twice."""
    from fractions import Fraction

    rng = np.random.default_rng(0)
    n = 3000
    a = np.ldexp(rng.standard_normal(n), rng.integers(-62, 62, n)).astype(np.float32)
    b = np.ldexp(rng.standard_normal(n), rng.integers(-62, 62, n)).astype(np.float32)
    p = (a * b).astype(np.float32)
    c = np.where(rng.random(n) < 0.5, -p, np.ldexp(rng.standard_normal(n), rng.integers(-140, 60, n)))
    c = c.astype(np.float32)
    got = oracle.fmaf(a, b, c)
    for i in range(n):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        want = _round_to_f32(exact)
        assert got[i].view(np.uint32) == want.view(np.uint32) or (got[i] == 0 and want == 0), i
    # known answer: (1 + 2^-12)^2 - (1 + 2^-11) = 2^-24 fused, 0 unfused
    x = np.float32(1 + 2.0 ** -12)
    y = np.float32(-(1 + 2.0 ** -11))
    assert oracle.fmaf(x, x, y) == np.float32(2.0 ** -24)
    assert np.float32(x * x) + y == 0.0
