"""Pins the oracle's restatement of the SET / RigL topology update and of the
dense gradient before the GPU path is checked against it.

Checks that do not share code with the oracle: the reference tests' literal
known answers (RigL grows column 15; small hand-worked drop sets), the
reference's own selection expression for RigL (np.argpartition, compared as
a set where |G| has no ties at the cut), a full sort for the threshold, the
published first outputs of splitmix64, structural invariants, and a
chi-square test of SET's grow distribution.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import assert_bits_equal


def _live(p, i):
    s, n = int(p.row_start[i]), int(p.row_nnz[i])
    return p.col_indices[s:s + n].copy(), p.values[s:s + n].copy()


def _check(p):
    msg = oracle.check_invariants(p.nrows, p.ncols, p.values, p.col_indices, p.row_start,
                                  p.row_nnz, p.row_capacity)
    assert msg == "", msg


# ───────────────────────────── threshold ───────────────────────────────

@pytest.mark.parametrize("seed", range(4))
def test_live_abs_kth_is_the_kth_of_a_full_sort(seed):
    p = oracle.uniform_rows(40, 60, 9, seed=seed, sigma=1.0)
    rng = np.random.default_rng(seed)
    # many duplicate magnitudes, signed zeros
    p.values[p.col_indices >= 0] = (rng.integers(-5, 6, size=p.nnz) * 0.25).astype(np.float32)
    live = np.sort(np.abs(np.concatenate([_live(p, i)[1] for i in range(p.nrows)])))
    for k in (1, 2, p.nnz // 3, p.nnz - 1, p.nnz):
        assert oracle.live_abs_kth(p, k) == live[k - 1]


# ───────────────────────────── generator ───────────────────────────────

def test_splitmix_keys_match_published_outputs():
    # splitmix64 seeded with 0: first outputs 0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4
    k = oracle.splitmix_keys(0, 0, 10, np.array([0, 1], np.int64))
    assert k.tolist() == [0xE220A839, 0x6E789E6A]
    # output number row*ncols + c + 1: row 1, col 0 of a 1-column matrix is the second
    assert oracle.splitmix_keys(0, 1, 1, np.array([0], np.int64)).tolist() == [0x6E789E6A]


# ───────────────────────────── known answers ───────────────────────────

def test_rigl_grows_at_the_highest_gradient_column():
    """test_rigl.py:127-183: one row, live cols [0, 1] = [0.01, 0.02],
    drop_fraction 0.5, G[0, k] = X[k] with X[15] = 100, X[12] = 50."""
    p = oracle.from_row_lists(1, 20, [np.array([0, 1], np.int32)],
                              [np.array([0.01, 0.02], np.float32)], padding_ratio=0.2)
    G = np.zeros((1, 20), np.float32)
    G[0, 15], G[0, 12] = 100.0, 50.0
    k_drop = max(1, int(0.5 * p.nnz))
    q = oracle.drop_grow(p, k_drop, "gradient", G)
    cols, vals = _live(q, 0)
    assert cols.tolist() == [1, 15]
    assert vals.tolist() == [np.float32(0.02), 0.0]


def test_drop_set_hand_worked():
    # |v| = .5 .1 .3 | .2 .05 | .4 ; k = int(0.5*6) = 3 -> threshold .2
    p = oracle.from_row_lists(3, 8, [np.array([0, 2, 5], np.int32), np.array([1, 6], np.int32),
                                     np.array([3], np.int32)],
                              [np.array([.5, -.1, .3], np.float32),
                               np.array([.2, -.05], np.float32), np.array([.4], np.float32)])
    q = oracle.drop_grow(p, 3, "random", seed=7)
    # row 0 keeps cols 0 and 5, regrows one; row 1 keeps nothing above .2, so
    # its largest (col 1, .2) survives and one column is regrown; row 2 intact.
    c0, v0 = _live(q, 0)
    assert {0, 5} <= set(c0.tolist()) and len(c0) == 3
    assert v0[c0 == 0][0] == np.float32(.5) and v0[c0 == 5][0] == np.float32(.3)
    c1, v1 = _live(q, 1)
    assert 1 in c1.tolist() and len(c1) == 2 and v1[c1 == 1][0] == np.float32(.2)
    c2, v2 = _live(q, 2)
    assert c2.tolist() == [3] and v2.tolist() == [np.float32(.4)]
    _check(q)


# ───────────────────────── against the reference rule ──────────────────

def _reference_rigl_row(cols, vals, thr, g_row, ncols):
    """The reference's per-row RigL choice, restated from router.py:676-732:
    survivors by the strict threshold (first argmax if none), then
    np.argpartition(-|G| with survivors at -inf) for the grows."""
    keep = np.abs(vals) > thr
    if not keep.any():
        keep[int(np.argmax(np.abs(vals)))] = True
    kc = cols[keep]
    n_drop = len(cols) - int(keep.sum())
    a = np.abs(g_row).astype(np.float32)
    a[kc] = -np.inf
    n_grow = min(n_drop, int((a > -np.inf).sum()))
    grow = np.argpartition(-a, n_grow - 1)[:n_grow] if n_grow else np.zeros(0, np.int64)
    return set(kc.tolist()), set(grow.tolist())


@pytest.mark.parametrize("seed,df,nan_frac", [(0, 0.3, 0.0), (1, 0.5, 0.0), (2, 0.99, 0.0),
                                               (3, 0.05, 0.0), (4, 0.5, 0.3), (5, 0.99, 0.9)])
def test_rigl_matches_reference_selection(seed, df, nan_frac):
    """The oracle's RigL rows against the reference's own selection expression,
    including G with NaN entries: the reference never grows a NaN column
    (available = empties with |G| > -inf) and its row then shrinks."""
    p = oracle.uniform_rows(30, 50, 12, seed=seed, sigma=1.0)
    rng = np.random.default_rng(seed)
    G = rng.standard_normal((30, 50)).astype(np.float32)  # no ties (continuous)
    G[rng.random((30, 50)) < nan_frac] = np.nan
    k_drop = max(1, int(df * p.nnz))
    thr = oracle.live_abs_kth(p, k_drop)
    q = oracle.drop_grow(p, k_drop, "gradient", G)
    shrunk = 0
    for i in range(p.nrows):
        cols, vals = _live(p, i)
        kept, grown = _reference_rigl_row(cols, vals, thr, G[i], p.ncols)
        new_cols, new_vals = _live(q, i)
        assert set(new_cols.tolist()) == kept | grown, i
        assert len(new_cols) == len(kept) + len(grown)
        shrunk += len(cols) - len(new_cols)
        for c, v in zip(new_cols, new_vals):
            if c in kept:
                assert v == vals[cols == c][0]
            else:
                assert v == 0.0
    _check(q)
    assert q.nnz == p.nnz - shrunk
    if nan_frac == 0.0:
        assert shrunk == 0 and np.array_equal(q.row_nnz, p.row_nnz)
    if nan_frac == 0.9:
        assert shrunk > 0  # the case is exercised


@pytest.mark.parametrize("df", [0.3, 0.99])
def test_set_structure(df):
    p = oracle.zipf_rows(64, 40, 0.2, 1.1, seed=4, sigma=1.0)
    q = oracle.drop_grow(p, max(1, int(df * p.nnz)), "random", seed=123)
    thr = oracle.live_abs_kth(p, max(1, int(df * p.nnz)))
    _check(q)
    assert np.array_equal(q.row_nnz, p.row_nnz)
    for i in range(p.nrows):
        cols, vals = _live(p, i)
        if len(cols) == 0:
            continue
        keep = np.abs(vals) > thr
        if not keep.any():
            keep[int(np.argmax(np.abs(vals)))] = True
        new_cols, new_vals = _live(q, i)
        old = dict(zip(cols[keep].tolist(), vals[keep].tolist()))
        for c, v in zip(new_cols.tolist(), new_vals.tolist()):
            assert v == (old[c] if c in old else 0.0)
        assert set(old) <= set(new_cols.tolist())
    # deterministic under the seed, different under another seed
    assert np.array_equal(oracle.drop_grow(p, 5, "random", seed=123).col_indices,
                          oracle.drop_grow(p, 5, "random", seed=123).col_indices)


def test_set_grow_is_uniform_over_empty_columns():
    """One row, 10 columns, live {0, 1}, col 0 dropped: the grown column must
    be uniform over the 9 columns outside {1} (a dropped column may regrow)."""
    p = oracle.from_row_lists(1, 10, [np.array([0, 1], np.int32)],
                              [np.array([0.1, 0.9], np.float32)])
    counts = np.zeros(10, np.int64)
    trials = 4500
    for s in range(trials):
        q = oracle.drop_grow(p, 1, "random", seed=s * 7919 + 1)
        cols, _ = _live(q, 0)
        assert 1 in cols.tolist()
        counts[[c for c in cols.tolist() if c != 1]] += 1
    assert counts[1] == 0 and counts.sum() == trials
    expected = trials / 9
    chi2 = float((((counts[[0, 2, 3, 4, 5, 6, 7, 8, 9]] - expected) ** 2) / expected).sum())
    assert chi2 < 33.7  # chi-square, 8 degrees of freedom, p = 1e-4


def test_rigl_ties_go_to_lower_columns_and_nan_is_never_grown():
    p = oracle.from_row_lists(1, 8, [np.array([0, 1, 2], np.int32)],
                              [np.array([0.01, 0.02, 0.9], np.float32)])
    G = np.array([[5, 5, 0, 3, 3, np.nan, 3, 3]], np.float32)
    q = oracle.drop_grow(p, 2, "gradient", G)  # drops cols 0 and 1
    cols, vals = _live(q, 0)
    # candidates are all but col 2: |G| 5 at cols 0, 1 win
    assert cols.tolist() == [0, 1, 2] and vals.tolist() == [0.0, 0.0, np.float32(0.9)]
    G2 = np.array([[0, 0, 0, 3, 3, np.nan, 3, 3]], np.float32)
    q2 = oracle.drop_grow(p, 2, "gradient", G2)
    assert _live(q2, 0)[0].tolist() == [2, 3, 4]
    # a zero |G| is preferred to a NaN at a lower column
    G3 = np.array([[np.nan, np.nan, 7, np.nan, np.nan, 0, np.nan, np.nan]], np.float32)
    q3 = oracle.drop_grow(p, 2, "gradient", G3)
    assert _live(q3, 0)[0].tolist() == [2, 5]  # one growable column: the row shrinks
    assert q3.row_nnz.tolist() == [2] and set(q3.col_indices.tolist()[2:]) == {-1}
    _check(q3)


def test_dense_row_regrows_its_dropped_columns():
    W = np.array([[0.1, -0.2, 0.3, -0.4]], np.float32)
    p = oracle.from_dense(W)
    q = oracle.drop_grow(p, 2, "random", seed=1)
    cols, vals = _live(q, 0)
    assert cols.tolist() == [0, 1, 2, 3]
    assert_bits_equal(vals, np.array([0, 0, 0.3, -0.4], np.float32), "vals")
