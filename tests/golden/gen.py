"""Library-independent deterministic inputs for the golden fixtures.

numpy's and torch's random streams are not promised to stay the same across
versions, so the fixtures here are generated from splitmix64 evaluated in
exact uint64 arithmetic and mapped to float32 with exact (power-of-two)
scalings or float64 sums rounded once. The same seed gives the same bits on
every machine; fixtures additionally record SHA-256 digests of the inputs so
a drift would be caught, not silently compared.
"""

from __future__ import annotations

import hashlib

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x.astype(np.uint64) + _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def words(seed: int, n: int) -> np.ndarray:
    base = np.uint64(seed) << np.uint64(40)
    return splitmix64(np.arange(n, dtype=np.uint64) + base)


def uniform(seed: int, n: int) -> np.ndarray:
    """float32 in [-1, 1) on a 2^-23 grid (exact)."""
    u = (words(seed, n) >> np.uint64(40)).astype(np.float64)  # 24-bit integer
    return (u * (2.0 ** -23) - 1.0).astype(np.float32)


def normalish(seed: int, n: int, sigma: float = 1.0) -> np.ndarray:
    """Irwin-Hall(4) with unit variance, times sigma, rounded once to float32."""
    s = np.zeros(n, dtype=np.float64)
    for k in range(4):
        s += uniform(seed * 4 + k + 1, n).astype(np.float64)
    return (s * (np.sqrt(3.0 / 4.0) * sigma)).astype(np.float32)


def pick_columns(seed: int, K: int, n: int) -> np.ndarray:
    """n distinct columns of [0, K), ascending."""
    keys = words(seed, K)
    return np.sort(np.argsort(keys, kind="stable")[:n]).astype(np.int32)


def padded_csr(M: int, K: int, row_nnz, seed: int, sigma: float, padding_ratio: float = 0.2):
    """Host arrays (values, col, row_start, row_nnz, row_capacity) of a padded CSR."""
    row_nnz = np.asarray(row_nnz, dtype=np.int32)
    cap = np.maximum(1, np.ceil(row_nnz.astype(np.float64) * (1.0 + padding_ratio))).astype(
        np.int32)
    start = np.zeros(M, dtype=np.int64)
    if M > 1:
        start[1:] = np.cumsum(cap[:-1].astype(np.int64))
    total = int(cap.astype(np.int64).sum())
    values = np.zeros(total, dtype=np.float32)
    col = np.full(total, -1, dtype=np.int32)
    vals = normalish(seed, int(row_nnz.astype(np.int64).sum()), sigma)
    off = 0
    for i in range(M):
        n = int(row_nnz[i])
        col[start[i]:start[i] + n] = pick_columns(seed * 1_000_003 + i + 1, K, n)
        values[start[i]:start[i] + n] = vals[off:off + n]
        off += n
    return values, col, start.astype(np.int32), row_nnz, cap


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
