"""Write the golden fixtures from the reference's own CPU kernels.

Run (only where the reference checkout exists, after `make -C oracle ref`):

    python tests/golden/make_golden.py

Inputs come from tests/golden/gen.py (bit-stable across numpy/torch versions).
Outputs come from oracle/_ref/libslref.so — the reference's csrc/kernels
compiled unchanged at its own flags — through oracle.RefCsr:

    Y      = spmm_simd(W, X)              csrc/kernels/spmm_avx2.cpp
    dW     = spmm_grad_w_simd(W, dY, X)   csrc/kernels/spmm_grad_avx2.cpp
    dW_sc  = spmm_grad_w(W, dY, X)        csrc/kernels/spmm_grad.cpp
    dX     = spmm_simd(WT, dY)            the reference backward's dX
                                          (WT = transpose_with_perm(W), whose
                                          layout is fixed uniquely by the
                                          PaddedCSR invariants)

Files
    kernels.npz   small cases, every input and output array in full
    c1.json       BASELINE config 1 (512x784, 78 live/row, N=256): SHA-256
                  digests of inputs and outputs plus sampled output values
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(HERE))

import gen  # noqa: E402
import oracle  # noqa: E402

SMALL_CASES = [
    # name, M, K, N, row_nnz rule, sigma, padding_ratio
    ("prime_7x13_n5", 7, 13, 5, "uniform4", 1.0, 0.2),
    ("n1", 32, 24, 1, "uniform5", 1.0, 0.2),
    ("n7", 16, 40, 7, "uniform6", 1.0, 0.0),
    ("n15", 16, 40, 15, "uniform6", 1.0, 0.5),
    ("n17", 16, 40, 17, "uniform6", 1.0, 1.0),
    ("n33", 20, 50, 33, "uniform9", 1.0, 0.2),
    ("n65_skew", 64, 64, 65, "skew", 0.5, 0.2),
    ("empty_rows", 10, 20, 9, "some_empty", 1.0, 0.2),
]


def row_rule(rule: str, M: int, K: int) -> np.ndarray:
    if rule.startswith("uniform"):
        return np.full(M, min(K, int(rule[len("uniform"):])), dtype=np.int32)
    if rule == "skew":  # one dense row, then a rank^-1.1 falloff down to 1
        r = np.arange(1, M + 1, dtype=np.float64)
        return np.maximum(1, np.minimum(K, np.floor(K * r ** -1.1))).astype(np.int32)
    if rule == "some_empty":
        n = np.array([0, 3, 0, 0, 5, 1, 0, 20, 2, 0], dtype=np.int32)
        return n[:M]
    raise ValueError(rule)


def reference_outputs(p: oracle.Csr, X: np.ndarray, dY: np.ndarray):
    ref = oracle.RefCsr(p)
    assert ref.check_invariants() == "", ref.check_invariants()
    WT, _ = oracle.transpose_with_perm(p)
    ref_t = oracle.RefCsr(WT)
    assert ref_t.check_invariants() == ""
    return {
        "Y": ref.spmm(X, "simd"),
        "dW": ref.sddmm(dY, X, "simd"),
        "dW_scalar": ref.sddmm(dY, X, "scalar"),
        "dX": ref_t.spmm(dY, "simd"),
    }


def main() -> None:
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libslref.so is missing: run `make -C oracle ref` first")
    arrays = {}
    for seed, (name, M, K, N, rule, sigma, pr) in enumerate(SMALL_CASES, start=1):
        parts = gen.padded_csr(M, K, row_rule(rule, M, K), seed, sigma, pr)
        p = oracle.Csr(M, K, *parts)
        X = gen.normalish(1000 + seed, K * N).reshape(K, N)
        dY = gen.normalish(2000 + seed, M * N).reshape(M, N)
        out = reference_outputs(p, X, dY)
        for key, val in zip(("values", "col_indices", "row_start", "row_nnz", "row_capacity"),
                            parts):
            arrays[f"{name}/{key}"] = val
        arrays[f"{name}/shape"] = np.array([M, K, N], dtype=np.int64)
        arrays[f"{name}/X"] = X
        arrays[f"{name}/dY"] = dY
        for key, val in out.items():
            arrays[f"{name}/{key}"] = val
    np.savez_compressed(HERE / "kernels.npz", **arrays)

    # W 512x784, 78 live columns per row, sigma 0.02, pr 0.2.
    M, K, N = 512, 784, 256
    parts = gen.padded_csr(M, K, np.full(M, 78, np.int32), 101, 0.02, 0.2)
    p = oracle.Csr(M, K, *parts)
    X = gen.normalish(102, K * N).reshape(K, N)
    dY = gen.normalish(103, M * N).reshape(M, N)
    out = reference_outputs(p, X, dY)
    pick = gen.words(104, 64)
    meta = {
        "config": "BASELINE configs[0]: 512x784 @ 78 live/row, sigma 0.02, pr 0.2, N=256",
        "gen": {"csr_seed": 101, "X_seed": 102, "dY_seed": 103, "sigma": 0.02,
                "padding_ratio": 0.2, "M": M, "K": K, "N": N, "nnz_per_row": 78},
        "inputs_sha256": {
            "values": gen.digest(p.values), "col_indices": gen.digest(p.col_indices),
            "X": gen.digest(X), "dY": gen.digest(dY),
        },
        "outputs_sha256": {k: gen.digest(v) for k, v in out.items()},
        "samples": {},
    }
    for k, v in out.items():
        flat = v.reshape(-1)
        idx = (pick % np.uint64(flat.shape[0])).astype(np.int64)
        meta["samples"][k] = {"index": idx.tolist(),
                              "value_bits": flat[idx].view(np.uint32).tolist()}
    (HERE / "c1.json").write_text(json.dumps(meta, indent=1) + "\n")
    print("wrote", HERE / "kernels.npz", "and", HERE / "c1.json")


if __name__ == "__main__":
    main()
