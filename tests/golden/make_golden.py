"""Writes tests/golden/dense_golden.npz + dense_golden.json.

Golden vectors for the dense path: seeded small inputs and the outputs
computed by exact rational arithmetic (tests/exact.py) -- neither the C
oracle nor the HIP kernels are involved, so these pin both.

Each f32 case holds the reference CPU-JIT result on both rounding chains it
can take: the ascending-k fma chain (static 8x8x8 tiles) under key
`Y_<epilogue>_fma` and the mulf+addf chain (dynamic tiles) under
`Y_<epilogue>_muladd`. i32 cases include values far outside int8 so that
products and sums wrap modulo 2^32.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import exact  # noqa: E402

F32_CASES = [
    # name, M, K, N, seed
    ("f32_8x8x8", 8, 8, 8, 11),
    ("f32_16x16x16", 16, 16, 16, 12),
    ("f32_2x4x3", 2, 4, 3, 13),
    ("f32_24x16x40", 24, 16, 40, 14),
    ("f32_5x9x7", 5, 9, 7, 15),
    ("f32_32x32x32", 32, 32, 32, 16),
    ("f32_1x64x64", 1, 64, 64, 17),
    ("f32_16x128x64", 16, 128, 64, 18),
]
I32_CASES = [
    # name, M, K, N, seed, value range
    ("i32_small_8x8x8", 8, 8, 8, 21, 8),
    ("i32_int8_16x32x24", 16, 32, 24, 22, 128),
    ("i32_wrap_9x13x11", 9, 13, 11, 23, 2**31 - 1),
    ("i32_big_12x20x16", 12, 20, 16, 24, 2**20),
]
ACTS = [("none", False), ("bias", True), ("relu", True), ("leaky", True), ("relu_nobias", False),
        ("if_relu", True), ("if_relu_nobias", False)]
F32_ACT = {"none": "none", "bias": "none", "relu": "relu", "leaky": "leaky", "relu_nobias": "relu",
           "if_relu": "if_relu", "if_relu_nobias": "if_relu"}
ALPHA = 0.01


def main():
    arrays = {}
    index = []
    for name, M, K, N, seed in F32_CASES:
        rng = np.random.default_rng(seed)
        X = rng.standard_normal((M, K), dtype=np.float32)
        W = (rng.standard_normal((K, N), dtype=np.float32) / np.float32(np.sqrt(K))).astype(np.float32)
        b = (rng.random(N, dtype=np.float32) * np.float32(0.2) - np.float32(0.1)).astype(np.float32)
        arrays[f"{name}/X"], arrays[f"{name}/W"], arrays[f"{name}/b"] = X, W, b
        for tag, use_b in ACTS:
            for chain, fma in (("fma", True), ("muladd", False)):
                arrays[f"{name}/Y_{tag}_{chain}"] = exact.dense_f32_exact(
                    X, W, b if use_b else None, F32_ACT[tag], ALPHA, fma)
        index.append({"name": name, "dtype": "f32", "M": M, "K": K, "N": N, "seed": seed,
                      "chains": ["fma", "muladd"], "alpha": ALPHA, "epilogues": [t for t, _ in ACTS]})
        print(name, flush=True)
    for name, M, K, N, seed, vr in I32_CASES:
        rng = np.random.default_rng(seed)
        lo, hi = (-vr, vr) if vr < 2**31 - 1 else (-(2**31), 2**31 - 1)
        X = rng.integers(lo, hi, size=(M, K), dtype=np.int64, endpoint=True).astype(np.int32)
        W = rng.integers(lo, hi, size=(K, N), dtype=np.int64, endpoint=True).astype(np.int32)
        b = rng.integers(lo, hi, size=(N,), dtype=np.int64, endpoint=True).astype(np.int32)
        arrays[f"{name}/X"], arrays[f"{name}/W"], arrays[f"{name}/b"] = X, W, b
        tags = []
        for tag, use_b in ACTS:
            if tag == "leaky" or tag.startswith("if_relu"):
                continue
            act = "relu" if tag.startswith("relu") else "none"
            arrays[f"{name}/Y_{tag}"] = exact.dense_i32_exact(X, W, b if use_b else None, act)
            tags.append(tag)
        index.append({"name": name, "dtype": "i32", "M": M, "K": K, "N": N, "seed": seed,
                      "value_range": vr, "epilogues": tags})
        print(name, flush=True)
    np.savez_compressed(os.path.join(HERE, "dense_golden.npz"), **arrays)
    with open(os.path.join(HERE, "dense_golden.json"), "w") as f:
        json.dump({"generator": "tests/golden/make_golden.py (exact rational arithmetic)",
                   "cases": index}, f, indent=1)


if __name__ == "__main__":
    main()
