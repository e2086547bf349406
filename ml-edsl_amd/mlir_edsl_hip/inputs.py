"""Seeded synthetic inputs for the dense-path workloads.

One generator feeds every consumer (tests, smoke check, benchmark, CPU
baseline) so the CPU and GPU paths see identical values: numpy's PCG64
(``numpy.random.default_rng(seed)``), drawing X, then W, then b.

Workloads (the reference never ran these sizes; its own benchmark draws
uniform[0,1) with seed 42, reference benchmarks/bench_matmul.py:97,109-111):
  c1  fp32 matmul 256^3, A and B ~ U[-1, 1), seed 0
  c2  fp32 dense 1024^3, X ~ N(0,1), W ~ N(0, 1/K), b ~ U[-0.1, 0.1), seed 1
  c3  fp32 dense 4096^3, same distributions, seed 2
  c4  fp32 dense M=16, K=N=8192 (W is 256 MiB), seed 3
  c5  integer dense 2048^3, X and W uniform ints in [-8, 7], b in [-512, 511], seed 4
  c3s8, c4s8  one GPU's share of c3 / c4 column-sharded over 8 GPUs (N / 8
      columns), seeds 5 and 6, c3's distributions
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

GENERATOR = "numpy.random.PCG64 via default_rng(seed); X, then W, then b"


@dataclass(frozen=True)
class Workload:
    name: str
    pattern: str        # backend pattern name
    dtype: str          # "f32" | "i32"
    M: int
    K: int
    N: int
    seed: int
    description: str

    @property
    def flops(self) -> int:
        """Algorithmic FLOP (or integer OP) count: 2*M*N*K (epilogue excluded)."""
        return 2 * self.M * self.N * self.K

    @property
    def compulsory_bytes(self) -> int:
        """Read X, W (and b) once, write Y once (4-byte elements)."""
        b = self.N if self.pattern != "matmul" else 0
        return 4 * (self.M * self.K + self.K * self.N + b + self.M * self.N)


WORKLOADS = {
    "c1": Workload("c1", "matmul", "f32", 256, 256, 256, 0,
                   "fp32 linalg.matmul 256^3, U[-1,1), seed 0"),
    "c2": Workload("c2", "dense_relu", "f32", 1024, 1024, 1024, 1,
                   "fp32 dense relu(X@W+b) 1024^3, seed 1"),
    "c3": Workload("c3", "dense_relu", "f32", 4096, 4096, 4096, 2,
                   "fp32 dense relu(X@W+b) 4096^3, seed 2"),
    "c4": Workload("c4", "dense_relu", "f32", 16, 8192, 8192, 3,
                   "fp32 dense relu(X@W+b) M=16 K=N=8192, seed 3"),
    "c5": Workload("c5", "dense_relu", "i32", 2048, 2048, 2048, 4,
                   "int dense relu(X@W+b) 2048^3, values in [-8,7], b in [-512,511], seed 4"),
    # One GPU's share of c3 and c4 when the layer is column-sharded 8 ways
    # (each GPU owns N/8 columns of W, b and Y; X is replicated).
    "c3s8": Workload("c3s8", "dense_relu", "f32", 4096, 4096, 512, 5,
                     "fp32 dense relu(X@W+b), c3's 8-way column shard: M=K=4096, N=512, seed 5"),
    "c4s8": Workload("c4s8", "dense_relu", "f32", 16, 8192, 1024, 6,
                     "fp32 dense relu(X@W+b), c4's 8-way column shard: M=16, K=8192, N=1024, seed 6"),
}


def uniform_f32(rng: np.random.Generator, shape, lo: float, hi: float) -> np.ndarray:
    """U[lo, hi) in float32 (24-bit uniform scaled; never returns hi)."""
    u = rng.random(shape, dtype=np.float32)
    return (u * np.float32(hi - lo) + np.float32(lo)).astype(np.float32)


def normal_f32(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def make_inputs(w: Workload, M: int | None = None, K: int | None = None, N: int | None = None,
                seed: int | None = None) -> list[np.ndarray]:
    """Inputs of workload `w` (shape and seed overridable for parity cases).
    Returns [A, B] for matmul, [X, W, b] otherwise."""
    M = w.M if M is None else M
    K = w.K if K is None else K
    N = w.N if N is None else N
    rng = np.random.default_rng(w.seed if seed is None else seed)
    if w.dtype == "i32":
        X = rng.integers(-8, 8, size=(M, K), dtype=np.int32)
        W = rng.integers(-8, 8, size=(K, N), dtype=np.int32)
        b = rng.integers(-512, 512, size=(N,), dtype=np.int32)
        return [X, W, b]
    if w.pattern == "matmul":
        A = uniform_f32(rng, (M, K), -1.0, 1.0)
        B = uniform_f32(rng, (K, N), -1.0, 1.0)
        return [A, B]
    X = normal_f32(rng, (M, K), 1.0)
    W = normal_f32(rng, (K, N), 1.0 / np.sqrt(K))
    b = uniform_f32(rng, (N,), -0.1, 0.1)
    return [X, W, b]
