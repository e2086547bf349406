"""ctypes binding of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY. The oracle restates the reference's CPU-JIT
lowering of the dense path (file:line citations in oracle.h). Only the test
suite, ``__graft_entry__.smoke()`` (as the checker) and the ``cpu_baseline``
leg of ``bench.py`` may import this package; the product path never does.

Every function is pinned in tests/test_oracle.py: reference known answers,
exact rational brute force of both f32 rounding chains (fma and mulf+addf),
fp64 error bounds, exact integer arithmetic, IEEE special values, and
planted-mistake checks.

f32 rounding chains. The reference sums each output element in ascending k
from +0.0, either as a vector.fma chain (static 8x8x8 tiles) or as mulf then
addf (dynamic tiles). Which one it takes for a shape is decided inside MLIR,
so ``dense_f32`` takes the chain explicitly and ``dense_f32_chains`` returns
both; the parity tests hold a result to the bar against both, element by
element.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import subprocess
from typing import NamedTuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

EPI_NONE, EPI_BIAS, EPI_RELU, EPI_BIAS_RELU, EPI_LEAKY, EPI_BIAS_LEAKY, EPI_IF_RELU, EPI_BIAS_IF_RELU = range(8)
CHAIN_FMA, CHAIN_MULADD = 0, 1
_CHAINS = {"fma": CHAIN_FMA, "muladd": CHAIN_MULADD}
# Activations: "relu" is arith.maximumf(v, 0) (NaN propagates); "if_relu" is
# the tensor_map body If(v > 0.0, v, 0.0) (cmpf ogt: NaN -> +0, -0 -> +0).
ACTS = {"none": 0, "relu": 1, "leaky": 2, "if_relu": 3}


class F32Chains(NamedTuple):
    """One f32 result on each rounding chain the reference can take."""
    fma: np.ndarray
    muladd: np.ndarray


_lib = None


def build() -> str:
    """Compile liboracle.so with oracle/Makefile (always rebuilds)."""
    subprocess.run(["make", "-B", "-s", "-f", os.path.join(HERE, "Makefile")], check=True,
                   cwd=HERE)
    global _lib
    _lib = None
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        f32p = ctypes.POINTER(ctypes.c_float)
        i32p = ctypes.POINTER(ctypes.c_int32)
        i64 = ctypes.c_int64
        L.oracle_dense_f32.argtypes = [f32p, f32p, f32p, f32p, i64, i64, i64, ctypes.c_int,
                                       ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.oracle_dense_f32.restype = ctypes.c_int
        L.oracle_dense_i32.argtypes = [i32p, i32p, i32p, i32p, i64, i64, i64, ctypes.c_int,
                                       ctypes.c_int]
        L.oracle_dense_i32.restype = ctypes.c_int
        L.oracle_dense_f32_vec.argtypes = [f32p, f32p, f32p, f32p, i64, i64, i64, ctypes.c_int,
                                           ctypes.c_float, ctypes.c_int]
        L.oracle_dense_f32_vec.restype = ctypes.c_int
        L.oracle_set_mutation.argtypes = [ctypes.c_int]
        L.oracle_set_mutation.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def epilogue_code(bias: bool, act: str) -> int:
    return (1 if bias else 0) | (ACTS[act] << 1)


def dense_f32(X, W, b=None, act: str = "none", alpha: float = 0.0, *, chain: str,
              threads: int = 0) -> np.ndarray:
    """Y = act(X @ W (+ b)) with the reference CPU-JIT arithmetic (fp32), the
    sums on the given rounding chain ("fma" or "muladd")."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    M, K = X.shape
    K2, N = W.shape
    assert K == K2, (X.shape, W.shape)
    bias = b is not None
    bb = np.ascontiguousarray(b if bias else np.zeros(max(N, 1)), dtype=np.float32)
    Y = np.empty((M, N), dtype=np.float32)
    rc = lib().oracle_dense_f32(_ptr(X, ctypes.c_float), _ptr(W, ctypes.c_float),
                                _ptr(bb, ctypes.c_float), _ptr(Y, ctypes.c_float), M, N, K,
                                epilogue_code(bias, act), alpha, _CHAINS[chain], threads)
    if rc != 0:
        raise ValueError(f"oracle_dense_f32 rejected epilogue {act!r} / chain {chain!r}")
    return Y


def dense_f32_chains(X, W, b=None, act: str = "none", alpha: float = 0.0,
                     threads: int = 0) -> F32Chains:
    """dense_f32 on both rounding chains."""
    return F32Chains(dense_f32(X, W, b, act, alpha, chain="fma", threads=threads),
                     dense_f32(X, W, b, act, alpha, chain="muladd", threads=threads))


def dense_f32_vec(X, W, b=None, act: str = "none", alpha: float = 0.0, threads: int = 0) -> np.ndarray:
    """dense_f32 on the fma chain with the reference JIT's 8-wide vector FMAs
    (bit-identical; M, N, K multiples of 8 only). For timing the CPU baseline."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    M, K = X.shape
    K2, N = W.shape
    assert K == K2, (X.shape, W.shape)
    bias = b is not None
    bb = np.ascontiguousarray(b if bias else np.zeros(max(N, 1)), dtype=np.float32)
    Y = np.empty((M, N), dtype=np.float32)
    rc = lib().oracle_dense_f32_vec(_ptr(X, ctypes.c_float), _ptr(W, ctypes.c_float),
                                    _ptr(bb, ctypes.c_float), _ptr(Y, ctypes.c_float), M, N, K,
                                    epilogue_code(bias, act), alpha, threads)
    if rc != 0:
        raise ValueError(f"oracle_dense_f32_vec rejected the call (code {rc}): shape {M}x{K}x{N} "
                         f"needs whole 8x8x8 tiles")
    return Y


def dense_i32(X, W, b=None, act: str = "none", threads: int = 0) -> np.ndarray:
    """Y = act(X @ W (+ b)) in wrapping i32 arithmetic."""
    X = np.ascontiguousarray(X, dtype=np.int32)
    W = np.ascontiguousarray(W, dtype=np.int32)
    M, K = X.shape
    K2, N = W.shape
    assert K == K2, (X.shape, W.shape)
    bias = b is not None
    bb = np.ascontiguousarray(b if bias else np.zeros(max(N, 1)), dtype=np.int32)
    Y = np.empty((M, N), dtype=np.int32)
    rc = lib().oracle_dense_i32(_ptr(X, ctypes.c_int32), _ptr(W, ctypes.c_int32),
                                _ptr(bb, ctypes.c_int32), _ptr(Y, ctypes.c_int32), M, N, K,
                                epilogue_code(bias, act), threads)
    if rc != 0:
        raise ValueError(f"oracle_dense_i32 rejected epilogue {act!r}")
    return Y


@contextlib.contextmanager
def mutation(m: int):
    """Plant mistake `m` (see oracle.c) for the duration of the block."""
    lib().oracle_set_mutation(m)
    try:
        yield
    finally:
        lib().oracle_set_mutation(0)


def cpu_threads() -> int:
    """Threads the OpenMP runtime will use (OMP_NUM_THREADS or all cores)."""
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.split(",")[0].strip().isdigit():
        return int(env.split(",")[0])
    return os.cpu_count() or 1
