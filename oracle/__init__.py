"""ctypes binding of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY. The oracle restates the reference's CPU-JIT
lowering of the dense path (file:line citations in oracle.h). Only the test
suite, ``__graft_entry__.smoke()`` (as the checker) and the ``cpu_baseline``
leg of ``bench.py`` may import this package; the product path never does.

Parity pinning of each function is documented in the test modules that check
it (tests/test_oracle_*.py): reference known answers, exact rational
brute force of the fma / mulf+addf chains, fp64 error bounds, exact integer
arithmetic, IEEE special values, and planted-mistake checks.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

EPI_NONE, EPI_BIAS, EPI_RELU, EPI_BIAS_RELU, EPI_LEAKY, EPI_BIAS_LEAKY = range(6)

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
                                       ctypes.c_float, ctypes.c_int]
        L.oracle_dense_f32.restype = ctypes.c_int
        L.oracle_dense_i32.argtypes = [i32p, i32p, i32p, i32p, i64, i64, i64, ctypes.c_int,
                                       ctypes.c_int]
        L.oracle_dense_i32.restype = ctypes.c_int
        L.oracle_dense_f32_vec.argtypes = L.oracle_dense_f32.argtypes
        L.oracle_dense_f32_vec.restype = ctypes.c_int
        L.oracle_static_tiles.argtypes = [i64, i64, i64]
        L.oracle_static_tiles.restype = ctypes.c_int
        L.oracle_set_mutation.argtypes = [ctypes.c_int]
        L.oracle_set_mutation.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def epilogue_code(bias: bool, act: str) -> int:
    return (1 if bias else 0) | ({"none": 0, "relu": 1, "leaky": 2}[act] << 1)


def dense_f32(X, W, b=None, act: str = "none", alpha: float = 0.0, threads: int = 0) -> np.ndarray:
    """Y = act(X @ W (+ b)) with the reference CPU-JIT arithmetic (fp32)."""
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
                                epilogue_code(bias, act), alpha, threads)
    if rc != 0:
        raise ValueError(f"oracle_dense_f32 rejected epilogue {act!r}")
    return Y


def dense_f32_vec(X, W, b=None, act: str = "none", alpha: float = 0.0, threads: int = 0) -> np.ndarray:
    """dense_f32 with the reference JIT's 8-wide vector FMAs (bit-identical;
    static-tile shapes only). For timing the CPU baseline."""
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
                         f"needs static 8x8x8 tiles")
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


def matmul_f32(A, B, threads: int = 0) -> np.ndarray:
    return dense_f32(A, B, None, "none", threads=threads)


def matmul_i32(A, B, threads: int = 0) -> np.ndarray:
    return dense_i32(A, B, None, "none", threads=threads)


def static_tiles(M: int, N: int, K: int) -> bool:
    return bool(lib().oracle_static_tiles(M, N, K))


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
