"""Host-buffer entry points on operands large enough for the pinned staging
ring (2 MiB and up): several chunks wrapping the 4-slot ring in both
directions, padded device rows (column counts not a multiple of 4), and host
operands that are strided views with an element offset, passed straight
through the memref ABI (the reference's JIT calling convention). The large
f32 cases take the pipelined path (row blocks uploaded, computed and
downloaded on three streams), the i32 and small ones the plain sequence.
Results are checked against the oracle: i32 bit-exact, f32 to the usual
bar."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from conftest import assert_f32_parity
from mlir_edsl_hip import _native

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    import torch
    assert torch.cuda.is_available()
    return _native.lib()


def _slice(buf, rows, cols, pad, off):
    """rows x cols view with row pitch cols + pad, starting `off` elements in."""
    return buf[off:off + rows * (cols + pad)].reshape(rows, cols + pad)[:, :cols]


def _view(rng, rows, cols, pad, off, dtype):
    """(buffer, view) with the view filled with random values."""
    buf = np.zeros(rows * (cols + pad) + off + 3, dtype=dtype)
    v = _slice(buf, rows, cols, pad, off)
    if dtype == np.float32:
        v[...] = rng.standard_normal((rows, cols), dtype=np.float32)
    else:
        v[...] = rng.integers(-128, 128, size=(rows, cols), dtype=np.int32)
    return buf, v


def _desc2(buf, v):
    p = buf.ctypes.data
    off = (v.__array_interface__["data"][0] - p) // v.itemsize
    return [p, p, off, v.shape[0], v.shape[1], v.strides[0] // v.itemsize, 1]


def _call_dense_relu(lib, dtype, Xb, X, Wb, W, b, Yb, Y):
    sym = "edsl_hip_dense_relu_f32" if dtype == np.float32 else "edsl_hip_dense_relu_i32"
    args = _desc2(Xb, X) + _desc2(Wb, W) + [b.ctypes.data, b.ctypes.data, 0, b.shape[0], 1] + _desc2(Yb, Y)
    fn = ctypes.CFUNCTYPE(None, *([ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 5) * 2 +
                          [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64] +
                          [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 5)(
        ctypes.cast(getattr(lib, sym), ctypes.c_void_p).value)
    lib.edsl_hip_clear_error()
    fn(*args)
    _native.raise_on_error(sym)


# (M, K, N, pads and offsets of X / W / Y): X, W, Y sizes chosen so the
# staged copies take 1 to 6 chunks of 8 MiB.
CASES = [
    # f32, padded device rows (K, N not multiples of 4), strided + offset host views
    ("f32", 4500, 1030, 1001, (7, 3), (0, 0), (9, 5)),
    # f32 contiguous, X and Y staged in 2 chunks each
    ("f32", 4096, 1024, 1024, (0, 0), (0, 0), (0, 0)),
    # i32: X of 40 MiB, 5 chunks (the ring wraps on the way in)
    ("i32", 5120, 2048, 64, (0, 0), (0, 0), (0, 0)),
    # i32: Y of 40 MiB + padding, 6 chunks (the ring wraps on the way out), strided Y
    ("i32", 5120, 16, 2050, (0, 0), (4, 1), (6, 2)),
    # small: below the staging threshold, strided (the direct copies)
    ("f32", 64, 33, 17, (3, 1), (5, 2), (2, 1)),
]


@pytest.mark.parametrize("dt, M, K, N, xpo, wpo, ypo", CASES)
def test_host_staging(dt, M, K, N, xpo, wpo, ypo, lib):
    dtype = np.float32 if dt == "f32" else np.int32
    rng = np.random.default_rng(M + K + N)
    Xb, X = _view(rng, M, K, *xpo, dtype)
    Wb, W = _view(rng, K, N, *wpo, dtype)
    b = (rng.standard_normal(N, dtype=np.float32) if dt == "f32"
         else rng.integers(-2**20, 2**20, size=N, dtype=np.int32))
    Yb, Y = _view(rng, M, N, *ypo, dtype)
    Y[...] = -3 if dt == "i32" else np.nan  # every element must be written
    outside = np.ones(Yb.shape, dtype=bool)
    _slice(outside, M, N, *ypo)[...] = False
    Yb_before = Yb.copy()
    _call_dense_relu(lib, dtype, Xb, X, Wb, W, b, Yb, Y)
    plan = _native.last_plan()
    what = f"{dt} M={M} K={K} N={N} X pad/off={xpo} W={wpo} Y={ypo} [{plan}]"
    # f32 layers with M >= 1024 rows and >= 16 MiB of X and Y overlap their
    # copies with the kernels (row blocks on three streams)
    pipelined = dt == "f32" and M >= 1024 and M * (K + N) * 4 >= 16 << 20
    assert plan.startswith("host pipeline") == pipelined, what
    if dt == "i32":
        ref = oracle.dense_i32(np.ascontiguousarray(X), np.ascontiguousarray(W), b, "relu")
        assert np.array_equal(Y, ref), what
    else:
        ref = oracle.dense_f32_chains(np.ascontiguousarray(X), np.ascontiguousarray(W), b, "relu")
        assert_f32_parity(np.ascontiguousarray(Y), ref, K)
    # nothing outside the output view was written
    assert np.array_equal(Yb[outside], Yb_before[outside]), what


def test_pipeline_with_device_weights(lib):
    """Host X and Y with W and b already on the device (zero-copy): the
    pipeline uploads only X's row blocks."""
    import torch
    rng = np.random.default_rng(7)
    M, K, N = 3000, 1024, 1536
    Xb, X = _view(rng, M, K, 0, 0, np.float32)
    W = rng.standard_normal((K, N), dtype=np.float32) / np.float32(np.sqrt(K))
    b = rng.standard_normal(N, dtype=np.float32)
    tW, tb = torch.from_numpy(W).cuda(), torch.from_numpy(b).cuda()
    Yb, Y = _view(rng, M, N, 0, 0, np.float32)
    Y[...] = np.nan
    args = (_desc2(Xb, X) + [tW.data_ptr(), tW.data_ptr(), 0, K, N, N, 1] +
            [tb.data_ptr(), tb.data_ptr(), 0, N, 1] + _desc2(Yb, Y))
    fn = ctypes.CFUNCTYPE(None, *([ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 5) * 2 +
                          [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64] +
                          [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 5)(
        ctypes.cast(lib.edsl_hip_dense_relu_f32, ctypes.c_void_p).value)
    lib.edsl_hip_clear_error()
    fn(*args)
    _native.raise_on_error("edsl_hip_dense_relu_f32")
    plan = _native.last_plan()
    assert plan.startswith("host pipeline"), plan
    assert_f32_parity(Y, oracle.dense_f32_chains(X, W, b, "relu"), K)
