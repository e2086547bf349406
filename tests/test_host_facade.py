"""Host facade logic (no device calls): descriptor packing identical to the
reference backend's, type rules, pattern -> entry-point binding."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from mlir_edsl_hip import _native
from mlir_edsl_hip.backend import (HipBackend, TensorType, check_dense_signature, epilogue_code, f32,
                                   i32, make_memref_descriptor, make_output_descriptor)
from mlir_edsl_hip.inputs import WORKLOADS, make_inputs


def test_memref_descriptor_layout_matches_reference_packing():
    # reference mlir_edsl/backend.py:70-102: [ptr, ptr, 0] + sizes + strides (elements)
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    types, vals, buf = make_memref_descriptor(a, TensorType((3, 4), f32))
    assert vals == [a.ctypes.data, a.ctypes.data, 0, 3, 4, 4, 1]
    assert types == [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 5
    assert buf is a


def test_non_contiguous_input_is_made_contiguous():
    a = np.arange(24, dtype=np.float32).reshape(4, 6)[:, ::2]
    _, vals, buf = make_memref_descriptor(a, TensorType((4, 3), f32))
    assert buf.flags["C_CONTIGUOUS"] and np.array_equal(buf, a)
    assert vals[3:] == [4, 3, 3, 1]


def test_dtype_mismatch_raises():
    with pytest.raises(TypeError, match="does not match"):
        make_memref_descriptor(np.zeros((2, 2), np.float64), TensorType((2, 2), f32))


def test_output_descriptor_row_major():
    # reference mlir_edsl/backend.py:37-67
    types, vals, buf = make_output_descriptor(TensorType((5, 7), i32))
    assert buf.dtype == np.int32 and buf.shape == (5, 7)
    assert vals == [buf.ctypes.data, buf.ctypes.data, 0, 5, 7, 7, 1]


def test_type_rules_follow_reference_messages():
    with pytest.raises(TypeError, match="2D tensor"):
        check_dense_signature("matmul", [TensorType((2,), f32), TensorType((2, 2), f32)])
    with pytest.raises(TypeError, match="inner dimensions must match"):
        check_dense_signature("matmul", [TensorType((2, 3), f32), TensorType((2, 2), f32)])
    with pytest.raises(TypeError, match="element types must match"):
        check_dense_signature("matmul", [TensorType((2, 2), f32), TensorType((2, 2), i32)])
    with pytest.raises(TypeError, match="bias"):
        check_dense_signature("dense_relu", [TensorType((2, 3), f32), TensorType((3, 4), f32),
                                             TensorType((3,), f32)])
    out = check_dense_signature("dense_relu", [TensorType((2, 3), f32), TensorType((3, 4), f32),
                                               TensorType((4,), f32)])
    assert out == TensorType((2, 4), f32)


def test_patterns_bind_the_declared_entry_points():
    be = HipBackend()
    cases = {
        "matmul": [TensorType((4, 4), f32)] * 2,
        "matmul_relu": [TensorType((4, 4), i32)] * 2,
        "matmul_bias": [TensorType((4, 4), f32)] * 2 + [TensorType((4,), f32)],
        "dense_relu": [TensorType((4, 4), i32)] * 2 + [TensorType((4,), i32)],
        "dense_leaky": [TensorType((4, 4), f32)] * 2 + [TensorType((4,), f32)],
    }
    L = _native.lib()
    for pattern, types in cases.items():
        fn = be.compile_dense(f"fn_{pattern}", pattern, types)
        assert fn.symbol in _native.MEMREF_ENTRY_POINTS
        addr = ctypes.cast(getattr(L, fn.symbol), ctypes.c_void_p).value
        assert be.get_function_pointer(f"fn_{pattern}") == addr
    assert sorted(be.list_functions()) == sorted(f"fn_{p}" for p in cases)
    with pytest.raises(TypeError):
        be.compile_dense("bad", "dense_leaky", [TensorType((4, 4), i32)] * 2 + [TensorType((4,), i32)])
    be.clear_module()
    assert be.list_functions() == []


def test_epilogue_codes_match_header():
    assert epilogue_code("matmul") == _native.EPI_NONE
    assert epilogue_code("matmul_bias") == _native.EPI_BIAS
    assert epilogue_code("matmul_relu") == _native.EPI_RELU
    assert epilogue_code("dense_relu") == _native.EPI_BIAS_RELU
    assert epilogue_code("dense_leaky") == _native.EPI_BIAS_LEAKY


def test_target_and_opt_level_validation():
    be = HipBackend()
    with pytest.raises(ValueError):
        be.set_target("tpu")
    with pytest.raises(ValueError):
        be.set_optimization_level(1)
    be.set_target("gpu")
    be.set_optimization_level(3)


def test_workload_inputs_are_deterministic_and_in_range():
    w = WORKLOADS["c5"]
    X1, W1, b1 = make_inputs(w, M=64, K=64, N=64)
    X2, W2, b2 = make_inputs(w, M=64, K=64, N=64)
    assert np.array_equal(X1, X2) and np.array_equal(b1, b2)
    assert X1.min() >= -8 and X1.max() <= 7 and b1.min() >= -512 and b1.max() <= 511
    A, B = make_inputs(WORKLOADS["c1"], M=64, K=64, N=64)
    assert A.dtype == np.float32 and A.min() >= -1 and A.max() < 1
    X, W, b = make_inputs(WORKLOADS["c2"], M=32, K=1024, N=16)
    assert abs(float(W.std()) - 1 / 32) < 0.005 and np.abs(b).max() <= 0.1


def test_execute_gpu_function_builds_no_reference_cycles():
    """The host-array entry reuses per-thread argument arrays: building them
    per call (ctypes.cast) left ~5 cyclic objects per call, which with torch
    loaded made every few hundred calls pay a full garbage collection of tens
    of ms. Here the call fails (no device in this container) after the
    marshalling; on a GPU box it succeeds; neither may leave cyclic garbage
    that grows with the number of calls."""
    import gc
    be = HipBackend()
    A = np.ones((4, 4), np.float32)
    be.compile_dense("cyc", "matmul", [TensorType((4, 4), f32)] * 2)

    def call():
        try:
            be.execute_gpu_function("cyc", A, A)
        except RuntimeError:
            pass

    call()  # creates this thread's argument arrays (once)
    gc.collect()
    gc.disable()
    try:
        for _ in range(200):
            call()
        unreachable = gc.collect()
    finally:
        gc.enable()
    assert unreachable < 20, unreachable  # the per-call arrays left ~1000 here


def test_dense_launch_rejects_host_tensors_before_any_device_call():
    # The combined operand check fails on a CPU tensor and the detailed
    # checks name the operand; nothing reaches the library.
    import torch
    from mlir_edsl_hip.device import dense_launch
    X, W, Y = torch.zeros(4, 8), torch.zeros(8, 16), torch.zeros(4, 16)
    with pytest.raises(ValueError, match="X must be a GPU tensor"):
        dense_launch(X, W, None, Y, 0)
    with pytest.raises(TypeError, match="unsupported dtype"):
        dense_launch(X.double(), W.double(), None, Y.double(), 0)
