"""GPU parity of the FunctionDef front end: the exact bytes the reference
front end serializes (single layers and chains of layers), compiled by the
`_mlir_backend`-compatible compiler and run three ways -- through the function pointer with host (numpy)
descriptors, as the reference's execute_function calls its JIT'd symbol
(reference mlir_edsl/backend.py:162-198); through the same pointer with
device tensors; and through execute_gpu_function with (pointer, shape)
pairs, as the reference's execute_gpu_function does
(reference mlir_edsl/backend.py:248-271). Each is checked against the oracle
(i32 bit-exact; f32 relative Frobenius <= 1e-5, max|delta| <= 1e-4*sqrt(K)).
"""
from __future__ import annotations

import ctypes
import json
import os

import numpy as np
import pytest

import oracle
from conftest import assert_f32_parity
from mlir_edsl_hip import _native
from mlir_edsl_hip._mlir_backend import MLIRCompiler

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
with open(os.path.join(GOLDEN, "wire_fixtures.json")) as _f:
    DENSE = [c for c in json.load(_f)["cases"] if "reject" not in c["expected"]]


def _inputs(case, seed, wide=False):
    rng = np.random.default_rng(seed)
    out = []
    for shape, dt in zip(case["param_shapes"], case["param_dtypes"]):
        if dt == "int32":
            lim = 2**20 if wide else 8
            out.append(rng.integers(-lim, lim, size=shape, dtype=np.int64).astype(np.int32))
        else:
            out.append(rng.standard_normal(shape, dtype=np.float32))
    return out


def _reference(form, args):
    """Layer by layer, as the reference lowering computes a chain: each
    layer's matmul in full, then its bias + activation, then the next."""
    h = None
    for L in form["layers"]:
        X = args[L["x"]] if L["x"] >= 0 else h
        W = args[L["w"]]
        b = args[L["b"]] if L["b"] >= 0 else None
        act = {0: "none", 1: "relu", 2: "leaky"}[L["epilogue"] >> 1]
        if form["dtype"] == "i32":
            h = oracle.dense_i32(X, W, b, act)
        else:
            h = oracle.dense_f32(X, W, b, act, L["alpha"])
    return h


def _check(got, ref, K):
    if ref.dtype == np.int32:
        assert got.dtype == np.int32 and np.array_equal(got, ref)
    else:
        assert_f32_parity(got, ref, K)


def _descriptor_types_and_values(a):
    """The reference's _make_memref_descriptor, for numpy or torch."""
    if hasattr(a, "data_ptr"):
        ptr, shape, strides = a.data_ptr(), list(a.shape), list(a.stride())
    else:
        ptr, shape, strides = a.ctypes.data, list(a.shape), [s // a.itemsize for s in a.strides]
    types = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64] + [ctypes.c_int64] * (2 * len(shape))
    return types, [ptr, ptr, 0] + shape + strides


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    return torch


@pytest.mark.parametrize("case", DENSE, ids=lambda c: c["fixture"])
def test_reference_program_runs_three_ways(case, torch_cuda):
    torch = torch_cuda
    comp = MLIRCompiler()
    comp.compile_function(open(os.path.join(GOLDEN, case["file"]), "rb").read())
    name = case["function"]
    form = comp.function_form(name)
    K = max(case["param_shapes"][L["w"]][0] for L in form["layers"])
    ptr = comp.get_function_pointer(name)
    for seed, wide in ((1, False), (2, True)):
        args = _inputs(case, seed, wide)
        ref = _reference(form, args)
        # 1) host buffers through the function pointer
        out = np.empty(ref.shape, dtype=ref.dtype)
        types, vals = [], []
        for a in args + [out]:
            t, v = _descriptor_types_and_values(a)
            types += t
            vals += v
        ctypes.CFUNCTYPE(None, *types)(ptr)(*vals)
        _native.raise_on_error(name)
        _check(out, ref, K)
        # 2) device tensors through the same pointer
        dargs = [torch.from_numpy(a).cuda() for a in args]
        dout = torch.empty(ref.shape, dtype=dargs[0].dtype, device="cuda")
        types, vals = [], []
        for a in dargs + [dout]:
            t, v = _descriptor_types_and_values(a)
            types += t
            vals += v
        ctypes.CFUNCTYPE(None, *types)(ptr)(*vals)
        _native.raise_on_error(name)
        torch.cuda.synchronize()
        _check(dout.cpu().numpy(), ref, K)
        # 3) execute_gpu_function with (pointer, shape) pairs, element size from the dtype
        raw = comp.execute_gpu_function(name, [(a.ctypes.data, list(a.shape)) for a in args],
                                        list(ref.shape), ref.dtype.itemsize)
        _check(np.frombuffer(raw, dtype=ref.dtype).reshape(ref.shape), ref, K)
    if "execute_gpu_function" in case:  # the reference front end's call has the same shapes
        call = case["execute_gpu_function"]
        assert call["input_shapes"] == case["param_shapes"] and call["element_size"] == 4
    comp.clear()
