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
    layer's matmul in full, then its bias + activation, then the next. f32
    chains are computed once per rounding chain, every layer on that chain."""
    def run(chain):
        h = None
        for L in form["layers"]:
            X = args[L["x"]] if L["x"] >= 0 else h
            W = args[L["w"]]
            b = args[L["b"]] if L["b"] >= 0 else None
            act = {0: "none", 1: "relu", 2: "leaky", 3: "if_relu"}[L["epilogue"] >> 1]
            if form["dtype"] == "i32":
                h = oracle.dense_i32(X, W, b, act)
            else:
                h = oracle.dense_f32(X, W, b, act, L["alpha"], chain=chain)
        return h
    if form["dtype"] == "i32":
        return run(None)
    return oracle.F32Chains(run("fma"), run("muladd"))


def _arr(ref):
    """The array whose shape and dtype the output has."""
    return ref.fma if isinstance(ref, oracle.F32Chains) else ref


def _check(got, ref, K):
    if isinstance(ref, oracle.F32Chains):
        assert_f32_parity(got, ref, K)
    else:
        assert got.dtype == np.int32 and np.array_equal(got, ref)


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
    comp.set_target("gpu")
    comp.compile_function(open(os.path.join(GOLDEN, case["file"]), "rb").read())
    name = case["function"]
    form = comp.function_form(name)
    K = max(case["param_shapes"][L["w"]][0] for L in form["layers"])
    ptr = comp.get_function_pointer(name)
    for seed, wide in ((1, False), (2, True)):
        args = _inputs(case, seed, wide)
        ref = _reference(form, args)
        like = _arr(ref)
        # 1) host buffers through the function pointer
        out = np.empty(like.shape, dtype=like.dtype)
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
        dout = torch.empty(like.shape, dtype=dargs[0].dtype, device="cuda")
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
                                        list(like.shape), like.dtype.itemsize)
        assert type(raw) is bytes and len(raw) == like.nbytes  # the reference returns py::bytes
        _check(np.frombuffer(raw, dtype=like.dtype).reshape(like.shape), ref, K)
        # a second call returns a new object; the first result is unchanged
        first = bytes(raw)
        raw2 = comp.execute_gpu_function(name, [(a.ctypes.data, list(a.shape)) for a in args],
                                         list(like.shape), like.dtype.itemsize)
        assert raw2 is not raw and raw == first and raw2 == first
    if "execute_gpu_function" in case:  # the reference front end's call has the same shapes
        call = case["execute_gpu_function"]
        assert call["input_shapes"] == case["param_shapes"] and call["element_size"] == 4
    comp.clear()


# --------------------------------------------- device-resident parameters
def _call_pointer(ptr, args, out):
    types, vals = [], []
    for a in list(args) + [out]:
        t, v = _descriptor_types_and_values(a)
        types += t
        vals += v
    _native.lib().edsl_hip_clear_error()
    ctypes.CFUNCTYPE(None, *types)(ptr)(*vals)
    _native.raise_on_error("function pointer")


def _layer_inputs(M, K, N, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.float32(np.sqrt(K))).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, N).astype(np.float32)
    return X, W, b


@pytest.mark.parametrize("M, K, N", [(16, 8192, 8192), (300, 257, 130), (2048, 1024, 1024)],
                         ids=["c4", "odd", "pipelined"])
def test_bound_parameters_match_unbound_calls_and_the_oracle(M, K, N, torch_cuda):
    """W and b bound as device-resident snapshots: calls through the function
    pointer and execute_gpu_function that pass the same arrays read them in
    place ([resident: W,b] in the plan) and give the unbound result bit for
    bit; rebinding to new values changes the result; another array of the
    same shape is copied in as usual; unbinding goes back to copying."""
    from mlir_edsl_hip import wire
    comp = MLIRCompiler()
    comp.set_target("gpu")
    name = "dense_bound"
    comp.compile_function(wire.dense_layer(name, M, K, N))
    ptr = comp.get_function_pointer(name)
    X, W, b = _layer_inputs(M, K, N, M + K)
    ref = oracle.dense_f32_chains(X, W, b, "relu")
    plain = np.empty((M, N), np.float32)
    _call_pointer(ptr, (X, W, b), plain)
    assert "resident" not in _native.last_plan()
    _check(plain, ref, K)

    comp.bind_parameter(name, "W", W)
    comp.bind_parameter(name, 2, b)
    bound = np.empty((M, N), np.float32)
    _call_pointer(ptr, (X, W, b), bound)
    assert _native.last_plan().endswith("[resident: W,b]"), _native.last_plan()
    assert np.array_equal(bound.view(np.uint32), plain.view(np.uint32))
    raw = comp.execute_gpu_function(name, [(a.ctypes.data, list(a.shape)) for a in (X, W, b)], [M, N], 4)
    assert _native.last_plan().endswith("[resident: W,b]"), _native.last_plan()
    assert np.array_equal(np.frombuffer(raw, np.float32).reshape(M, N), plain)
    desc = comp.get_module_ir()
    assert "// resident: %W on device" in desc and "// resident: %b on device" in desc
    assert "// last run: " in desc and "[resident: W,b]" in desc

    # The snapshot is what was bound: writing the array does not change it ...
    W2 = (W * np.float32(-0.5)).astype(np.float32)
    W[...] = W2
    stale = np.empty((M, N), np.float32)
    _call_pointer(ptr, (X, W, b), stale)
    assert np.array_equal(stale, plain)
    # ... until it is bound again.
    comp.bind_parameter(name, "W", W)
    rebound = np.empty((M, N), np.float32)
    _call_pointer(ptr, (X, W, b), rebound)
    ref2 = oracle.dense_f32_chains(X, W2, b, "relu")
    _check(rebound, ref2, K)
    assert not np.array_equal(rebound, plain)

    # A different array of the same shape is copied in, not mistaken for W.
    W3 = np.ascontiguousarray(W2[::-1])
    other = np.empty((M, N), np.float32)
    _call_pointer(ptr, (X, W3, b), other)
    assert _native.last_plan().endswith("[resident: b]"), _native.last_plan()
    _check(other, oracle.dense_f32_chains(X, W3, b, "relu"), K)

    comp.unbind_parameter(name)
    again = np.empty((M, N), np.float32)
    _call_pointer(ptr, (X, W, b), again)
    assert "resident" not in _native.last_plan()
    assert np.array_equal(again, rebound)
    comp.clear()


def test_bound_parameters_in_a_chain_and_with_device_operands(torch_cuda):
    """A two-layer chain with both weights bound, called with host X; then
    with device tensors, which never match a host snapshot."""
    from mlir_edsl_hip import wire
    torch = torch_cuda
    comp = MLIRCompiler()
    comp.set_target("gpu")
    name = "chain_bound"
    comp.compile_function(wire.dense_program(name, ("X", 64, 512), [wire.Layer("W1", 256, "b1", "relu"),
                                                                    wire.Layer("W2", 96, "b2", "leaky", 0.1)]))
    rng = np.random.default_rng(5)
    X = rng.standard_normal((64, 512), dtype=np.float32)
    W1 = (rng.standard_normal((512, 256), dtype=np.float32) / 23).astype(np.float32)
    b1 = rng.uniform(-0.1, 0.1, 256).astype(np.float32)
    W2 = (rng.standard_normal((256, 96), dtype=np.float32) / 16).astype(np.float32)
    b2 = rng.uniform(-0.1, 0.1, 96).astype(np.float32)
    args = (X, W1, b1, W2, b2)
    ref = _reference(comp.function_form(name), list(args))
    for p in ("W1", "W2"):
        comp.bind_parameter(name, p, args[comp._param_index(name, p)])
    out = np.empty((64, 96), np.float32)
    _call_pointer(comp.get_function_pointer(name), args, out)
    assert "[resident: W1,W2]" in _native.last_plan(), _native.last_plan()
    _check(out, ref, 512)
    dargs = [torch.from_numpy(a).cuda() for a in args]
    dout = torch.empty((64, 96), device="cuda")
    _call_pointer(comp.get_function_pointer(name), dargs, dout)
    torch.cuda.synchronize()
    assert "resident" not in _native.last_plan()
    _check(dout.cpu().numpy(), ref, 512)
    comp.clear()


def test_a_freed_bound_array_cannot_lend_its_address(torch_cuda):
    """The compiler holds the bound array until it is unbound, so dropping
    the caller's last reference frees nothing: new arrays of the same shape
    get other addresses and are copied in, never mistaken for the snapshot
    (a freed block is otherwise handed to the next array of its size)."""
    import gc
    import weakref
    from mlir_edsl_hip import wire
    M, K, N = 16, 64, 32
    comp = MLIRCompiler()
    comp.set_target("gpu")
    name = "dense_bound_lifetime"
    comp.compile_function(wire.dense_layer(name, M, K, N))
    ptr = comp.get_function_pointer(name)
    X, W, b = _layer_inputs(M, K, N, 77)
    comp.bind_parameter(name, "W", W)
    addr, alive = W.ctypes.data, weakref.ref(W)
    del W
    gc.collect()
    assert alive() is not None, "the bound array was released while bound"
    rng = np.random.default_rng(78)
    for trial in range(16):
        Wn = rng.standard_normal((K, N), dtype=np.float32)
        assert Wn.ctypes.data != addr, trial
        out = np.empty((M, N), np.float32)
        _call_pointer(ptr, (X, Wn, b), out)
        assert "resident: W" not in _native.last_plan(), _native.last_plan()
        _check(out, oracle.dense_f32_chains(X, Wn, b, "relu"), K)
        del Wn
    comp.unbind_parameter(name, "W")
    gc.collect()
    assert alive() is None, "unbinding keeps no reference"
    comp.clear()


def test_dyn_specialisations_run_from_one_compiler(torch_cuda):
    """Every shape variant of the DYN-declared functions (reference
    tests/linalg/test_linalg_dyn.py:86-95: one compile per call shape, under
    the shape-mangled name) compiled into one compiler, then each run through
    its function pointer and through execute_gpu_function against the
    oracle."""
    comp = MLIRCompiler()
    comp.set_target("gpu")
    cases = [c for c in DENSE if c.get("declared_dyn")]
    assert len(cases) == 6
    for c in cases:
        comp.compile_function(open(os.path.join(GOLDEN, c["file"]), "rb").read())
    for i, c in enumerate(cases):
        name = c["function"]
        form = comp.function_form(name)
        K = c["param_shapes"][0][1]
        args = _inputs(c, 40 + i, wide=True)
        ref = _reference(form, args)
        like = _arr(ref)
        print(f"{name}: {form['form']} {like.shape}", flush=True)
        out = np.empty(like.shape, like.dtype)
        _call_pointer(comp.get_function_pointer(name), args, out)
        _check(out, ref, K)
        raw = comp.execute_gpu_function(name, [(a.ctypes.data, list(a.shape)) for a in args], list(like.shape), 4)
        _check(np.frombuffer(raw, dtype=like.dtype).reshape(like.shape), ref, K)
    comp.clear()


def test_f32_if_relu_program_maps_nan_and_negative_zero_to_zero(torch_cuda):
    """tensor_map(X @ W + b, lambda v: If(v > 0.0, v, 0.0)) from the front
    end's bytes: NaN rows and -0 sums come out +0, bit for bit with the
    oracle's If epilogue (reference LinalgBuilder.cpp:141-178, cmpf ogt)."""
    c = next(c for c in DENSE if c["fixture"] == "dense_if_relu_f32")
    comp = MLIRCompiler()
    comp.set_target("gpu")
    comp.compile_function(open(os.path.join(GOLDEN, c["file"]), "rb").read())
    X, W, b = _inputs(c, 9)
    X[3, :] = np.nan                    # a NaN row: maximumf would keep NaN
    X[5, :] = 0.0
    b[:4] = -0.0                        # row 5: 0 * w sums to +0; +0 + -0 = +0
    X[7, :] = np.float32(-1e-30)        # tiny negative sums underflow toward -0
    W[:, 0] = np.float32(1e-30)
    ref = oracle.dense_f32_chains(X, W, b, "if_relu")
    out = np.empty(ref.fma.shape, np.float32)
    _call_pointer(comp.get_function_pointer(c["function"]), (X, W, b), out)
    assert not np.isnan(out).any() and not np.signbit(out).any()
    assert np.array_equal(out[3], np.zeros_like(out[3]))
    _check(out, ref, X.shape[1])
    comp.clear()
