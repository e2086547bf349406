"""Host facade for the gfx950 dense path.

Mirrors the reference backend's calling sequence (reference
mlir_edsl/backend.py:37-102 for descriptor packing, :162-198 for the JIT call,
:248-271 for the GPU host-array entry) on top of libedsl_hip's C ABI:

* ``execute_function(name, *arrays)`` flattens every array into MLIR's
  expanded memref descriptor (allocated, aligned, offset, sizes, strides),
  appends a freshly allocated output descriptor, and calls the bound C-ABI
  function pointer through ``ctypes.CFUNCTYPE(None, *types)(ptr)(*args)`` --
  the same call the reference makes on its JIT'd symbol.
* ``execute_gpu_function(name, *arrays)`` hands (pointer, shape) pairs to
  ``edsl_hip_execute_gpu_function``, the counterpart of the reference's
  pybind ``execute_gpu_function`` (cpp/src/python_bindings.cpp:69-97).

Operands may be numpy arrays (host memory: copied in and out by the library)
or torch tensors on the GPU (used in place; the output is then a GPU tensor).

A function is bound to one of the dense-path patterns when it is compiled:
``matmul``, ``matmul_relu``, ``matmul_bias``, ``dense_relu``, ``dense_leaky``,
and the f32 If-ReLU map forms ``dense_if_relu`` and ``matmul_if_relu``.
"""
from __future__ import annotations

import ctypes
import enum
import threading
from dataclasses import dataclass, field
from typing import Any, Sequence

import numpy as np

from . import _native


class ScalarType(enum.Enum):
    F32 = "f32"
    I32 = "i32"

    @property
    def numpy_dtype(self):
        return np.float32 if self is ScalarType.F32 else np.int32

    @property
    def torch_dtype(self):
        import torch
        return torch.float32 if self is ScalarType.F32 else torch.int32

    @property
    def code(self) -> int:
        return _native.DTYPE_F32 if self is ScalarType.F32 else _native.DTYPE_I32


f32 = ScalarType.F32
i32 = ScalarType.I32


@dataclass(frozen=True)
class TensorType:
    shape: tuple[int, ...]
    element_type: ScalarType

    def __post_init__(self):
        object.__setattr__(self, "shape", tuple(int(d) for d in self.shape))


# pattern -> (has_bias, activation, number of inputs)
PATTERNS = {
    "matmul": (False, "none", 2),
    "matmul_relu": (False, "relu", 2),
    "matmul_bias": (True, "none", 3),
    "dense_relu": (True, "relu", 3),
    "dense_leaky": (True, "leaky", 3),
    # tensor_map(... , lambda v: If(v > 0.0, v, 0.0)) over f32: NaN and -0 give +0
    "dense_if_relu": (True, "if_relu", 3),
    "matmul_if_relu": (False, "if_relu", 2),
}

_SYMBOLS = {
    ("matmul", f32): "edsl_hip_matmul_f32",
    ("matmul", i32): "edsl_hip_matmul_i32",
    ("matmul_relu", f32): "edsl_hip_matmul_relu_f32",
    ("matmul_relu", i32): "edsl_hip_matmul_relu_i32",
    ("matmul_bias", f32): "edsl_hip_matmul_bias_f32",
    ("matmul_bias", i32): "edsl_hip_matmul_bias_i32",
    ("dense_relu", f32): "edsl_hip_dense_relu_f32",
    ("dense_relu", i32): "edsl_hip_dense_relu_i32",
    ("dense_leaky", f32): "edsl_hip_dense_leaky_relu_f32",
    ("dense_if_relu", f32): "edsl_hip_dense_if_relu_f32",
    ("matmul_if_relu", f32): "edsl_hip_matmul_if_relu_f32",
}

_PATTERN_CODES = {
    "matmul": _native.PATTERN_MATMUL,
    "matmul_relu": _native.PATTERN_MATMUL_RELU,
    "matmul_bias": _native.PATTERN_MATMUL_BIAS,
    "dense_relu": _native.PATTERN_DENSE_RELU,
    "dense_leaky": _native.PATTERN_DENSE_LEAKY,
    "dense_if_relu": _native.PATTERN_DENSE_IF_RELU,
    "matmul_if_relu": _native.PATTERN_MATMUL_IF_RELU,
}


def epilogue_code(pattern: str) -> int:
    bias, act, _ = PATTERNS[pattern]
    return (1 if bias else 0) | ({"none": 0, "relu": 1, "leaky": 2, "if_relu": 3}[act] << 1)


@dataclass
class DenseFunction:
    """A compiled function bound to a dense-path pattern."""
    name: str
    pattern: str
    param_types: list[TensorType]
    return_type: TensorType
    alpha: float = 0.01
    symbol: str = field(init=False)

    def __post_init__(self):
        et = self.return_type.element_type
        key = (self.pattern, et)
        if key not in _SYMBOLS:
            raise TypeError(f"pattern {self.pattern!r} is not defined for {et.value}")
        self.symbol = _SYMBOLS[key]


def check_dense_signature(pattern: str, param_types: Sequence[TensorType]) -> TensorType:
    """Type rules of the reference AST nodes for the dense path; returns the
    result type. Messages follow LinalgMatmul._validate / LinalgBinaryOp
    (reference mlir_edsl/ast/nodes/linalg.py:95-123, 183-198)."""
    if pattern not in PATTERNS:
        raise ValueError(f"unknown dense pattern {pattern!r}")
    bias, _, n_in = PATTERNS[pattern]
    if len(param_types) != n_in:
        raise TypeError(f"{pattern} takes {n_in} tensors, got {len(param_types)}")
    lhs, rhs = param_types[0], param_types[1]
    if len(lhs.shape) != 2 or len(rhs.shape) != 2:
        raise TypeError(f"matmul requires 2D tensor operands, got {lhs.shape} and {rhs.shape}")
    if lhs.element_type is not rhs.element_type:
        raise TypeError(f"matmul operand element types must match: {lhs.element_type.value} "
                        f"vs {rhs.element_type.value}")
    if lhs.shape[1] != rhs.shape[0]:
        raise TypeError(f"matmul inner dimensions must match: {lhs.shape[1]} vs {rhs.shape[0]}")
    out = TensorType((lhs.shape[0], rhs.shape[1]), lhs.element_type)
    if bias:
        b = param_types[2]
        if len(b.shape) != 1 or b.shape[0] != out.shape[1]:
            raise TypeError(f"bias shape {b.shape} does not broadcast over {out.shape}")
        if b.element_type is not out.element_type:
            raise TypeError("bias element type must match the matmul result")
    return out


def _is_torch(x) -> bool:
    return type(x).__module__.startswith("torch")


def make_memref_descriptor(data, tensor_type: TensorType):
    """(c_types, c_values, keepalive) for one tensor argument.

    numpy arrays are made C-contiguous like the reference does
    (mlir_edsl/backend.py:70-102); torch tensors keep their row stride and
    must have unit inner stride."""
    et = tensor_type.element_type
    ndim = len(tensor_type.shape)
    if _is_torch(data):
        if data.dtype != et.torch_dtype:
            raise TypeError(f"tensor dtype {data.dtype} does not match expected {et.value}")
        if data.dim() != ndim:
            raise TypeError(f"expected a {ndim}-D tensor, got {data.dim()}-D")
        if ndim and data.shape[-1] > 1 and data.stride(-1) != 1:
            data = data.contiguous()
        ptr = data.data_ptr()
        shape = list(data.shape)
        strides = list(data.stride())
    else:
        data = np.asarray(data)
        if data.dtype != et.numpy_dtype:
            raise TypeError(f"ndarray dtype {data.dtype} does not match expected "
                            f"{np.dtype(et.numpy_dtype)} for {tensor_type}")
        if data.ndim != ndim:
            raise TypeError(f"expected a {ndim}-D array, got {data.ndim}-D")
        if not data.flags["C_CONTIGUOUS"]:
            data = np.ascontiguousarray(data)
        ptr = data.ctypes.data
        shape = list(data.shape)
        strides = [s // data.itemsize for s in data.strides]
    c_types = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64] + [ctypes.c_int64] * (2 * ndim)
    c_vals = [ptr, ptr, 0] + shape + strides
    return c_types, c_vals, data


def make_output_descriptor(tensor_type: TensorType, like=None):
    """Output buffer + descriptor: numpy for host callers, a torch tensor on
    the same device when the inputs are GPU tensors."""
    shape = list(tensor_type.shape)
    et = tensor_type.element_type
    if like is not None and _is_torch(like) and like.is_cuda:
        import torch
        buf = torch.empty(shape, dtype=et.torch_dtype, device=like.device)
        ptr = buf.data_ptr()
    else:
        buf = np.empty(shape, dtype=et.numpy_dtype)
        ptr = buf.ctypes.data
    strides = [1] * len(shape)
    for i in range(len(shape) - 2, -1, -1):
        strides[i] = strides[i + 1] * shape[i + 1]
    c_types = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64] + [ctypes.c_int64] * (2 * len(shape))
    c_vals = [ptr, ptr, 0] + shape + strides
    return c_types, c_vals, buf


def _data_ptr(a: np.ndarray) -> int:
    return a.__array_interface__["data"][0]


class _GpuArgs:
    """Argument arrays of edsl_hip_execute_gpu_function for n inputs of rank
    <= 2: pointers, per-input shape arrays (and the array of pointers to
    them), ranks and the output shape."""

    def __init__(self, n: int):
        self.ptrs = (ctypes.c_void_p * n)()
        self.ranks = (ctypes.c_int * n)()
        self.dims = [(ctypes.c_int64 * 2)() for _ in range(n)]
        self.shapes = (ctypes.POINTER(ctypes.c_int64) * n)(
            *[ctypes.cast(d, ctypes.POINTER(ctypes.c_int64)) for d in self.dims])
        self.oshape = (ctypes.c_int64 * 2)()


class HipBackend:
    """Function registry + execution for the HIP dense path (one per process,
    see :func:`get_backend`)."""

    def __init__(self):
        self._lib = _native.lib()
        self._functions: dict[str, DenseFunction] = {}
        self._target = "gpu"
        self._opt_level = 2
        self._tls = threading.local()  # per-thread argument arrays of execute_gpu_function

    # ---------------------------------------------------------- compilation
    def compile_dense(self, name: str, pattern: str, param_types: Sequence[TensorType],
                      alpha: float = 0.01) -> DenseFunction:
        ret = check_dense_signature(pattern, param_types)
        fn = DenseFunction(name, pattern, list(param_types), ret, alpha)
        self._functions[name] = fn
        return fn

    def _gpu_args(self, n: int) -> "_GpuArgs":
        cache = self._tls.__dict__.setdefault("gpu_args", {})
        if n not in cache:
            cache[n] = _GpuArgs(n)
        return cache[n]

    def has_function(self, name: str) -> bool:
        return name in self._functions

    def list_functions(self) -> list[str]:
        return list(self._functions)

    def clear_module(self) -> None:
        self._functions.clear()

    def set_target(self, target: str) -> None:
        if target not in ("cpu", "gpu"):
            raise ValueError(f"Invalid target '{target}'. Must be 'cpu' or 'gpu'.")
        self._target = target

    def set_optimization_level(self, level: int) -> None:
        if level not in (0, 2, 3):
            raise ValueError(f"Invalid optimization level {level}. Must be 0, 2, or 3.")
        self._opt_level = level

    def get_function_pointer(self, name: str) -> int:
        fn = self._functions[name]
        return ctypes.cast(getattr(self._lib, fn.symbol), ctypes.c_void_p).value

    # ------------------------------------------------------------ execution
    def execute_function(self, name: str, *args):
        """Call the bound entry point with flattened memref descriptors."""
        fn = self._functions[name]
        if len(args) != len(fn.param_types):
            raise TypeError(f"{name} takes {len(fn.param_types)} arguments, got {len(args)}")
        flat_types: list[Any] = []
        flat_vals: list[Any] = []
        live = []
        for pt, val in zip(fn.param_types, args):
            t, v, buf = make_memref_descriptor(val, pt)
            flat_types += t
            flat_vals += v
            live.append(buf)
        t, v, out = make_output_descriptor(fn.return_type, like=args[0])
        flat_types += t
        flat_vals += v
        live.append(out)
        if fn.pattern == "dense_leaky":
            flat_types.append(ctypes.c_float)
            flat_vals.append(fn.alpha)
        self._lib.edsl_hip_clear_error()
        ctypes.CFUNCTYPE(None, *flat_types)(self.get_function_pointer(name))(*flat_vals)
        _native.raise_on_error(name)
        return out

    def execute_gpu_function(self, name: str, *args) -> np.ndarray:
        """Host arrays in, host array out (reference execute_gpu_function)."""
        fn = self._functions[name]
        n = len(fn.param_types)
        if len(args) != n:
            raise TypeError(f"{name} takes {n} arguments, got {len(args)}")
        arrays = []
        for pt, val in zip(fn.param_types, args):
            a = np.asarray(val)
            if a.dtype != pt.element_type.numpy_dtype:
                raise TypeError(f"ndarray dtype {a.dtype} does not match expected "
                                f"{np.dtype(pt.element_type.numpy_dtype)}")
            if a.ndim > 2:
                raise TypeError(f"rank {a.ndim} operand: the dense path takes 1-D and 2-D arrays")
            arrays.append(np.ascontiguousarray(a))
        # The argument arrays are reused per thread and filled in place: building
        # them per call (ctypes.cast in particular) leaves reference cycles that
        # pile up until a full garbage collection, tens of ms with torch loaded.
        a_ = self._gpu_args(n)
        for i, a in enumerate(arrays):
            a_.ptrs[i] = _data_ptr(a)
            a_.ranks[i] = a.ndim
            for d, extent in enumerate(a.shape):
                a_.dims[i][d] = extent
        out = np.empty(fn.return_type.shape, dtype=fn.return_type.element_type.numpy_dtype)
        a_.oshape[0], a_.oshape[1] = out.shape
        rc = self._lib.edsl_hip_execute_gpu_function(
            _PATTERN_CODES[fn.pattern], fn.return_type.element_type.code, n, a_.ptrs, a_.shapes, a_.ranks,
            _data_ptr(out), a_.oshape, 2, 4, fn.alpha)
        if rc != 0:
            _native.raise_on_error(name)
        return out


_global_backend: HipBackend | None = None


_backend_lock = threading.Lock()


def get_backend() -> HipBackend:
    """The process-wide backend, created on first use (by one thread only)."""
    global _global_backend
    if _global_backend is None:
        with _backend_lock:
            if _global_backend is None:
                _global_backend = HipBackend()
    return _global_backend


def tensor_type_of(x) -> TensorType:
    if _is_torch(x):
        import torch
        et = {torch.float32: f32, torch.int32: i32}.get(x.dtype)
        shape = tuple(x.shape)
    else:
        et = {np.dtype(np.float32): f32, np.dtype(np.int32): i32}.get(np.asarray(x).dtype)
        shape = np.asarray(x).shape
    if et is None:
        raise TypeError(f"unsupported element type {x.dtype} (f32 and i32 only)")
    return TensorType(shape, et)


def run(pattern: str, *args, alpha: float = 0.01):
    """Compile (once per shape/dtype) and execute a dense-path pattern."""
    be = get_backend()
    types = [tensor_type_of(a) for a in args]
    name = f"{pattern}_" + "_".join(f"{t.element_type.value}{'x'.join(map(str, t.shape))}" for t in types)
    if pattern == "dense_leaky":
        name += f"_a{alpha!r}"
    if not be.has_function(name):
        be.compile_dense(name, pattern, types, alpha=alpha)
    return be.execute_function(name, *args)


def matmul(A, B):
    return run("matmul", A, B)


def dense(X, W, b=None, act: str = "relu", alpha: float = 0.01):
    """act(X @ W (+ b)) with act in {'none', 'relu', 'leaky', 'if_relu'}
    ('if_relu': the f32 map body If(v > 0.0, v, 0.0))."""
    if b is None:
        if act == "none":
            return run("matmul", X, W)
        if act == "relu":
            return run("matmul_relu", X, W)
        if act == "if_relu":
            return run("matmul_if_relu", X, W)
        raise ValueError("leaky_relu without bias is not a dense-path pattern")
    pattern = {"none": "matmul_bias", "relu": "dense_relu", "leaky": "dense_leaky", "if_relu": "dense_if_relu"}[act]
    return run(pattern, X, W, b, alpha=alpha)
