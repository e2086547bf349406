"""`_mlir_backend`-compatible compiler for the HIP dense path.

The reference front end reaches its native backend through one pybind
module, ``mlir_edsl._mlir_backend``, and one class in it, ``MLIRCompiler``
(reference cpp/src/python_bindings.cpp:8-98, used by mlir_edsl/backend.py).
This module provides that class with the same methods, argument names and
error behaviour, implemented on the C ABI of include/edsl_hip_program.h:
serialized ``FunctionDef`` bytes in, the dense-path program recognised and
bound to the gfx950 kernels, function pointers with the reference JIT's
memref calling convention out.

Installed as ``mlir_edsl/_mlir_backend.py`` containing
``from mlir_edsl_hip._mlir_backend import MLIRCompiler``, it lets the
unchanged front end (``@ml_function`` / ``CppMLIRBackend``) run dense-path
functions on the GPU, for either ``target``.

Only dense-path programs compile (matmul, relu(matmul), matmul + bias,
relu / leaky_relu of it, the integer tensor_map If-ReLU, and chains of such
layers); anything else raises RuntimeError naming what was found.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

from . import _native

_lib = None


def _L() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        L = _native.lib()
        vp, c_int, sz, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_int64
        L.edsl_hip_module_create.argtypes = []
        L.edsl_hip_module_create.restype = vp
        L.edsl_hip_module_destroy.argtypes = [vp]
        L.edsl_hip_module_destroy.restype = None
        L.edsl_hip_module_compile_function.argtypes = [vp, ctypes.c_char_p, sz]
        L.edsl_hip_module_compile_function.restype = c_int
        L.edsl_hip_module_has_function.argtypes = [vp, ctypes.c_char_p]
        L.edsl_hip_module_has_function.restype = c_int
        L.edsl_hip_module_list_functions.argtypes = [vp, ctypes.c_char_p, sz]
        L.edsl_hip_module_list_functions.restype = c_int
        L.edsl_hip_module_clear.argtypes = [vp]
        L.edsl_hip_module_clear.restype = None
        L.edsl_hip_module_get_function_pointer.argtypes = [vp, ctypes.c_char_p]
        L.edsl_hip_module_get_function_pointer.restype = vp
        L.edsl_hip_module_execute_gpu_function.argtypes = [
            vp, ctypes.c_char_p, c_int, ctypes.POINTER(vp), ctypes.POINTER(ctypes.POINTER(i64)),
            ctypes.POINTER(c_int), vp, ctypes.POINTER(i64), c_int, sz]
        L.edsl_hip_module_execute_gpu_function.restype = c_int
        L.edsl_hip_module_describe.argtypes = [vp, ctypes.c_char_p, sz]
        L.edsl_hip_module_describe.restype = c_int
        L.edsl_hip_module_last_failure.argtypes = [vp, ctypes.c_char_p, sz]
        L.edsl_hip_module_last_failure.restype = c_int
        L.edsl_hip_module_function_form.argtypes = [
            vp, ctypes.c_char_p, ctypes.POINTER(c_int), ctypes.POINTER(c_int), ctypes.c_char_p, sz]
        L.edsl_hip_module_function_form.restype = c_int
        L.edsl_hip_module_function_layer.argtypes = [
            vp, ctypes.c_char_p, c_int, ctypes.POINTER(c_int), ctypes.POINTER(c_int),
            ctypes.POINTER(c_int), ctypes.POINTER(c_int), ctypes.POINTER(ctypes.c_float)]
        L.edsl_hip_module_function_layer.restype = c_int
        _lib = L
    return _lib


def _text(fn, *args) -> str:
    """Calls a (..., char* buf, size_t len) -> needed-length entry point."""
    n = fn(*args, None, 0)
    buf = ctypes.create_string_buffer(n + 1)
    fn(*args, buf, n + 1)
    return buf.value.decode(errors="replace")


def _raise(where: str) -> None:
    code, msg = _native.last_error()
    raise RuntimeError(msg if msg else f"{where} failed (code {code})")


_INJECTED = "__test_failure_inject__"


class MLIRCompiler:
    """Same surface as the reference pybind class ``MLIRCompiler``."""

    def __init__(self):
        self._m = _L().edsl_hip_module_create()
        if not self._m:
            raise MemoryError("edsl_hip_module_create failed")
        self._target = "cpu"
        self._opt_level = 2
        self._capture = False
        self._snapshots: list[tuple[str, str]] = []
        self._failure = ""
        self._injected = False

    def __del__(self):
        m, self._m = getattr(self, "_m", None), None
        if m and _lib is not None:
            _lib.edsl_hip_module_destroy(m)

    # ---------------------------------------------------------- compilation
    def compile_function(self, function_def_bytes: bytes) -> None:
        """Compile function from protobuf FunctionDef bytes."""
        data = bytes(function_def_bytes)
        if _L().edsl_hip_module_compile_function(self._m, data, len(data)) != 0:
            self._failure = _text(_L().edsl_hip_module_last_failure, self._m)
            _raise("compile_function")
        self._failure = ""

    def _finalize(self) -> None:
        # The reference lowers the whole module on first use; an injected
        # ill-typed function makes that fail for every function.
        if self._injected:
            self._failure = (f"func.func @{_INJECTED}() -> f64 {{\n  %c0_i32 = arith.constant 0 : i32\n"
                             f"  return %c0_i32 : i32  // type mismatch\n}}\n" + self.get_module_ir())
            raise RuntimeError("Lowering pipeline failed: 'func.return' op type of return operand 0 "
                               f"('i32') doesn't match function result type ('f64') in @{_INJECTED}")
        if self._capture:
            self._snapshots = [("hip-dense-dispatch", self.get_module_ir())]

    def get_function_pointer(self, name: str) -> int:
        """Entry point with the reference JIT symbol's calling convention."""
        self._finalize()
        p = _L().edsl_hip_module_get_function_pointer(self._m, name.encode())
        if not p:
            _raise("get_function_pointer")
        return int(p)

    def has_function(self, name: str) -> bool:
        return bool(_L().edsl_hip_module_has_function(self._m, name.encode()))

    def list_functions(self) -> list[str]:
        s = _text(_L().edsl_hip_module_list_functions, self._m)
        return s.split("\n") if s else []

    def get_module_ir(self) -> str:
        return _text(_L().edsl_hip_module_describe, self._m)

    def clear(self) -> None:
        """Forget every compiled function (and any injected failure)."""
        _L().edsl_hip_module_clear(self._m)
        self._failure = ""
        self._injected = False
        self._snapshots = []

    def get_lowering_snapshots(self) -> list[tuple[str, str]]:
        return list(self._snapshots)

    def enable_snapshot_capture(self) -> None:
        self._capture = True

    def get_failure_ir(self) -> str:
        return self._failure

    def inject_test_failure(self) -> None:
        """Testing only: the next finalize fails as with an ill-typed function."""
        self._injected = True

    def set_optimization_level(self, level: int) -> None:
        # Kernels are compiled ahead of time; the level is recorded only.
        self._opt_level = level if level in (0, 2, 3) else 2

    def set_target(self, target: str) -> None:
        # Both targets run on the HIP kernels: "cpu" calls go through the
        # function pointer with host buffers, "gpu" through execute_gpu_function.
        self._target = "gpu" if target == "gpu" else "cpu"

    # ------------------------------------------------------------ execution
    def execute_gpu_function(self, name: str, inputs: Sequence, output_shape: Sequence[int],
                             element_size: int) -> bytes:
        """inputs: list of (data_ptr_int, shape_list); returns the raw output bytes."""
        self._finalize()
        n = len(inputs)
        ptrs = (ctypes.c_void_p * n)(*[int(p) for p, _ in inputs])
        shape_arrays = [(ctypes.c_int64 * len(s))(*[int(d) for d in s]) for _, s in inputs]
        shapes = (ctypes.POINTER(ctypes.c_int64) * n)(
            *[ctypes.cast(a, ctypes.POINTER(ctypes.c_int64)) for a in shape_arrays])
        ranks = (ctypes.c_int * n)(*[len(s) for _, s in inputs])
        out_elems = 1
        for d in output_shape:
            out_elems *= int(d)
        out = ctypes.create_string_buffer(out_elems * int(element_size))
        oshape = (ctypes.c_int64 * len(output_shape))(*[int(d) for d in output_shape])
        rc = _L().edsl_hip_module_execute_gpu_function(
            self._m, name.encode(), n, ptrs, shapes, ranks, ctypes.cast(out, ctypes.c_void_p), oshape,
            len(output_shape), int(element_size))
        if rc != 0:
            _raise("execute_gpu_function")
        return out.raw

    # ----------------------------------------------------------- extension
    def function_form(self, name: str) -> dict:
        """How a compiled function was matched (no reference counterpart):
        dtype, the program as text, and its layers in execution order (x = -1
        reads the previous layer's output). The top-level x is the first
        layer's input; w, b, epilogue and alpha are the last layer's."""
        L = _L()
        dt, nl = ctypes.c_int(), ctypes.c_int()
        buf = ctypes.create_string_buffer(512)
        if L.edsl_hip_module_function_form(self._m, name.encode(), ctypes.byref(dt), ctypes.byref(nl), buf,
                                           len(buf)) != 0:
            _raise("function_form")
        layers = []
        for i in range(nl.value):
            x, w, b, epi = (ctypes.c_int() for _ in range(4))
            alpha = ctypes.c_float()
            if L.edsl_hip_module_function_layer(self._m, name.encode(), i, ctypes.byref(x), ctypes.byref(w),
                                                ctypes.byref(b), ctypes.byref(epi), ctypes.byref(alpha)) != 0:
                _raise("function_layer")
            layers.append({"x": x.value, "w": w.value, "b": b.value, "epilogue": epi.value,
                           "alpha": alpha.value})
        return {"dtype": "f32" if dt.value == _native.DTYPE_F32 else "i32", "form": buf.value.decode(),
                "layers": layers, "x": layers[0]["x"], "w": layers[-1]["w"], "b": layers[-1]["b"],
                "epilogue": layers[-1]["epilogue"], "alpha": layers[-1]["alpha"]}
