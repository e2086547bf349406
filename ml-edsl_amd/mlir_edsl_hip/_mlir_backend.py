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
functions on the GPU.

Coexistence with the reference compiler. The front end imports exactly one
native module (reference mlir_edsl/backend.py:8-11), so replacing it would
leave every program outside the dense path (scalars, control flow, arrays,
the rest of the DSL) without a compiler. When the reference's own compiled
module is importable -- kept under another name, ``mlir_edsl._mlir_backend_ref``
or ``_mlir_backend_ref`` by default, or the module named by
``EDSL_HIP_REFERENCE_BACKEND`` -- this class owns one of its
``MLIRCompiler`` objects and hands it every function compiled while the
target is ``"cpu"`` (the front end sets the target before each compile,
reference mlir_edsl/functions/compilation.py:67): the caller asked for the CPU
JIT. Routing is by target only. A ``"gpu"`` function always compiles here,
and one that is not a dense-path program raises RuntimeError with the
decoder's message: the reference module built for this host has no GPU
support (its executeGPUFunction throws "GPU support not compiled in",
reference cpp/src/MLIRCompiler.cpp:456-461), so handing it a GPU program would
only defer the failure and hide its cause. Later calls are routed by function
name. Without a reference module, every dense function runs on the HIP
kernels whatever the target, and anything else raises RuntimeError naming
what was found.

Device-resident parameters (no reference counterpart): ``bind_parameter``
keeps a snapshot of a weight or bias in HBM, so calls that pass that same
array skip its host-to-device copy (include/edsl_hip_program.h). The bound
object is kept alive until it is unbound, rebound or the module is cleared,
so its memory cannot be freed and handed to another array while calls still
match the snapshot by address.
"""
from __future__ import annotations

import ctypes
import importlib
import os
from typing import Sequence

from . import _native

_lib = None

ERR_PROGRAM = -7  # not a dense-path program (or malformed bytes)


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
        L.edsl_hip_module_bind_parameter.argtypes = [vp, ctypes.c_char_p, c_int, vp, ctypes.POINTER(i64), c_int]
        L.edsl_hip_module_bind_parameter.restype = c_int
        L.edsl_hip_module_unbind_parameter.argtypes = [vp, ctypes.c_char_p, c_int]
        L.edsl_hip_module_unbind_parameter.restype = c_int
        L.edsl_hip_module_param_index.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(c_int)]
        L.edsl_hip_module_param_index.restype = c_int
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


_new_bytes = ctypes.pythonapi.PyBytes_FromStringAndSize
_new_bytes.restype = ctypes.py_object
_new_bytes.argtypes = [ctypes.c_void_p, ctypes.c_ssize_t]
_bytes_data = ctypes.pythonapi.PyBytes_AsString
_bytes_data.restype = ctypes.c_void_p
_bytes_data.argtypes = [ctypes.py_object]


def _output_bytes(nbytes: int):
    """A new, not yet shared bytes object of nbytes (> 0) bytes, left
    uninitialised, and the address of its contents: the runtime writes the
    result there, as a C extension fills a bytes object before returning it
    (no zero fill and no copy of the result into a second object)."""
    out = _new_bytes(None, nbytes)
    return out, _bytes_data(out)


_INJECTED = "__test_failure_inject__"
_REFERENCE_MODULES = ("mlir_edsl._mlir_backend_ref", "_mlir_backend_ref")
_UNSET = object()
_reference_override = _UNSET


def set_reference_backend(module) -> None:
    """Use `module` (an object with an ``MLIRCompiler`` class, or None for
    none) as the reference compiler for MLIRCompiler objects created from
    now on, instead of importing one. Mainly for tests and embedders."""
    global _reference_override
    _reference_override = module


def reference_backend():
    """The reference's own compiled module, or None when it is not importable."""
    if _reference_override is not _UNSET:
        return _reference_override
    names = [os.environ["EDSL_HIP_REFERENCE_BACKEND"]] if os.environ.get("EDSL_HIP_REFERENCE_BACKEND") \
        else list(_REFERENCE_MODULES)
    for name in names:
        try:
            return importlib.import_module(name)
        except ImportError:
            continue
    return None


class MLIRCompiler:
    """Same surface as the reference pybind class ``MLIRCompiler``."""

    def __init__(self):
        self._m = _L().edsl_hip_module_create()
        if not self._m:
            raise MemoryError("edsl_hip_module_create failed")
        ref = reference_backend()
        self._ref = ref.MLIRCompiler() if ref is not None else None
        self._routes: dict[str, str] = {}  # function name -> "hip" | "ref"
        self._target = "cpu"
        self._opt_level = 2
        self._capture = False
        self._snapshots: list[tuple[str, str]] = []
        self._failure = ""
        self._injected = False
        # (function, parameter index) -> the bound object: held so that its
        # address stays its own while the snapshot is matched by address.
        self._bound: dict[tuple[str, int], object] = {}

    def __del__(self):
        m, self._m = getattr(self, "_m", None), None
        if m and _lib is not None:
            _lib.edsl_hip_module_destroy(m)

    @property
    def reference(self):
        """The delegated reference compiler object, or None."""
        return self._ref

    def backend_of(self, name: str) -> str:
        """Where `name` runs: "hip" (the gfx950 kernels) or "reference"."""
        if name not in self._routes:
            raise RuntimeError(f"Function not compiled: {name}")
        return "hip" if self._routes[name] == "hip" else "reference"

    # ---------------------------------------------------------- compilation
    def compile_function(self, function_def_bytes: bytes) -> None:
        """Compile function from protobuf FunctionDef bytes."""
        data = bytes(function_def_bytes)
        if self._ref is not None and self._target == "cpu":
            self._compile_on_reference(data)
            return
        if _L().edsl_hip_module_compile_function(self._m, data, len(data)) == 0:
            self._failure = ""
            names = self._hip_names()
            for n in names:
                self._routes.setdefault(n, "hip")
            return
        code, msg = _native.last_error()
        self._failure = _text(_L().edsl_hip_module_last_failure, self._m)
        raise RuntimeError(msg if msg else f"compile_function failed (code {code})")

    def _compile_on_reference(self, data: bytes) -> None:
        before = set(self._ref.list_functions())
        self._ref.set_target(self._target)
        self._ref.compile_function(data)
        self._failure = ""
        for n in set(self._ref.list_functions()) - before:
            self._routes[n] = "ref"

    def _hip_names(self) -> list[str]:
        s = _text(_L().edsl_hip_module_list_functions, self._m)
        return s.split("\n") if s else []

    def _on_reference(self, name: str) -> bool:
        return self._ref is not None and self._routes.get(name) == "ref"

    def _finalize(self) -> None:
        # The reference lowers the whole module on first use, and an injected
        # ill-typed function makes that fail for every function. The HIP
        # module has no lowering pipeline: the injection is recorded and the
        # failure raised here, with the module as it stands.
        if self._injected:
            self._failure = (f"injected test failure: function @{_INJECTED} was added by "
                             f"inject_test_failure() with a result type its body does not return; "
                             f"nothing below was finalized\n" + self.get_module_ir())
            raise RuntimeError(f"Lowering pipeline failed: injected test failure in @{_INJECTED} "
                               "(inject_test_failure)")
        if self._capture:
            runs = [sn for sn in self._snapshots if sn[0].startswith("run:")]
            self._snapshots = [(f"match:{n}", self._match_text(n)) for n in self._hip_names()] + runs

    def _match_text(self, name: str) -> str:
        f = self.function_form(name)
        lines = [f"{name}: {f['form']} ({f['dtype']})"]
        for i, L in enumerate(f["layers"]):
            lines.append(f"layer {i}: x={L['x']} w={L['w']} b={L['b']} epilogue={L['epilogue']} "
                         f"alpha={L['alpha']:g}")
        return "\n".join(lines)

    def get_function_pointer(self, name: str) -> int:
        """Entry point with the reference JIT symbol's calling convention."""
        if self._on_reference(name):
            return self._ref.get_function_pointer(name)
        self._finalize()
        p = _L().edsl_hip_module_get_function_pointer(self._m, name.encode())
        if not p:
            _raise("get_function_pointer")
        return int(p)

    def has_function(self, name: str) -> bool:
        if bool(_L().edsl_hip_module_has_function(self._m, name.encode())):
            return True
        return self._ref is not None and bool(self._ref.has_function(name))

    def list_functions(self) -> list[str]:
        names = set(self._hip_names())
        if self._ref is not None:
            names |= set(self._ref.list_functions())
        return sorted(names)

    def get_module_ir(self) -> str:
        text = _text(_L().edsl_hip_module_describe, self._m)
        if self._ref is not None and self._ref.list_functions():
            text += "// reference compiler module\n" + self._ref.get_module_ir()
        return text

    def clear(self) -> None:
        """Forget every compiled function (and any injected failure)."""
        _L().edsl_hip_module_clear(self._m)
        if self._ref is not None:
            self._ref.clear()
        self._routes.clear()
        self._bound.clear()
        self._failure = ""
        self._injected = False
        self._snapshots = []

    def get_lowering_snapshots(self) -> list[tuple[str, str]]:
        snaps = list(self._snapshots)
        if self._ref is not None:
            snaps += list(self._ref.get_lowering_snapshots())
        return snaps

    def enable_snapshot_capture(self) -> None:
        self._capture = True
        if self._ref is not None:
            self._ref.enable_snapshot_capture()

    def get_failure_ir(self) -> str:
        if self._failure:
            return self._failure
        return self._ref.get_failure_ir() if self._ref is not None else ""

    def inject_test_failure(self) -> None:
        """Testing only: the next finalize fails as with an ill-typed function
        (on the reference compiler when there is one, as there the whole
        module is lowered at once)."""
        if self._ref is not None:
            self._ref.inject_test_failure()
        else:
            self._injected = True

    def set_optimization_level(self, level: int) -> None:
        # The HIP kernels are compiled ahead of time; the level applies to the
        # reference compiler's JIT when there is one.
        self._opt_level = level if level in (0, 2, 3) else 2
        if self._ref is not None:
            self._ref.set_optimization_level(level)

    def set_target(self, target: str) -> None:
        self._target = "gpu" if target == "gpu" else "cpu"
        if self._ref is not None:
            self._ref.set_target(target)

    # ------------------------------------------------------------ execution
    def execute_gpu_function(self, name: str, inputs: Sequence, output_shape: Sequence[int],
                             element_size: int) -> bytes:
        """inputs: list of (data_ptr_int, shape_list); returns the raw output bytes."""
        if self._on_reference(name):
            return self._ref.execute_gpu_function(name, inputs, output_shape, element_size)
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
        nbytes = out_elems * int(element_size)
        if nbytes > 0:
            out, out_ptr = _output_bytes(nbytes)
        else:  # the shared empty bytes object is never written
            out, out_ptr = b"", ctypes.cast(ctypes.create_string_buffer(1), ctypes.c_void_p)
        oshape = (ctypes.c_int64 * len(output_shape))(*[int(d) for d in output_shape])
        rc = _L().edsl_hip_module_execute_gpu_function(
            self._m, name.encode(), n, ptrs, shapes, ranks, out_ptr, oshape, len(output_shape),
            int(element_size))
        if rc != 0:
            _raise("execute_gpu_function")
        if self._capture:  # the kernels of the latest run of each function
            run = (f"run:{name}", _native.last_plan())
            self._snapshots = [sn for sn in self._snapshots if sn[0] != run[0]] + [run]
        return out

    # ----------------------------------------------------------- extension
    def _param_index(self, name: str, param) -> int:
        if isinstance(param, str):
            idx = ctypes.c_int(-1)
            if _L().edsl_hip_module_param_index(self._m, name.encode(), param.encode(), ctypes.byref(idx)) != 0:
                _raise("param_index")
            return idx.value
        return int(param)

    def bind_parameter(self, name: str, param, array) -> None:
        """Keep a device-resident snapshot of `array` as parameter `param`
        (its name, or its position in the function's signature) of the
        HIP-compiled function `name`.

        Calls of the function that pass this same array (same address, shape
        and contiguous rows) then read the snapshot in HBM instead of copying
        the operand in; any other array is copied in as usual. The snapshot
        is taken now: writes to `array` after this call are not seen until
        it is bound again. `array` must be C-contiguous with the parameter's
        compiled shape and element type (float32 or int32) -- a numpy array,
        or anything exposing ``__array_interface__`` or a GPU torch tensor.
        This object keeps a reference to `array` until the parameter is
        unbound or rebound or the module is cleared, so no other array can be
        given its address (and be mistaken for it) in the meantime."""
        if self._on_reference(name):
            raise RuntimeError(f"function '{name}' runs on the reference compiler: only HIP-compiled "
                               "functions have device-resident parameters")
        idx = self._param_index(name, param)
        if hasattr(array, "data_ptr") and hasattr(array, "is_contiguous"):  # torch tensor
            if not array.is_contiguous():
                raise ValueError("bind_parameter needs a contiguous tensor")
            ptr, shape = array.data_ptr(), list(array.shape)
            itemsize = array.element_size()
        else:
            import numpy as np
            a = np.asarray(array)
            if not a.flags["C_CONTIGUOUS"]:
                raise ValueError("bind_parameter needs a C-contiguous array (calls must pass the same "
                                 "array for the snapshot to be used)")
            ptr, shape, itemsize = a.ctypes.data, list(a.shape), a.itemsize
            array = (array, a)  # `a` may be a view np.asarray made of `array`
        if itemsize != 4:
            raise TypeError(f"element size {itemsize}: the dense path binds f32 and i32 parameters")
        dims = (ctypes.c_int64 * max(1, len(shape)))(*shape)
        if _L().edsl_hip_module_bind_parameter(self._m, name.encode(), idx, ptr, dims, len(shape)) != 0:
            _raise("bind_parameter")
        self._bound[(name, idx)] = array

    def unbind_parameter(self, name: str, param=None) -> None:
        """Release the snapshot of `param` (name or position), or of every
        parameter of `name` when `param` is None."""
        idx = -1 if param is None else self._param_index(name, param)
        if _L().edsl_hip_module_unbind_parameter(self._m, name.encode(), idx) != 0:
            _raise("unbind_parameter")
        for key in [k for k in self._bound if k[0] == name and idx in (-1, k[1])]:
            del self._bound[key]

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
