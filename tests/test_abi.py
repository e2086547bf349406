"""The C-ABI library: loads, exports every declared symbol, validates
descriptors on the host (no device call is made for a malformed call)."""
from __future__ import annotations

import ctypes
import glob
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from mlir_edsl_hip import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_functions():
    names = []
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:void|int|edsl_hip_module)\s*\**\s*(edsl_hip_\w+)\s*\(", text,
                            flags=re.M)
    return names


def test_headers_declare_the_boundary():
    names = declared_functions()
    for n in _native.MEMREF_ENTRY_POINTS:
        assert n in names
    assert "edsl_hip_execute_gpu_function" in names
    assert "edsl_hip_last_error" in names
    for n in ("edsl_hip_module_create", "edsl_hip_module_get_function_pointer",
              "edsl_hip_module_compile_function", "edsl_hip_module_execute_gpu_function"):
        assert n in names
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol():
    L = _native.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert missing == []


@pytest.mark.parametrize("lang,compiler", [("c", "gcc"), ("c++", "g++")])
def test_headers_compile_standalone(tmp_path, lang, compiler):
    src = tmp_path / ("t.c" if lang == "c" else "t.cpp")
    src.write_text("".join(f'#include "{h}"\n' for h in HEADERS) + "int main(void){return 0;}\n")
    subprocess.run([compiler, "-Wall", "-Werror", "-fsyntax-only", str(src)], check=True)


def _d2(a, dims=None, strides=None, offset=0):
    """Flat memref descriptor values for a 2-D numpy array."""
    dims = list(a.shape) if dims is None else dims
    strides = [s // a.itemsize for s in a.strides] if strides is None else strides
    return [a.ctypes.data, a.ctypes.data, offset] + dims + strides


def _d1(a):
    return [a.ctypes.data, a.ctypes.data, 0, a.shape[0], 1]


def _err():
    return _native.last_error()


def test_inner_dimension_mismatch_is_rejected_before_launch():
    L = _native.lib()
    A = np.zeros((4, 3), np.float32)
    B = np.zeros((5, 2), np.float32)
    C = np.zeros((4, 2), np.float32)
    L.edsl_hip_matmul_f32(*_d2(A), *_d2(B), *_d2(C))
    code, msg = _err()
    assert code == -1 and "inner dimensions must match" in msg


def test_output_shape_mismatch():
    L = _native.lib()
    A = np.zeros((4, 3), np.float32)
    B = np.zeros((3, 2), np.float32)
    C = np.zeros((4, 3), np.float32)
    L.edsl_hip_matmul_f32(*_d2(A), *_d2(B), *_d2(C))
    code, msg = _err()
    assert code == -1 and "output shape" in msg


def test_non_unit_inner_stride_rejected():
    L = _native.lib()
    A = np.zeros((4, 6), np.float32)
    B = np.zeros((3, 2), np.float32)
    C = np.zeros((4, 2), np.float32)
    L.edsl_hip_matmul_f32(*_d2(A, dims=[4, 3], strides=[6, 2]), *_d2(B), *_d2(C))
    code, msg = _err()
    assert code == -2 and "innermost stride" in msg


def test_row_stride_shorter_than_row_rejected():
    L = _native.lib()
    A = np.zeros((4, 3), np.float32)
    B = np.zeros((3, 2), np.float32)
    C = np.zeros((4, 2), np.float32)
    L.edsl_hip_matmul_f32(*_d2(A, strides=[2, 1]), *_d2(B), *_d2(C))
    code, msg = _err()
    assert code == -2 and "row stride" in msg


def test_negative_size_rejected():
    L = _native.lib()
    A = np.zeros((4, 3), np.float32)
    B = np.zeros((3, 2), np.float32)
    C = np.zeros((4, 2), np.float32)
    L.edsl_hip_matmul_f32(*_d2(A, dims=[-4, 3]), *_d2(B), *_d2(C))
    code, _ = _err()
    assert code == -1


def test_bias_length_mismatch():
    L = _native.lib()
    X = np.zeros((4, 3), np.float32)
    W = np.zeros((3, 2), np.float32)
    b = np.zeros(3, np.float32)
    Y = np.zeros((4, 2), np.float32)
    L.edsl_hip_dense_relu_f32(*_d2(X), *_d2(W), *_d1(b), *_d2(Y))
    code, msg = _err()
    assert code == -1 and "bias length" in msg


def test_bias_stride_rejected():
    L = _native.lib()
    X = np.zeros((4, 3), np.float32)
    W = np.zeros((3, 2), np.float32)
    b = np.zeros(4, np.float32)
    Y = np.zeros((4, 2), np.float32)
    L.edsl_hip_matmul_bias_i32(*_d2(X.astype(np.int32)), *_d2(W.astype(np.int32)),
                               b.ctypes.data, b.ctypes.data, 0, 2, 2, *_d2(Y.astype(np.int32)))
    code, msg = _err()
    assert code == -2 and "stride" in msg


def test_null_pointer_rejected():
    L = _native.lib()
    B = np.zeros((3, 2), np.float32)
    C = np.zeros((4, 2), np.float32)
    L.edsl_hip_matmul_f32(None, None, 0, 4, 3, 3, 1, *_d2(B), *_d2(C))
    code, msg = _err()
    assert code == -4 and "null" in msg


def test_error_is_cleared_by_next_validation_pass():
    L = _native.lib()
    A = np.zeros((4, 3), np.float32)
    B = np.zeros((5, 2), np.float32)
    C = np.zeros((4, 2), np.float32)
    L.edsl_hip_matmul_f32(*_d2(A), *_d2(B), *_d2(C))
    assert _err()[0] != 0
    L.edsl_hip_clear_error()
    assert _err() == (0, "")


def test_execute_gpu_function_argument_checks():
    L = _native.lib()
    X = np.zeros((2, 2), np.float32)
    ptrs = (ctypes.c_void_p * 2)(X.ctypes.data, X.ctypes.data)
    s = (ctypes.c_int64 * 2)(2, 2)
    shapes = (ctypes.POINTER(ctypes.c_int64) * 2)(s, s)
    ranks = (ctypes.c_int * 2)(2, 2)
    out = np.zeros((2, 2), np.float32)
    oshape = (ctypes.c_int64 * 2)(2, 2)
    rc = L.edsl_hip_execute_gpu_function(0, 0, 2, ptrs, shapes, ranks, out.ctypes.data, oshape, 2, 8, 0.0)
    assert rc == -3 and "element_size" in _err()[1]
    rc = L.edsl_hip_execute_gpu_function(9, 0, 2, ptrs, shapes, ranks, out.ctypes.data, oshape, 2, 4, 0.0)
    assert rc == -4 and "pattern" in _err()[1]
    rc = L.edsl_hip_execute_gpu_function(2, 0, 2, ptrs, shapes, ranks, out.ctypes.data, oshape, 2, 4, 0.0)
    assert rc == -4 and "takes 3 inputs" in _err()[1]


def test_device_launch_requires_bias_when_epilogue_adds_one():
    L = _native.lib()
    rc = L.edsl_hip_dense_f32_launch(None, 4, None, 4, None, None, 4, 4, 4, 4, 3, 0.0, None)
    assert rc == -4 and "bias" in _err()[1]


def test_config_table_is_exposed():
    names = _native.f32_config_names()
    assert len(names) >= 5 and all(n.startswith("f32_") for n in names)
    assert any("guard" in n for n in names)


def test_fastcall_launch_module_reaches_the_same_library():
    """The METH_FASTCALL binding (csrc/pylaunch.c) is built beside the
    library, maps the same library instance that ctypes loads (one set of
    runtime state, one last-error slot), and reports the entries' status
    codes; argument errors are Python errors. No call here reaches a kernel."""
    from mlir_edsl_hip import device
    L = _native.lib()
    device._torch_module()  # loads the binding after the library
    assert device._launch is not None, "the launch module is not built"
    maps = {line.split()[-1] for line in open("/proc/self/maps") if "libedsl_hip" in line}
    assert len(maps) == 1, maps
    # bias epilogue with a null bias: rejected by the library before any device call
    rc = device._launch.dense_f32(0, 4, 0, 4, None, 0, 4, 4, 4, 4, 1, 0.0, 0)
    assert rc == _native.last_error()[0] != 0
    assert "bias" in _native.last_error()[1]
    rc = device._launch.dense_i32(0, 4, 0, 4, None, 0, 4, 4, 4, 4, 1, 0)
    assert rc != 0 and "bias" in _native.last_error()[1]
    # ldx < K with M > 1: the stride check, through both bindings, same code
    rc_fast = device._launch.dense_f32(8, 2, 8, 4, None, 8, 4, 4, 4, 4, 0, 0.0, 0)
    rc_ctypes = L.edsl_hip_dense_f32_launch(8, 2, 8, 4, None, 8, 4, 4, 4, 4, 0, 0.0, 0)
    assert rc_fast == rc_ctypes != 0
    with pytest.raises(TypeError, match="13 arguments"):
        device._launch.dense_f32(1, 2, 3)
    with pytest.raises(TypeError):
        device._launch.dense_i32(0, "4", 0, 4, None, 0, 4, 4, 4, 4, 1, 0)


@pytest.mark.parametrize("order", ["library_first", "torch_first"])
def test_one_hip_runtime_whichever_loads_first(order):
    """torch carries its own HIP runtime with the system one's SONAME; the
    library must share it in either import order (two runtimes in one process
    cannot both open the device). Run in a fresh process."""
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "if %r == 'torch_first':\n    import torch\n"
        "from mlir_edsl_hip import _native, device\n"
        "_native.lib()\n"
        "import torch\n"
        "device._torch_module()\n"
        "maps = {l.split()[-1] for l in open('/proc/self/maps') if 'libamdhip64' in l}\n"
        "print(len(maps))\n" % (os.path.join(os.path.dirname(os.path.dirname(__file__)), "ml-edsl_amd"), order))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip().splitlines()[-1] == "1", out.stdout
