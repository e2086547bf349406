"""ctypes loader for libedsl_hip.so, the gfx950 dense-path runtime.

There is no fallback: if the library is missing or cannot be loaded the
import of the ops that need it fails with :class:`NativeLibraryError`.
"""
from __future__ import annotations

import ctypes
import importlib.util
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libedsl_hip.so")

EPI_NONE, EPI_BIAS, EPI_RELU, EPI_BIAS_RELU, EPI_LEAKY, EPI_BIAS_LEAKY, EPI_IF_RELU, EPI_BIAS_IF_RELU = range(8)
(PATTERN_MATMUL, PATTERN_MATMUL_BIAS, PATTERN_DENSE_RELU, PATTERN_DENSE_LEAKY, PATTERN_MATMUL_RELU,
 PATTERN_DENSE_IF_RELU, PATTERN_MATMUL_IF_RELU) = range(7)
DTYPE_F32, DTYPE_I32 = 0, 1
NOALLOC_SCRATCH_BYTES = 16 << 20  # EDSL_NOALLOC_SCRATCH_BYTES (include/edsl_hip_device.h)

# Flat scalar run of one expanded memref argument (MLIR func-to-llvm):
# allocated ptr, aligned ptr, offset, sizes[r], strides[r].
MEMREF2 = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 5
MEMREF1 = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 3

# name -> argtypes of the memref-ABI entry points (include/edsl_hip.h)
MEMREF_ENTRY_POINTS = {
    "edsl_hip_matmul_f32": MEMREF2 * 3,
    "edsl_hip_matmul_i32": MEMREF2 * 3,
    "edsl_hip_matmul_relu_f32": MEMREF2 * 3,
    "edsl_hip_matmul_relu_i32": MEMREF2 * 3,
    "edsl_hip_matmul_bias_f32": MEMREF2 * 2 + MEMREF1 + MEMREF2,
    "edsl_hip_matmul_bias_i32": MEMREF2 * 2 + MEMREF1 + MEMREF2,
    "edsl_hip_dense_relu_f32": MEMREF2 * 2 + MEMREF1 + MEMREF2,
    "edsl_hip_dense_relu_i32": MEMREF2 * 2 + MEMREF1 + MEMREF2,
    "edsl_hip_dense_leaky_relu_f32": MEMREF2 * 2 + MEMREF1 + MEMREF2 + [ctypes.c_float],
    "edsl_hip_dense_if_relu_f32": MEMREF2 * 2 + MEMREF1 + MEMREF2,
    "edsl_hip_matmul_if_relu_f32": MEMREF2 * 3,
}


class NativeLibraryError(ImportError):
    pass


_lib = None


def _declare(L: ctypes.CDLL) -> None:
    i64, vp, c_int, c_float = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    for name, argtypes in MEMREF_ENTRY_POINTS.items():
        fn = getattr(L, name)
        fn.argtypes = argtypes
        fn.restype = None
    L.edsl_hip_execute_gpu_function.argtypes = [
        c_int, c_int, c_int, ctypes.POINTER(vp), ctypes.POINTER(ctypes.POINTER(i64)),
        ctypes.POINTER(c_int), vp, ctypes.POINTER(i64), c_int, ctypes.c_size_t, c_float]
    L.edsl_hip_execute_gpu_function.restype = c_int
    L.edsl_hip_last_error.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    L.edsl_hip_last_error.restype = c_int
    L.edsl_hip_clear_error.argtypes = []
    L.edsl_hip_clear_error.restype = None
    L.edsl_hip_dense_f32_launch.argtypes = [vp, i64, vp, i64, vp, vp, i64, i64, i64, i64, c_int,
                                            c_float, vp]
    L.edsl_hip_dense_f32_launch.restype = c_int
    L.edsl_hip_dense_f32_launch_noalloc.argtypes = L.edsl_hip_dense_f32_launch.argtypes
    L.edsl_hip_dense_f32_launch_noalloc.restype = c_int
    L.edsl_hip_dense_f32_launch_unfused.argtypes = L.edsl_hip_dense_f32_launch.argtypes
    L.edsl_hip_dense_f32_launch_unfused.restype = c_int
    L.edsl_hip_dense_i32_launch.argtypes = [vp, i64, vp, i64, vp, vp, i64, i64, i64, i64, c_int, vp]
    L.edsl_hip_dense_i32_launch.restype = c_int
    L.edsl_hip_last_plan.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    L.edsl_hip_last_plan.restype = c_int
    L.edsl_hip_set_f32_config.argtypes = [c_int]
    L.edsl_hip_set_f32_config.restype = None
    L.edsl_hip_set_gemv_ksplit.argtypes = [c_int]
    L.edsl_hip_set_gemv_ksplit.restype = None
    L.edsl_hip_set_gemv_cols.argtypes = [c_int]
    L.edsl_hip_set_gemv_cols.restype = None
    L.edsl_hip_set_small_m.argtypes = [c_int]
    L.edsl_hip_set_small_m.restype = None
    L.edsl_hip_set_i8_variant.argtypes = [c_int]
    L.edsl_hip_set_i8_variant.restype = None
    L.edsl_hip_i8_variant_count.argtypes = []
    L.edsl_hip_i8_variant_count.restype = c_int
    L.edsl_hip_f32_config_count.argtypes = []
    L.edsl_hip_f32_config_count.restype = c_int
    L.edsl_hip_f32_config_name.argtypes = [c_int, ctypes.c_char_p, ctypes.c_size_t]
    L.edsl_hip_f32_config_name.restype = c_int


def _share_torch_hip_runtime() -> None:
    """Map torch's own HIP runtime, when torch is installed, before the
    library. torch ships a libamdhip64 with the same SONAME as the system one
    the library is linked against, but asks for it under another file name:
    had the library come first, importing torch later would map a second HIP
    runtime, and two in one process fail to find the device. Mapped first
    (by path, without importing torch), it serves both: the library's
    dependency matches its SONAME and torch's its file."""
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.origin:
        return
    runtime = os.path.join(os.path.dirname(spec.origin), "lib", "libamdhip64.so")
    if os.path.exists(runtime):
        try:
            ctypes.CDLL(runtime)
        except OSError:  # unusable: the library brings the system runtime
            pass


def lib() -> ctypes.CDLL:
    """The loaded runtime library (loaded once per process)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() (or "
                "python -m mlir_edsl_hip.build) first")
        _share_torch_hip_runtime()
        try:
            L = ctypes.CDLL(LIB_PATH)
        except OSError as e:
            raise NativeLibraryError(f"cannot load {LIB_PATH}: {e}") from e
        _declare(L)
        _lib = L
    return _lib


def last_error() -> tuple[int, str]:
    buf = ctypes.create_string_buffer(1024)
    code = lib().edsl_hip_last_error(buf, len(buf))
    return code, buf.value.decode(errors="replace")


def raise_on_error(what: str) -> None:
    code, msg = last_error()
    if code != 0:
        raise RuntimeError(f"{what}: {msg} (code {code})")


def last_plan() -> str:
    buf = ctypes.create_string_buffer(256)
    lib().edsl_hip_last_plan(buf, len(buf))
    return buf.value.decode()


def f32_config_names() -> list[str]:
    L = lib()
    out = []
    for i in range(L.edsl_hip_f32_config_count()):
        buf = ctypes.create_string_buffer(128)
        L.edsl_hip_f32_config_name(i, buf, len(buf))
        out.append(buf.value.decode())
    return out
