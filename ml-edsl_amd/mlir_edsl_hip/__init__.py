"""mlir_edsl_hip -- MI355X (gfx950) runtime for ml-edsl's dense hot path.

linalg.matmul and the dense layer relu(X @ W + b) as hand-written HIP kernels
behind the memref-descriptor C ABI of include/edsl_hip.h. This package is the
host side: the ctypes binding, a facade with the reference backend's calling
sequence, device-resident launches, and the seeded workload inputs.
"""
from ._native import LIB_PATH, NativeLibraryError, last_plan, lib  # noqa: F401
from .backend import (HipBackend, TensorType, dense, f32, get_backend, i32,  # noqa: F401
                      matmul, run)
from .inputs import WORKLOADS, Workload, make_inputs  # noqa: F401

__all__ = ["LIB_PATH", "NativeLibraryError", "HipBackend", "TensorType", "dense", "f32",
           "get_backend", "i32", "lib", "last_plan", "matmul", "run", "WORKLOADS", "Workload",
           "make_inputs"]
