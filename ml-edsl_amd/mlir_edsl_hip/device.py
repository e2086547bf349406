"""Device-resident, asynchronous launches on torch GPU tensors.

Thin wrappers over ``edsl_hip_dense_{f32,i32}_launch`` (include/edsl_hip_device.h):
operands stay in HBM and the kernels are enqueued on a torch stream (the
current one by default), so torch stream events time exactly the launched
kernels. torch provides memory and streams only; the arithmetic is the HIP
library's.
"""
from __future__ import annotations

from . import _native


def _check_operand(t, name, dtype):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if t.dim() >= 1 and t.shape[-1] > 1 and t.stride(-1) != 1:
        raise ValueError(f"{name} must have unit inner stride")


def dense_launch(X, W, b, Y, epilogue: int, alpha: float = 0.0, stream=None) -> None:
    """Y = epilogue(X @ W (+ b)); returns once the kernels are enqueued."""
    import torch
    dtype = X.dtype
    if dtype not in (torch.float32, torch.int32):
        raise TypeError(f"unsupported dtype {dtype}")
    for t, n in ((X, "X"), (W, "W"), (Y, "Y")):
        _check_operand(t, n, dtype)
    if b is not None:
        _check_operand(b, "b", dtype)
    M, K = X.shape
    K2, N = W.shape
    if K2 != K or tuple(Y.shape) != (M, N):
        raise ValueError(f"shape mismatch: X{tuple(X.shape)} W{tuple(W.shape)} Y{tuple(Y.shape)}")
    if b is not None and tuple(b.shape) != (N,):
        raise ValueError(f"bias shape {tuple(b.shape)} != ({N},)")
    s = stream if stream is not None else torch.cuda.current_stream()
    L = _native.lib()
    bp = b.data_ptr() if b is not None else None
    if dtype == torch.float32:
        rc = L.edsl_hip_dense_f32_launch(X.data_ptr(), X.stride(0), W.data_ptr(), W.stride(0), bp,
                                         Y.data_ptr(), Y.stride(0), M, N, K, epilogue, alpha,
                                         s.cuda_stream)
    else:
        rc = L.edsl_hip_dense_i32_launch(X.data_ptr(), X.stride(0), W.data_ptr(), W.stride(0), bp,
                                         Y.data_ptr(), Y.stride(0), M, N, K, epilogue, s.cuda_stream)
    if rc != 0:
        _native.raise_on_error("dense_launch")


def set_f32_config(cfg: int) -> None:
    _native.lib().edsl_hip_set_f32_config(cfg)


def set_gemv_ksplit(ksplit: int) -> None:
    _native.lib().edsl_hip_set_gemv_ksplit(ksplit)


def set_gemv_cols(cols: int) -> None:
    _native.lib().edsl_hip_set_gemv_cols(cols)


def set_i8_variant(variant: int) -> None:
    _native.lib().edsl_hip_set_i8_variant(variant)
