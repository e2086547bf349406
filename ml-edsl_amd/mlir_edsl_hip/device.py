"""Device-resident, asynchronous launches on torch GPU tensors.

Thin wrappers over ``edsl_hip_dense_{f32,i32}_launch`` (include/edsl_hip_device.h):
operands stay in HBM and the kernels are enqueued on a torch stream (the
current one by default), so torch stream events time exactly the launched
kernels. torch provides memory and streams only; the arithmetic is the HIP
library's.
"""
from __future__ import annotations

from . import _native

_launch = None  # METH_FASTCALL binding of the two entries (csrc/pylaunch.c), once loaded
_torch = None
_raw_stream = None  # (current device index) -> raw hipStream_t of that device's current stream


def _torch_module():
    """torch, imported on first use, and the fastest way it offers to read the
    current stream's raw handle: torch.cuda.current_stream() builds a Python
    stream object (~2.6 us per call on the GPU host), the raw accessor returns
    the same integer in ~0.1 us."""
    global _torch, _raw_stream, _launch
    if _torch is None:
        import torch
        # The binding links the library: load it through _native first, which
        # maps the HIP runtime both share. Not built: ctypes calls the entries.
        _native.lib()
        try:
            from . import _launch as fast
            _launch = fast
        except ImportError:
            _launch = None
        get_dev = getattr(torch._C, "_cuda_getDevice", None)
        get_raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
        if get_dev is not None and get_raw is not None:
            _raw_stream = lambda: get_raw(get_dev())
        else:
            _raw_stream = lambda: torch.cuda.current_stream().cuda_stream
        _torch = torch
    return _torch


def _check_operand(t, name, dtype):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if t.dim() >= 1 and t.shape[-1] > 1 and t.stride(-1) != 1:
        raise ValueError(f"{name} must have unit inner stride")


def _validate(X, W, b, Y, torch) -> None:
    """Every operand check of dense_launch, raising with a message that names
    the operand (run only when the combined check there fails)."""
    dtype = X.dtype
    if dtype not in (torch.float32, torch.int32):
        raise TypeError(f"unsupported dtype {dtype}")
    for t, n in ((X, "X"), (W, "W"), (Y, "Y")):
        _check_operand(t, n, dtype)
    if b is not None:
        _check_operand(b, "b", dtype)
    if X.dim() != 2 or W.dim() != 2:
        raise ValueError(f"X and W must be 2-D, got X{tuple(X.shape)} W{tuple(W.shape)}")
    M, K = X.shape
    K2, N = W.shape
    if K2 != K or tuple(Y.shape) != (M, N):
        raise ValueError(f"shape mismatch: X{tuple(X.shape)} W{tuple(W.shape)} Y{tuple(Y.shape)}")
    if b is not None and tuple(b.shape) != (N,):
        raise ValueError(f"bias shape {tuple(b.shape)} != ({N},)")


def dense_launch(X, W, b, Y, epilogue: int, alpha: float = 0.0, stream=None) -> None:
    """Y = epilogue(X @ W (+ b)); returns once the kernels are enqueued."""
    torch = _torch if _torch is not None else _torch_module()
    dtype = X.dtype
    xs, ws = X.shape, W.shape
    # Everything _validate checks, as one short-circuit test of cheap tensor
    # attributes (per-operand checks cost ~2 us a call, as much as a launch
    # of a small layer); _validate runs only to name what is wrong.
    ok = ((dtype is torch.float32 or dtype is torch.int32)
          and len(xs) == 2 and len(ws) == 2 and xs[1] == ws[0] and Y.shape == (xs[0], ws[1])
          and X.is_cuda and W.is_cuda and Y.is_cuda and W.dtype is dtype and Y.dtype is dtype
          and (xs[1] <= 1 or X.stride(1) == 1)
          and (ws[1] <= 1 or (W.stride(1) == 1 and Y.stride(1) == 1)))
    if ok and b is not None:
        ok = (b.is_cuda and b.dtype is dtype and b.shape == (ws[1],)
              and (ws[1] <= 1 or b.stride(0) == 1))
    if not ok:
        _validate(X, W, b, Y, torch)
    M, K = xs
    N = ws[1]
    sp = stream.cuda_stream if stream is not None else _raw_stream()
    bp = b.data_ptr() if b is not None else None
    if _launch is not None:
        if dtype is torch.float32:
            rc = _launch.dense_f32(X.data_ptr(), X.stride(0), W.data_ptr(), W.stride(0), bp,
                                   Y.data_ptr(), Y.stride(0), M, N, K, epilogue, alpha, sp)
        else:
            rc = _launch.dense_i32(X.data_ptr(), X.stride(0), W.data_ptr(), W.stride(0), bp,
                                   Y.data_ptr(), Y.stride(0), M, N, K, epilogue, sp)
        if rc != 0:
            _native.raise_on_error("dense_launch")
        return
    L = _native.lib()
    if dtype is torch.float32:
        rc = L.edsl_hip_dense_f32_launch(X.data_ptr(), X.stride(0), W.data_ptr(), W.stride(0), bp,
                                         Y.data_ptr(), Y.stride(0), M, N, K, epilogue, alpha, sp)
    else:
        rc = L.edsl_hip_dense_i32_launch(X.data_ptr(), X.stride(0), W.data_ptr(), W.stride(0), bp,
                                         Y.data_ptr(), Y.stride(0), M, N, K, epilogue, sp)
    if rc != 0:
        _native.raise_on_error("dense_launch")


def set_f32_config(cfg: int) -> None:
    _native.lib().edsl_hip_set_f32_config(cfg)


def set_gemv_ksplit(ksplit: int) -> None:
    _native.lib().edsl_hip_set_gemv_ksplit(ksplit)


def set_gemv_cols(cols: int) -> None:
    _native.lib().edsl_hip_set_gemv_cols(cols)


def set_small_m(mode: int) -> None:
    """0: automatic; 1: the small-M kernel whenever it can plan the layer."""
    _native.lib().edsl_hip_set_small_m(mode)


def set_i8_variant(variant: int) -> None:
    _native.lib().edsl_hip_set_i8_variant(variant)
