"""Several Python threads calling the library at once. ctypes releases the
GIL for the call, so the runtime sees truly concurrent callers: host-buffer
calls (memref ABI and the pybind-style entry) serialise on the runtime's lock
and share the staging buffers and the pinned ring; device launches come from
each thread's own stream and share the workspaces. Every result is checked
against the oracle, and each thread's last-plan and last-error state must be
its own: every iteration also makes a failing C-ABI call."""
from __future__ import annotations

import threading

import numpy as np
import pytest

import oracle
from conftest import assert_f32_parity
from mlir_edsl_hip import _native, backend
from mlir_edsl_hip.device import dense_launch

pytestmark = pytest.mark.gpu

SHAPES = [(64, 96, 128), (16, 2048, 1024), (256, 256, 384), (1500, 640, 1200), (33, 70, 45)]


def _worker(tid, iters, errors):
    import torch
    rng = np.random.default_rng(100 + tid)
    stream = torch.cuda.Stream()
    try:
        for it in range(iters):
            M, K, N = SHAPES[(tid + it) % len(SHAPES)]
            dtype = "i32" if (tid + it) % 3 == 0 else "f32"
            if dtype == "f32":
                X = rng.standard_normal((M, K), dtype=np.float32)
                W = rng.standard_normal((K, N), dtype=np.float32)
                b = rng.standard_normal(N, dtype=np.float32)
                ref = oracle.dense_f32_chains(X, W, b, "relu")
            else:
                X = rng.integers(-128, 128, size=(M, K), dtype=np.int32)
                W = rng.integers(-128, 128, size=(K, N), dtype=np.int32)
                b = rng.integers(-512, 512, size=N, dtype=np.int32)
                ref = oracle.dense_i32(X, W, b, "relu")
            mode = (tid + 2 * it) % 3
            if mode == 0:  # host buffers through the memref ABI
                got = backend.run("dense_relu", X, W, b)
                plan = _native.last_plan()
            elif mode == 1:  # host buffers through the pybind-style entry
                be = backend.get_backend()
                name = f"thr_{tid}_{it}"
                be.compile_dense(name, "dense_relu", [backend.tensor_type_of(a) for a in (X, W, b)])
                got = be.execute_gpu_function(name, X, W, b)
                plan = _native.last_plan()
            else:  # device launch on this thread's stream
                with torch.cuda.stream(stream):
                    tX, tW, tb = (torch.from_numpy(a).cuda() for a in (X, W, b))
                    tY = torch.empty((M, N), dtype=tX.dtype, device="cuda")
                    dense_launch(tX, tW, tb, tY, _native.EPI_BIAS_RELU, stream=stream)
                    plan = _native.last_plan()
                stream.synchronize()
                got = tY.cpu().numpy()
            what = f"thread {tid} iter {it} mode {mode} {dtype} {M}x{K}x{N} [{plan}]"
            if dtype == "i32":
                assert np.array_equal(got, ref), what
            else:
                try:
                    assert_f32_parity(got, ref, K)
                except AssertionError as e:
                    raise AssertionError(f"{what}: {e}") from None
            # this thread's plan matches what it ran (the plan string is thread-local)
            assert plan and plan != "empty", what
            # a failing C-ABI call: its error stays in this thread (the others
            # check their own error state after every call and would fail)
            L = _native.lib()
            rc = L.edsl_hip_dense_f32_launch(None, 2, None, 8, None, None, 8, 4, 8, 8, 0, 0.0, None)
            assert rc != 0
            assert "null operand" in _native.last_error()[1], what
            L.edsl_hip_clear_error()
        # the facade's type rules raise TypeError, as the reference's do
        with pytest.raises(TypeError, match="inner dimensions"):
            backend.run("dense_relu", np.ones((4, 5), np.float32), np.ones((6, 3), np.float32),
                        np.ones(3, np.float32))
    except BaseException as e:  # noqa: BLE001 - reported by the main thread
        errors.append(e)


def test_concurrent_callers():
    import torch
    assert torch.cuda.is_available()
    errors: list = []
    threads = [threading.Thread(target=_worker, args=(t, 9, errors)) for t in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a caller thread did not finish"
    if errors:
        raise errors[0]


def test_device_launches_do_not_wait_for_host_copies():
    """One thread makes host-buffer calls of the c3 size (copies of 128 MiB
    in and 64 MiB out, ~5 ms each); another enqueues small device launches
    on its own stream meanwhile. The launch lock is held only while a launch
    is enqueued, so no enqueue waits for a host call's copies: the slowest
    one stays far below a host call's duration."""
    import time

    import torch
    rng = np.random.default_rng(7)
    M = K = N = 4096
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / 64).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, N).astype(np.float32)
    backend.run("dense_relu", X, W, b)  # sizes the staging buffers
    host_times, enqueue_times, errors = [], [], []
    stop = threading.Event()

    def host_calls():
        try:
            for _ in range(8):
                t0 = time.perf_counter()
                backend.run("dense_relu", X, W, b)
                host_times.append(time.perf_counter() - t0)
        except Exception as e:  # noqa: BLE001 -- reported below
            errors.append(repr(e))
        finally:
            stop.set()

    s = torch.cuda.Stream()
    x = torch.randn(16, 512, device="cuda")
    w = torch.randn(512, 256, device="cuda")
    y = torch.empty(16, 256, device="cuda")
    dense_launch(x, w, None, y, _native.EPI_NONE, stream=s)  # warm: plan, workspace
    torch.cuda.synchronize()
    t = threading.Thread(target=host_calls)
    t.start()
    while not stop.is_set():
        t0 = time.perf_counter()
        dense_launch(x, w, None, y, _native.EPI_NONE, stream=s)
        enqueue_times.append(time.perf_counter() - t0)
        time.sleep(0.0002)
    t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    slow_host = min(host_times)
    enqueue_times.sort()
    p99 = enqueue_times[int(0.99 * (len(enqueue_times) - 1))]
    assert len(enqueue_times) > 20, len(enqueue_times)
    assert p99 < 0.25 * slow_host, (p99, slow_host, enqueue_times[-5:])
