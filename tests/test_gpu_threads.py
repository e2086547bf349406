"""Several Python threads calling the library at once. ctypes releases the
GIL for the call, so the runtime sees truly concurrent callers: host-buffer
calls (memref ABI and the pybind-style entry) serialise on the runtime's lock
and share the staging buffers and the pinned ring; device launches come from
each thread's own stream and share the workspaces. Every result is checked
against the oracle, and each thread's last-plan and last-error state must be
its own: every iteration also makes a failing C-ABI call."""
from __future__ import annotations

import threading
import time

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
    is enqueued, never for a host call's copies, so launches start and return
    inside a host call. Checked by order, not by duration: the host thread
    bumps a counter as each call starts and again as it returns, and a launch
    counts when the counter reads the same odd value before and after it. Had
    the host path held the launch lock for its whole call, a launch started
    during a call could only return after the call ended."""
    import torch
    rng = np.random.default_rng(7)
    M = K = N = 4096
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / 64).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, N).astype(np.float32)
    backend.run("dense_relu", X, W, b)  # sizes the staging buffers
    calls = [0]  # odd while a host call is in progress
    errors = []
    stop = threading.Event()

    def host_calls():
        try:
            for _ in range(8):
                calls[0] += 1
                backend.run("dense_relu", X, W, b)
                calls[0] += 1
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
    inside, total = {}, 0
    t = threading.Thread(target=host_calls)
    t.start()
    while not stop.is_set():
        c0 = calls[0]
        dense_launch(x, w, None, y, _native.EPI_NONE, stream=s)
        if calls[0] == c0 and c0 % 2 == 1:
            inside[c0] = inside.get(c0, 0) + 1
        total += 1
        time.sleep(0.0002)
    t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    # Launches completed inside at least half of the eight host calls.
    assert len(inside) >= 4, (inside, total)
