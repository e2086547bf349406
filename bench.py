#!/usr/bin/env python3
"""Benchmark of the dense hot path on one MI355X.

Headline (BASELINE.json metric): fused fp32 matmul+bias+ReLU at M=N=K=4096
(workload c3), in TFLOP/s and as a fraction of the dense fp32 MFMA peak.
Secondary lines (same run): the M=16, K=N=8192 layer in GB/s (c4, W rotated
over 3 buffers so the 256 MB Infinity Cache cannot serve it), the integer
layer 2048^3 (c5, X and W rotated over 10 buffer pairs; the cache-resident
figure beside it), 1024^3 (c2, fused and the reference's unfused
three-launch sequence), the 256^3 matmul (c1), and one GPU's share of c4 and
c3 column-sharded over 8 GPUs (c4s8: N=1024, W rotated over 12 buffers;
c3s8: N=512).

A step is one call of the dense layer on device-resident inputs (the
C-ABI launch entry point, enqueued on torch's current stream). W warmup
steps, then K timed steps between two device synchronisations (the wall
clock gives `value`; two events on the stream give the same region's device
span, region_ms_per_step). A second pass enqueues K more steps behind a
short spin kernel, so the GPU never waits on the host, between two HIP
events on the same stream: their device time / K is the average launch
duration used for the roofline. A third pass with one event pair per launch
reports the spread.

Every workload's inputs are generated and uploaded before the first
measurement, and the workloads run back to back with the headline last: the
GPU's clock takes ~20 ms of sustained load to ramp up from idle (measured:
the first c3 launches after an idle second take 1140-1220 us, later ones
980 us), so a headline measured first, after a few ms of warmup, would time
the ramp.

Then, on host buffers (never `value`): the reference's GPU calling pattern
(H2D + kernels + D2H per call) for every workload, c4 with its weights bound
device-resident, and the reference's own GPU benchmark points (matmul and
dense at 256, 512, 1024). Last, the CPU baseline: the oracle (a C
restatement of the reference CPU-JIT schedule) on a row sample of each
workload, on this host's cores.

Prints one JSON line on stdout.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "ml-edsl_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "fused matmul+bias+ReLU TFLOP/s & % roofline (4096^3 fp32); GB/s at M=16"
PEAK = {  # MI355X published dense peaks
    "fp32_mfma_tflops": 157.3,
    "int8_mfma_tops": 5000.0,
    "hbm_gbs": 8000.0,
}
KERNEL_NAMES = {"c1": "gemm_f32_direct16_kernel", "c2": "gemm_f32_direct_rc_kernel", "c3": "gemm_f32_direct_kernel",
                "c4": "gemv_f32_kernel + gemv_reduce_kernel", "c5": "narrow_i8_kernel + gemm_i8_ksplit_kernel",
                "c3s8": "gemm_f32_direct64_kernel", "c4s8": "gemv_f32_kernel + gemv_reduce_kernel"}
UNITS = {"c1": "TFLOP/s", "c2": "TFLOP/s", "c3": "TFLOP/s", "c4": "GB/s", "c5": "TOP/s",
         "c3s8": "TFLOP/s", "c4s8": "GB/s"}
# (steps, warmup, input sets rotated) of each workload when it is not the
# headline. The inputs that would otherwise be served from the 256 MB Infinity
# Cache are rotated past it: c4 W 3 x 256 MiB, c4s8 W 12 x 32 MiB, c5 X and W
# 10 x 32 MiB.
SECONDARY_PLAN = {"c4": (200, 20, 3), "c5": (200, 20, 10), "c2": (100, 20, 1), "c1": (200, 20, 1),
                  "c3": (50, 20, 1), "c3s8": (100, 100, 1), "c4s8": (300, 30, 12)}
ROTATE_X = {"c5"}           # workloads whose X is rotated together with W
RESIDENT_TOO = {"c5"}       # also measured without rotation (inputs cache-resident)
UNFUSED_TOO = {"c2", "c3"}  # also timed as the reference's unfused three-launch sequence
LIBRARY_TOO = {"c2", "c3", "c5"}  # the vendor library's GEMM on the same operands, for reference


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


_SLEEP_RATE = None


def sleep_cycles_per_s() -> float:
    """Rate of torch.cuda._sleep's cycle argument on this device (measured once)."""
    global _SLEEP_RATE
    if _SLEEP_RATE is None:
        import torch
        n = 1_000_000
        torch.cuda._sleep(n)  # first call compiles / warms up
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        torch.cuda._sleep(n)
        b.record()
        torch.cuda.synchronize()
        _SLEEP_RATE = n / max(a.elapsed_time(b) * 1e-3, 1e-6)
    return _SLEEP_RATE


class Prepared:
    """A workload's host arrays and their device copies (rotated sets)."""

    def __init__(self, wname: str, rotate: int):
        import torch
        from mlir_edsl_hip.inputs import WORKLOADS, make_inputs
        self.w = WORKLOADS[wname]
        self.name = wname
        self.arrays = make_inputs(self.w)
        dev = [torch.from_numpy(a).cuda() for a in self.arrays]
        self.X, self.W = dev[0], dev[1]
        self.b = dev[2] if len(dev) > 2 else None
        self.rotate = rotate
        self.Ws = [self.W] + [self.W.clone() for _ in range(rotate - 1)]
        self.Xs = [self.X] + ([self.X.clone() for _ in range(rotate - 1)] if wname in ROTATE_X else [])
        dtype = torch.float32 if self.w.dtype == "f32" else torch.int32
        self.Y = torch.empty((self.w.M, self.w.N), dtype=dtype, device="cuda")

    def free(self) -> None:
        import torch
        del self.X, self.W, self.Ws, self.Xs, self.Y, self.b
        torch.cuda.empty_cache()


def measure(p: Prepared, steps: int, warmup: int, rotate: int | None = None, unfused: bool = False) -> dict:
    import torch

    from mlir_edsl_hip import _native
    from mlir_edsl_hip.device import dense_launch

    rotate = p.rotate if rotate is None else rotate
    epi = _native.EPI_BIAS_RELU if p.w.pattern == "dense_relu" else _native.EPI_NONE
    nx = min(rotate, len(p.Xs))
    L = _native.lib()
    M, K, N = p.w.M, p.w.K, p.w.N

    def launch(i: int) -> None:
        if unfused:
            X, W = p.Xs[i % nx], p.Ws[i % rotate]
            rc = L.edsl_hip_dense_f32_launch_unfused(X.data_ptr(), K, W.data_ptr(), N, p.b.data_ptr(),
                                                     p.Y.data_ptr(), N, M, N, K, epi, 0.0,
                                                     torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                _native.raise_on_error("unfused launch")
        else:
            dense_launch(p.Xs[i % nx], p.Ws[i % rotate], p.b, p.Y, epi)

    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    plan = _native.last_plan()
    # Timed region (the contract's): K steps between two synchronisations;
    # the wall clock gives `value`. Two events on the stream record its device
    # span as well (region_ms_per_step).
    region = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    region[0].record()
    for i in range(steps):
        launch(i)
    t_enq = time.perf_counter()
    region[1].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    region_ms = region[0].elapsed_time(region[1]) / steps
    # Device time per launch with the GPU never waiting on the host: a short
    # spin kernel holds the stream while the K launches are enqueued behind
    # it, and the events bracket only the K launches. (When the host issues
    # slower than the GPU runs -- small shapes -- the timed region above is
    # host-bound.)
    enqueue_s = t_enq - t0  # host time to enqueue the K launches
    torch.cuda._sleep(int(sleep_cycles_per_s() * (enqueue_s * 1.5 + 2e-4)))
    backlog = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    backlog[0].record()
    for i in range(steps):
        launch(i)
    backlog[1].record()
    torch.cuda.synchronize()
    device_ms = backlog[0].elapsed_time(backlog[1]) / steps
    # Spread: one event pair around each launch (each pair carries the event
    # latency, so these read high for short launches).
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        starts[i].record()
        launch(i)
        ends[i].record()
    torch.cuda.synchronize()
    kms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return {
        "workload": p.name,
        "ms_per_step": (t1 - t0) * 1e3 / steps,
        "kernel_ms_mean": device_ms,
        "region_ms_per_step": region_ms,
        "event_pair_ms_median": statistics.median(kms),
        "event_pair_ms_min": min(kms),
        "plan": plan,
        "rotate_w": rotate,
        "rotate_x": nx,
    }


def measure_library(p: Prepared, steps: int, warmup: int) -> float:
    """Device ms per launch of torch.mm (hipBLASLt) on the workload's own device
    operands, no bias or activation, timed like kernel_ms_mean (launches
    queued behind a spin kernel). A reference point beside the fused kernel;
    nothing of the product path runs through it."""
    import torch
    X, W, Y = p.Xs[0], p.Ws[0], p.Y
    for _ in range(warmup):
        torch.mm(X, W, out=Y)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        torch.mm(X, W, out=Y)
    enqueue_s = time.perf_counter() - t0
    torch.cuda.synchronize()
    torch.cuda._sleep(int(sleep_cycles_per_s() * (enqueue_s * 1.5 + 2e-4)))
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(steps):
        torch.mm(X, W, out=Y)
    ev[1].record()
    torch.cuda.synchronize()
    return ev[0].elapsed_time(ev[1]) / steps


def measure_library_int8(p: Prepared, steps: int, warmup: int) -> float:
    """Device ms per launch of torch._int_mm (the vendor library's int8 GEMM,
    i32 accumulation) on int8 copies of the workload's X and W, no bias or
    activation, timed like kernel_ms_mean. The narrowing to int8 is not
    included: this is the reference point for the GEMM half of the layer."""
    import torch
    X8, W8 = p.Xs[0].to(torch.int8), p.Ws[0].to(torch.int8)
    out = torch.empty((p.w.M, p.w.N), dtype=torch.int32, device="cuda")

    def run():
        torch._int_mm(X8, W8, out=out)
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    rows = min(64, p.w.M)  # a row sample against exact float64 sums on the host (|sum| < 2^53)
    want = (X8[:rows].cpu().double() @ W8.cpu().double()).to(torch.int64)
    if not torch.equal(out[:rows].cpu().to(torch.int64), want):
        raise RuntimeError("torch._int_mm is not exact on these operands")
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    enqueue_s = time.perf_counter() - t0
    torch.cuda.synchronize()
    torch.cuda._sleep(int(sleep_cycles_per_s() * (enqueue_s * 1.5 + 2e-4)))
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(steps):
        run()
    ev[1].record()
    torch.cuda.synchronize()
    return ev[0].elapsed_time(ev[1]) / steps


def measure_shapes(spec: str, steps: int, warmup: int) -> int:
    """--shapes "M,K,N;M,K,N...": the fused fp32 layer relu(X @ W + b) at each
    shape through the device entry (automatic plan), and the vendor's
    torch.mm (no bias or activation) on the same operands, both timed like
    kernel_ms_mean (launches queued behind a spin kernel). One JSON line per
    shape. A sample of rows is checked against a float64 torch product first."""
    import torch
    from mlir_edsl_hip import _native
    from mlir_edsl_hip.device import dense_launch
    shapes = [tuple(int(v) for v in t.split(",")) for t in spec.split(";") if t.strip()]
    g = torch.Generator(device="cuda").manual_seed(1234)

    def backlogged(fn) -> float:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        enqueue_s = time.perf_counter() - t0
        torch.cuda.synchronize()
        torch.cuda._sleep(int(sleep_cycles_per_s() * (enqueue_s * 1.5 + 2e-4)))
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record()
        for _ in range(steps):
            fn()
        ev[1].record()
        torch.cuda.synchronize()
        return ev[0].elapsed_time(ev[1]) / steps

    for M, K, N in shapes:
        X = torch.randn(M, K, device="cuda", generator=g)
        W = torch.randn(K, N, device="cuda", generator=g) / K ** 0.5
        b = torch.randn(N, device="cuda", generator=g)
        Y = torch.empty(M, N, device="cuda")
        dense_launch(X, W, b, Y, _native.EPI_BIAS_RELU)
        torch.cuda.synchronize()
        rows = torch.arange(0, M, max(1, M // 64), device="cuda")
        ref = torch.relu(X[rows].double() @ W.double() + b.double())
        err = ((Y[rows].double() - ref).norm() / ref.norm().clamp_min(1e-300)).item()
        if not err <= 1e-5:
            raise RuntimeError(f"{M}x{K}x{N}: relative error {err:.2e} against float64")
        plan = _native.last_plan()
        ms = backlogged(lambda: dense_launch(X, W, b, Y, _native.EPI_BIAS_RELU))
        vendor_ms = backlogged(lambda: torch.mm(X, W, out=Y))
        flops = 2.0 * M * N * K
        print(json.dumps({"shape": {"M": M, "K": K, "N": N}, "plan": plan, "kernel_ms_mean": round(ms, 5),
                          "tflops": round(flops / (ms * 1e-3) / 1e12, 2), "vendor_ms": round(vendor_ms, 5),
                          "vendor_vs_fused": round(vendor_ms / ms, 3), "rel_err_f64": float(f"{err:.2e}")}),
              flush=True)
    return 0


def step_value(wname: str, step_s: float) -> float:
    """Whole-step throughput in the workload's unit."""
    from mlir_edsl_hip.inputs import WORKLOADS
    wl = WORKLOADS[wname]
    if UNITS[wname] == "GB/s":
        return wl.compulsory_bytes / step_s / 1e9
    return wl.flops / step_s / 1e12


def load_traffic() -> dict:
    """HBM bytes per launch from the committed rocprofv3 PMC passes
    (FETCH_SIZE and WRITE_SIZE, copy-calibrated), keyed by workload."""
    p = os.path.join(ROOT, "profiles", "hbm_traffic_pmc.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f)
    return {}


def roofline_for(wname: str, r: dict, traffic: dict) -> dict:
    from mlir_edsl_hip.inputs import WORKLOADS
    w = WORKLOADS[wname]
    t = r["kernel_ms_mean"] * 1e-3
    tr = traffic.get(wname, {}).get("hbm_bytes_per_launch")
    if wname in ("c4", "c4s8"):
        achieved = w.compulsory_bytes / t / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK["hbm_gbs"],
                "unit": "GB/s", "frac": round(achieved / PEAK["hbm_gbs"], 4), "traffic": tr,
                "kernel": KERNEL_NAMES[wname], "algorithmic_bytes": w.compulsory_bytes}
    if wname == "c5":
        achieved = w.compulsory_bytes / t / 1e9
        tops = w.flops / t / 1e12
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK["hbm_gbs"],
                "unit": "GB/s", "frac": round(achieved / PEAK["hbm_gbs"], 4), "traffic": tr,
                "kernel": KERNEL_NAMES[wname], "algorithmic_bytes": w.compulsory_bytes,
                "int8_mfma": {"achieved": round(tops, 2), "peak": PEAK["int8_mfma_tops"],
                              "unit": "TOP/s", "frac": round(tops / PEAK["int8_mfma_tops"], 4)}}
    achieved = w.flops / t / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK["fp32_mfma_tflops"],
            "unit": "TFLOP/s", "frac": round(achieved / PEAK["fp32_mfma_tflops"], 4), "traffic": tr,
            "kernel": KERNEL_NAMES[wname], "algorithmic_flops": w.flops}


# ------------------------------------------------------------ host buffers
def _mean_call_s(fn, warmup: int, calls: int) -> float:
    for _ in range(warmup):
        fn()
    t0 = time.perf_counter()
    for _ in range(calls):
        fn()
    return (time.perf_counter() - t0) / calls


def measure_host_path(wname: str, arrays, calls: int) -> dict:
    """The reference's GPU calling pattern: host arrays in, host array out,
    through the memref-descriptor C ABI (include/edsl_hip.h). Each call copies
    the operands to the device, runs the kernels and copies Y back."""
    from mlir_edsl_hip import backend
    w_pattern = {"c1": "matmul"}.get(wname, "dense_relu")
    t = _mean_call_s(lambda: backend.run(w_pattern, *arrays), 1, calls)
    return {"value": round(step_value(wname, t), 3), "unit": UNITS[wname], "ms_per_call": round(t * 1e3, 4),
            "calls": calls, "what": "host numpy buffers through the memref-ABI entry: H2D + kernels + D2H"}


def _gpu_call(comp, name, arrays, out_shape):
    """The reference backend's execute_gpu_function marshalling (reference
    mlir_edsl/backend.py:248-271): (pointer, shape) pairs, raw bytes back,
    copied into a fresh array."""
    import numpy as np
    inputs = [(a.ctypes.data, list(a.shape)) for a in arrays]
    raw = comp.execute_gpu_function(name, inputs, list(out_shape), 4)
    return np.frombuffer(raw, dtype=arrays[0].dtype).reshape(out_shape).copy()


def measure_resident_host_path(wname: str, arrays, calls: int) -> dict:
    """The drop-in compiler (FunctionDef -> MLIRCompiler) called the way the
    reference front end calls execute_gpu_function, first as is (every
    operand copied in) and then with W and b bound device-resident: only X
    goes up and Y comes down per call."""
    from mlir_edsl_hip import _native, wire
    from mlir_edsl_hip._mlir_backend import MLIRCompiler
    from mlir_edsl_hip.inputs import WORKLOADS
    w = WORKLOADS[wname]
    comp = MLIRCompiler()
    comp.set_target("gpu")
    name = f"bench_{wname}_resident"
    comp.compile_function(wire.dense_layer(name, w.M, w.K, w.N, dtype=w.dtype))
    shape = (w.M, w.N)
    t_copy = _mean_call_s(lambda: _gpu_call(comp, name, arrays, shape), 1, calls)
    t0 = time.perf_counter()
    comp.bind_parameter(name, "W", arrays[1])
    comp.bind_parameter(name, "b", arrays[2])
    t_bind = time.perf_counter() - t0
    t_res = _mean_call_s(lambda: _gpu_call(comp, name, arrays, shape), 2, calls * 4)
    plan = _native.last_plan()
    comp.clear()
    return {"value": round(step_value(wname, t_res), 3), "unit": UNITS[wname], "ms_per_call": round(t_res * 1e3, 4),
            "calls": calls * 4, "plan": plan, "bind_ms": round(t_bind * 1e3, 2),
            "unbound_ms_per_call": round(t_copy * 1e3, 4),
            "what": "MLIRCompiler.execute_gpu_function on host arrays with W and b bound device-resident "
                    "(bind_parameter): X H2D + kernels + Y D2H per call; unbound_ms_per_call copies every "
                    "operand, as the reference does"}


def reference_gpu_points() -> list:
    """The reference's GPU benchmark (reference tests/gpu/test_gpu_benchmark.py:
    matmul and dense relu(X @ W + b) at 256, 512, 1024, np.random.rand inputs,
    3 warmup calls, mean wall-clock ms over 10) through the drop-in compiler,
    called the way the reference front end calls execute_gpu_function."""
    import numpy as np
    from mlir_edsl_hip import wire
    from mlir_edsl_hip._mlir_backend import MLIRCompiler
    comp = MLIRCompiler()
    comp.set_target("gpu")
    points = []
    for kind in ("matmul", "dense"):
        for n in (256, 512, 1024):
            name = f"ref_bench_{kind}_{n}"
            comp.compile_function(wire.dense_layer(name, n, n, n, bias=kind == "dense",
                                                   act="relu" if kind == "dense" else "none"))
            rng = np.random.default_rng(n)
            arrays = [rng.random((n, n), dtype=np.float32), rng.random((n, n), dtype=np.float32)]
            if kind == "dense":
                arrays.append(rng.random(n, dtype=np.float32))
            t = _mean_call_s(lambda: _gpu_call(comp, name, arrays, (n, n)), 3, 10)
            points.append({"kind": kind, "size": n, "ms_per_call": round(t * 1e3, 4),
                           "tflops": round(2 * n ** 3 / t / 1e12, 4)})
    comp.clear()
    return points


# --------------------------------------------------------------- CPU side
def cpu_model() -> str:
    """The host CPU: model name, family / model / stepping, logical CPUs on
    the host and in this process's affinity set."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" in line:
                    k, v = (s.strip() for s in line.split(":", 1))
                    if k in ("model name", "cpu family", "model", "stepping", "cpu MHz", "cpu cores",
                             "siblings") and k not in info:
                        info[k] = v
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 0
    return (f"{info.get('model name', 'unknown')} (family {info.get('cpu family', '?')}, model "
            f"{info.get('model', '?')}, stepping {info.get('stepping', '?')}, {info.get('cpu MHz', '?')} MHz; "
            f"{os.cpu_count()} logical CPUs on the host, {avail} in this process's affinity set)")


def cpu_baseline(wname: str, arrays, budget_s: float) -> dict:
    """The reference CPU-JIT schedule restated in C (the oracle: OpenMP over
    64x64 tiles, 8x8x8 fma micro-kernel, separate bias+ReLU pass; exact
    wrapping i32 for c5) on the first R rows of the workload, in the
    workload's unit. For f32 the micro-kernel runs on 8-wide FMA vectors as
    the reference JIT emits it (oracle_dense_f32_vec, bit-identical to the
    scalar restatement). R is sized so that one run takes about a third of the
    budget (at most the whole workload); runs repeat while the budget lasts
    (at least 3) and the median is reported."""
    import oracle
    from mlir_edsl_hip.inputs import WORKLOADS

    w = WORKLOADS[wname]
    threads = oracle.cpu_threads()
    bias = w.pattern != "matmul"

    def run(R: int) -> None:
        X = arrays[0][:R]
        if w.dtype == "i32":
            oracle.dense_i32(X, arrays[1], arrays[2], "relu", threads=threads)
        elif bias:
            oracle.dense_f32_vec(X, arrays[1], arrays[2], "relu", threads=threads)
        else:
            oracle.dense_f32_vec(X, arrays[1], None, "none", threads=threads)

    unit = min(64, w.M)
    t0 = time.perf_counter()
    run(unit)
    per_row = (time.perf_counter() - t0) / unit
    R = int(max(unit, min(w.M, (budget_s / 3) / max(per_row, 1e-9))) // unit * unit)
    times = []
    spent = 0.0
    # At least 3 runs; more while the budget lasts (the sample is capped at the
    # whole workload, which can take well under a third of the budget).
    while len(times) < 3 or (spent + times[-1] <= budget_s and len(times) < 25):
        t0 = time.perf_counter()
        run(R)
        times.append(time.perf_counter() - t0)
        spent += times[-1]
    t = statistics.median(times)
    if UNITS[wname] == "GB/s":
        work = 4 * (R * w.K + w.K * w.N + (w.N if bias else 0) + R * w.N)
        value = work / t / 1e9
    else:
        value = 2 * R * w.N * w.K / t / 1e12
    what = "X[R,K] @ W[K,N]" + (" + b, ReLU" if bias else "")
    what += "; wrapping i32" if w.dtype == "i32" else "; 8x8x8 fma micro-kernel on 8-wide AVX2 FMA vectors"
    return {"value": round(value, 5), "unit": UNITS[wname], "cores": threads, "kind": "port",
            "sample": f"rows 0..{R - 1} of {wname} ({what}, R={R}, K={w.K}, N={w.N}), "
                      f"median of {len(times)} runs, {t:.4g} s each",
            "host_cpu": cpu_model()}


# ------------------------------------------------------- trace summaries
def _short_kernel(name: str) -> str:
    """`gemm_f32_direct_kernel<0, 3>` from the demangled kernel name."""
    n = name.replace("void ", "").replace("(anonymous namespace)::", "")
    depth, end = 0, len(n)
    for i, ch in enumerate(n):  # the argument list: the first '(' outside template brackets
        depth += ch == "<"
        depth -= ch == ">"
        if ch == "(" and depth == 0:
            end = i
            break
    return n[:end].split("::")[-1]


def trace_summary(trace_csv: str, line_json: str, wname: str | None, warmup: int, steps: int) -> int:
    """Markdown summary of a rocprofv3 kernel trace of one bench run, beside
    the JSON line that run printed: every kernel's dispatch count and mean,
    then one workload's steps split into the bench's passes (warmup, timed
    region, backlogged device-time pass, event pairs; for c5 a second set, the
    cache-resident inputs) and the roofline its backlogged pass gives, against
    the line's own `roofline.frac`.

    A step is one dispatch of the workload's first kernel (KERNEL_NAMES) plus
    the dispatches right after it that belong to the same step (the split-K
    reduce of the small-M kernel; the int8 GEMM after the narrowing pass). The
    first kernel's name, template arguments included, is the one whose steps
    in the backlogged pass come closest to the line's kernel_ms_mean (the
    unfused sequence's GEMM and other workloads' instances of the same kernel
    are other template instances or other steps)."""
    import csv
    with open(line_json) as f:
        line = json.loads(f.read().strip().splitlines()[-1])
    head_name = line["config"]["workload"].split(":")[0]
    wname = wname or head_name
    if wname == head_name:
        rec = line
    else:
        rec = next(r for r in line["secondary"] if r["workload"] == wname)
        steps, warmup = SECONDARY_PLAN[wname][0], SECONDARY_PLAN[wname][1]
    with open(trace_csv) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Dispatch_Id"]))
    # A kernel that runs with several grids (the same tile for two workloads)
    # is told apart by its grid, so that one workload's steps are not mixed
    # with another's.
    grids: dict[str, set] = {}
    for r in rows:
        grids.setdefault(r["Kernel_Name"], set()).add(r.get("Grid_Size_X", r.get("Grid_Size", "")))

    def key(r):
        g = r.get("Grid_Size_X", r.get("Grid_Size", ""))
        return r["Kernel_Name"] + (f" [grid {g}]" if len(grids[r["Kernel_Name"]]) > 1 else "")
    disp = [(key(r), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3) for r in rows]
    by_name: dict[str, list[float]] = {}
    for name, us in disp:
        by_name.setdefault(name, []).append(us)
    subs = [k.strip() for k in KERNEL_NAMES[wname].split("+")]
    block = warmup + 3 * steps

    def steps_of(lead: str) -> list[list[tuple[str, float]]]:
        out = []
        for i, (name, us) in enumerate(disp):
            if name != lead:
                continue
            st = [(name, us)]
            for nm, u in disp[i + 1:]:
                if nm == lead or not any(k in nm for k in subs[1:]):
                    break
                st.append((nm, u))
            out.append(st)
        return out

    target_us = rec["kernel_ms_mean"] * 1e3
    best = None
    for name in by_name:
        if subs[0] not in name:
            continue
        st = steps_of(name)
        if len(st) < block:
            continue
        back = st[warmup + steps:warmup + 2 * steps]
        err = abs(statistics.mean(sum(u for _, u in s) for s in back) - target_us)
        if best is None or err < best[0]:
            best = (err, name, st)
    if best is None:
        print(f"no {subs[0]} kernel has {block} steps in the trace", file=sys.stderr)
        return 1
    _, lead, st = best
    out = ["| kernel | dispatches | mean us | median us |", "|---|---|---|---|"]
    for n, v in sorted(by_name.items(), key=lambda kv: -sum(kv[1])):
        base, sep, grid = n.partition(" [grid ")
        short = base if len(base) <= 90 else base[:87] + "..."
        if sep:
            short += sep + grid
        out.append(f"| `{short}` | {len(v)} | {statistics.mean(v):.1f} | {statistics.median(v):.1f} |")
    kinds = sorted({nm for s in st[:block] for nm, _ in s}, key=lambda nm: nm != lead)
    out += ["", f"Workload {wname}: a step is `{lead}`" +
            "".join(f" then `{k}`" for k in kinds[1:]) + f"; {len(st)} steps in the trace, "
            f"{block} per pass set ({warmup} warmup + 3 x {steps}).", "",
            "| pass | steps | step mean us | step median us | " +
            " | ".join(f"{_short_kernel(k)} mean us" for k in kinds) + " |",
            "|---|---|---|---|" + "---|" * len(kinds)]
    labels = ["warmup", "timed region", "backlogged (device time)", "event pairs"]
    sets = [("", st[:block])]
    if wname in RESIDENT_TOO and len(st) >= 2 * block:
        sets.append((" (inputs cache-resident)", st[block:2 * block]))
    backs = {}
    for tag, blk in sets:
        cuts = [blk[:warmup], blk[warmup:warmup + steps], blk[warmup + steps:warmup + 2 * steps],
                blk[warmup + 2 * steps:]]
        for label, part in zip(labels, cuts):
            tot = [sum(u for _, u in s) for s in part]
            per = [statistics.mean([u for s in part for nm, u in s if nm == k] or [0.0]) for k in kinds]
            out.append(f"| {label}{tag} | {len(part)} | {statistics.mean(tot):.2f} | {statistics.median(tot):.2f} | " +
                       " | ".join(f"{v:.2f}" for v in per) + " |")
        backs[tag] = statistics.mean(sum(u for _, u in s) for s in cuts[2])
    roof = rec["roofline"]
    work = roof.get("algorithmic_flops") or roof.get("algorithmic_bytes")
    scale = 1e12 if roof["unit"] == "TFLOP/s" else 1e9
    back = backs[""]
    achieved = work / (back * 1e-6) / scale
    frac = achieved / roof["peak"]
    out += ["", f"Backlogged pass, mean step of {steps}: {back:.2f} us -> {achieved:.2f} {roof['unit']}, "
                f"frac {frac:.4f} of {roof['peak']} {roof['unit']} (kernel durations only). The line: kernel_ms_mean "
                f"{rec['kernel_ms_mean'] * 1e3:.2f} us (the same pass's event span / {steps}, gaps between "
                f"dispatches included), achieved {roof['achieved']} {roof['unit']}, frac {roof['frac']}; relative "
                f"difference {abs(frac - roof['frac']) / roof['frac'] * 100:.2f} %."]
    print("\n".join(out))
    return 0


# -------------------------------------------------------------------- main
def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="c3", choices=sorted(UNITS),
                    help="workload of the headline line (default c3, the BASELINE metric's config)")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--secondary", default="c4,c5,c2,c1,c4s8,c3s8",
                    help="comma-separated workloads measured before the headline one")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="CPU budget of the headline's baseline (each secondary gets a third)")
    ap.add_argument("--no-host-path", action="store_true",
                    help="skip the host-buffer measurements (reference calling pattern, resident "
                         "weights, the reference's GPU benchmark points)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device-to-device copy of BYTES (3 times) and exit; "
                         "its FETCH_SIZE / WRITE_SIZE counters calibrate the traffic figures")
    ap.add_argument("--trace-summary", nargs=2, metavar=("KERNEL_TRACE_CSV", "BENCH_LINE_JSON"),
                    help="no GPU: summarize a rocprofv3 kernel trace of a bench run (with the same "
                         "--steps / --warmup) beside the JSON line that run printed; --summary-workload "
                         "picks the workload (default: the line's headline)")
    ap.add_argument("--summary-workload", default=None, choices=sorted(UNITS))
    ap.add_argument("--shapes", default=None, metavar="M,K,N;...",
                    help="only time the fused fp32 layer and the vendor's torch.mm at these shapes, "
                         "one JSON line each (--steps / --warmup apply)")
    args = ap.parse_args()
    if args.trace_summary:
        return trace_summary(args.trace_summary[0], args.trace_summary[1], args.summary_workload, args.warmup,
                             args.steps)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures the dense path on one GPU only: this build has no multi-GPU "
              "path. One GPU's share of an 8-way column-sharded layer is measured as the "
              "c4s8 and c3s8 workloads; run with --gpus 1.",
              file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    if args.shapes:
        return measure_shapes(args.shapes, args.steps, args.warmup)
    if args.copy_calibration:
        n = args.copy_calibration // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copied {n * 4} bytes x3")
        return 0
    from mlir_edsl_hip.inputs import WORKLOADS

    traffic = load_traffic()
    head_name = args.workload
    w = WORKLOADS[head_name]
    names = [] if args.no_secondary else [x.strip() for x in args.secondary.split(",") if x.strip()]
    names = [n for n in names if n != head_name] + [head_name]
    prepared = {}
    for n in names:
        prepared[n] = Prepared(n, SECONDARY_PLAN[n][2])
    torch.cuda.synchronize()
    log(f"[bench] inputs of {', '.join(names)} generated and resident")

    # Device-resident timing, back to back, headline last.
    results = {}
    for n in names:
        p = prepared[n]
        if n == head_name:
            log(f"[bench] {n} {p.w.description}: warmup {args.warmup}, steps {args.steps}")
            r = measure(p, args.steps, args.warmup)
        else:
            steps, warm, _ = SECONDARY_PLAN[n]
            r = measure(p, steps, warm)
        val = step_value(n, r["ms_per_step"] * 1e-3)
        r.update({"value": round(val, 3), "unit": UNITS[n], "roofline": roofline_for(n, r, traffic),
                  "config": {"M": p.w.M, "K": p.w.K, "N": p.w.N, "seed": p.w.seed, "dtype": p.w.dtype}})
        if n in RESIDENT_TOO and p.rotate > 1:
            rr = measure(p, SECONDARY_PLAN[n][0], SECONDARY_PLAN[n][1], rotate=1)
            r["inputs_cache_resident"] = {
                "ms_per_step": rr["ms_per_step"], "kernel_ms_mean": rr["kernel_ms_mean"],
                "value": round(step_value(n, rr["ms_per_step"] * 1e-3), 3), "unit": UNITS[n],
                "roofline": roofline_for(n, rr, traffic),
                "what": "the same layer with one input set, which the 256 MB Infinity Cache holds"}
        if n in UNFUSED_TOO:
            steps = args.steps if n == head_name else SECONDARY_PLAN[n][0]
            ru = measure(p, max(10, steps // 2), SECONDARY_PLAN[n][1], unfused=True)
            r["unfused_reference_sequence"] = {
                "ms_per_step": round(ru["ms_per_step"], 5), "kernel_ms_mean": round(ru["kernel_ms_mean"], 5),
                "value": round(step_value(n, ru["ms_per_step"] * 1e-3), 3), "unit": UNITS[n],
                "launches": 3, "plan": ru["plan"],
                "fused_speedup_device": round(ru["kernel_ms_mean"] / r["kernel_ms_mean"], 3),
                "what": "fill + GEMM without epilogue + separate bias/ReLU kernel: the reference GPU "
                        "lowering's three launches (reference cpp/src/MLIRLowering.cpp:495-518), on this "
                        "library's kernels"}
        if n in LIBRARY_TOO and p.w.dtype == "f32":
            steps = args.steps if n == head_name else SECONDARY_PLAN[n][0]
            lib_ms = measure_library(p, steps, SECONDARY_PLAN[n][1])
            r["vendor_library"] = {
                "kernel_ms_mean": round(lib_ms, 5),
                "tflops": round(p.w.flops / (lib_ms * 1e-3) / 1e12, 2),
                "fused_kernel_vs_library": round(lib_ms / r["kernel_ms_mean"], 3),
                "what": "torch.mm (hipBLASLt) on the same device operands, no bias or ReLU, timed like "
                        "kernel_ms_mean; a reference point, not part of the product path"}
        elif n in LIBRARY_TOO:
            steps = args.steps if n == head_name else SECONDARY_PLAN[n][0]
            lib_ms = measure_library_int8(p, steps, SECONDARY_PLAN[n][1])
            r["vendor_library"] = {
                "kernel_ms_mean": round(lib_ms, 5),
                "tops": round(p.w.flops / (lib_ms * 1e-3) / 1e12, 2),
                "layer_vs_library_gemm": round(lib_ms / r["kernel_ms_mean"], 3),
                "what": "torch._int_mm (the vendor int8 GEMM, i32 accumulation) on int8 copies of the same "
                        "X and W (one input set, narrowing not included), no bias or ReLU, timed like "
                        "kernel_ms_mean; compare with this layer's GEMM kernel alone in a kernel trace. "
                        "A reference point, not part of the product path"}
        log(f"[bench] {n} done: {val:.2f} {UNITS[n]}, kernel {r['kernel_ms_mean'] * 1e3:.1f} us, region "
            f"{r['region_ms_per_step'] * 1e3:.1f} us/step [{r['plan']}]")
        results[n] = r
    head = results[head_name]
    for p in prepared.values():
        p.free()

    # Host buffers: the reference's calling pattern, resident weights, the
    # reference's own GPU benchmark points.
    host, ref_points = {}, None
    if not args.no_host_path:
        for n in names:
            steps = 10 if WORKLOADS[n].flops < 2e11 else 5
            host[n] = measure_host_path(n, prepared[n].arrays, steps)
            log(f"[bench] host path {n}: {host[n]['ms_per_call']:.3f} ms/call")
        if "c4" in names and WORKLOADS["c4"].dtype == "f32":
            host["c4_resident"] = measure_resident_host_path("c4", prepared["c4"].arrays, 10)
            log(f"[bench] c4 with W, b resident: {host['c4_resident']['ms_per_call']:.3f} ms/call "
                f"(every operand copied: {host['c4_resident']['unbound_ms_per_call']:.3f})")
        ref_points = reference_gpu_points()
        log("[bench] reference GPU benchmark points: " +
            ", ".join(f"{q['kind']} {q['size']}: {q['ms_per_call']:.3f} ms" for q in ref_points))

    cpu = {}
    if not args.no_cpu_baseline:
        for n in names:
            budget = args.cpu_seconds if n == head_name else args.cpu_seconds / 3
            log(f"[bench] cpu baseline (oracle, row sample of {n}, {budget:.0f} s)")
            cpu[n] = cpu_baseline(n, prepared[n].arrays, budget)
            log(f"[bench] cpu baseline {n}: {cpu[n]['value']} {cpu[n]['unit']} on {cpu[n]['cores']} threads")

    secondary = []
    for n in names:
        if n == head_name:
            continue
        r = results[n]
        if n in host:
            r["host_path"] = host[n]
        if n == "c4" and "c4_resident" in host:
            r["host_path_resident_weights"] = host["c4_resident"]
        if n in cpu:
            r["cpu_baseline"] = cpu[n]
        secondary.append(r)

    value = step_value(head_name, head["ms_per_step"] * 1e-3)
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": UNITS[head_name],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "region_ms_per_step": round(head["region_ms_per_step"], 4),
        "kernel_ms_mean": round(head["kernel_ms_mean"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if w.dtype == "f32" else "i32 (int8 MFMA)",
        "data": "synthetic: numpy PCG64 default_rng(seed); X~N(0,1), W~N(0,1/K), b~U[-0.1,0.1) "
                "(c5: ints in [-8,7], b in [-512,511])",
        "config": {"workload": f"{head_name}: {w.description}", "M": w.M, "N": w.N, "K": w.K,
                   "seed": w.seed, "parallelism": "single GPU", "plan": head["plan"],
                   "w_buffers_rotated": head["rotate_w"], "x_buffers_rotated": head["rotate_x"]},
        "roofline": roofline_for(head_name, head, traffic),
        "cpu_baseline": cpu.get(head_name),
        "secondary": secondary,
    }
    for k in ("unfused_reference_sequence", "inputs_cache_resident", "vendor_library"):
        if k in head:
            line[k] = head[k]
    if head_name in host:
        line["host_path"] = host[head_name]
    if ref_points is not None:
        line["reference_gpu_benchmark"] = {
            "points": ref_points,
            "what": "the reference's GPU benchmark (tests/gpu/test_gpu_benchmark.py): matmul and dense "
                    "relu(X@W+b) at 256/512/1024 on host arrays through the drop-in compiler's "
                    "execute_gpu_function, 3 warmup calls, mean of 10"}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
