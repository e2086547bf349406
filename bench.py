#!/usr/bin/env python3
"""Benchmark of the dense hot path on one MI355X.

Headline (BASELINE.json metric): fused fp32 matmul+bias+ReLU at M=N=K=4096
(workload c3), in TFLOP/s and as a fraction of the dense fp32 MFMA peak.
Secondary lines (same run): the M=16, K=N=8192 layer in GB/s (c4, W rotated
over 3 buffers so the 256 MB Infinity Cache cannot serve it), the integer
layer 2048^3 (c5), 1024^3 (c2), the 256^3 matmul (c1), and one GPU's share
of c4 and c3 column-sharded over 8 GPUs (c4s8: N=1024, W rotated over 12
buffers; c3s8: N=512).

A step is one call of the dense layer on device-resident inputs (the
C-ABI launch entry point, enqueued on torch's current stream). W warmup
steps, then K timed steps between two device synchronisations (the wall
clock gives `value`). A second pass enqueues K more steps behind a short
spin kernel, so the GPU never waits on the host, between two HIP events on
the same stream: their device time / K is the average launch duration used
for the roofline. A third pass with one event pair per launch reports the
spread.
The CPU baseline times the oracle (a C restatement of the reference CPU-JIT
schedule) on a row sample of the same workload, on this host's cores.

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
KERNEL_NAMES = {"c1": "gemm_f32_kernel", "c2": "gemm_f32_kernel", "c3": "gemm_f32_kernel",
                "c4": "gemv_f32_kernel + gemv_reduce_kernel", "c5": "narrow_i8_kernel + gemm_i8_ksplit_kernel",
                "c3s8": "gemm_f32_kernel", "c4s8": "gemv_f32_kernel + gemv_reduce_kernel"}


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


def measure(wname: str, steps: int, warmup: int, rotate: int = 1) -> dict:
    import torch

    from mlir_edsl_hip import _native
    from mlir_edsl_hip.device import dense_launch
    from mlir_edsl_hip.inputs import WORKLOADS, make_inputs

    w = WORKLOADS[wname]
    arrays = make_inputs(w)
    dev = [torch.from_numpy(a).cuda() for a in arrays]
    X, W = dev[0], dev[1]
    b = dev[2] if len(dev) > 2 else None
    Ws = [W] + [W.clone() for _ in range(rotate - 1)]
    dtype = torch.float32 if w.dtype == "f32" else torch.int32
    Y = torch.empty((w.M, w.N), dtype=dtype, device="cuda")
    epi = _native.EPI_BIAS_RELU if w.pattern == "dense_relu" else _native.EPI_NONE

    def launch(i: int) -> None:
        dense_launch(X, Ws[i % rotate], b, Y, epi)

    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    plan = _native.last_plan()
    # Timed region (the contract's): K steps between two synchronisations;
    # the wall clock gives `value`. Two events on the stream record its device
    # span as well (reported as region_ms_per_step).
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
    wall_region_ms = region[0].elapsed_time(region[1]) / steps
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
    res = {
        "workload": wname,
        "ms_per_step": (t1 - t0) * 1e3 / steps,
        "kernel_ms_mean": device_ms,
        "region_ms_per_step": wall_region_ms,
        "event_pair_ms_median": statistics.median(kms),
        "event_pair_ms_min": min(kms),
        "plan": plan,
        "rotate_w": rotate,
    }
    del X, W, Ws, Y, dev
    torch.cuda.empty_cache()
    return res


def measure_host_path(wname: str, calls: int) -> dict:
    """The reference's GPU calling pattern: host arrays in, host array out,
    through the memref-descriptor C ABI (include/edsl_hip.h). Each call copies
    the operands to the device, runs the kernels and copies Y back."""
    from mlir_edsl_hip import backend
    from mlir_edsl_hip.inputs import WORKLOADS, make_inputs

    w = WORKLOADS[wname]
    arrays = make_inputs(w)
    backend.run(w.pattern, *arrays)  # first call sizes the staging buffers
    t0 = time.perf_counter()
    for _ in range(calls):
        backend.run(w.pattern, *arrays)
    t = (time.perf_counter() - t0) / calls
    return {"value": round(step_value(wname, t), 3), "unit": UNITS[wname], "ms_per_call": round(t * 1e3, 4),
            "calls": calls, "what": "host numpy buffers through the memref-ABI entry: H2D + kernels + D2H"}


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


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(wname: str, budget_s: float) -> dict:
    """The oracle (C restatement of the reference CPU-JIT schedule: OpenMP
    over 64x64 tiles, 8x8x8 fma micro-kernel, separate bias+ReLU pass; exact
    wrapping i32 for c5) on the first R rows of the workload, in the
    workload's unit. R is sized so that one run takes about a third of the
    budget (at most the whole workload); runs repeat while the budget lasts
    (at least 3) and the median is reported."""
    import oracle
    from mlir_edsl_hip.inputs import WORKLOADS, make_inputs

    w = WORKLOADS[wname]
    arrays = make_inputs(w)
    threads = oracle.cpu_threads()
    bias = w.pattern != "matmul"

    def run(R: int) -> None:
        X = arrays[0][:R]
        if w.dtype == "i32":
            oracle.dense_i32(X, arrays[1], arrays[2], "relu", threads=threads)
        elif bias:
            oracle.dense_f32(X, arrays[1], arrays[2], "relu", threads=threads)
        else:
            oracle.dense_f32(X, arrays[1], None, "none", threads=threads)

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
    return {"value": round(value, 5), "unit": UNITS[wname], "cores": threads, "kind": "port",
            "sample": f"rows 0..{R - 1} of {wname} ({what}, R={R}, K={w.K}, N={w.N}), "
                      f"median of {len(times)} runs, {t:.3f} s each",
            "host_cpu": cpu_model()}


UNITS = {"c1": "TFLOP/s", "c2": "TFLOP/s", "c3": "TFLOP/s", "c4": "GB/s", "c5": "TOP/s",
         "c3s8": "TFLOP/s", "c4s8": "GB/s"}
# (steps, warmup, W buffers rotated) of each workload when it is not the headline.
# W is rotated over enough copies to exceed the 256 MB Infinity Cache where it
# would otherwise be served from there: c4 3 x 256 MiB, c4s8 12 x 32 MiB.
SECONDARY_PLAN = {"c4": (200, 20, 3), "c5": (100, 20, 1), "c2": (100, 20, 1), "c1": (200, 20, 1),
                  "c3": (50, 10, 1), "c3s8": (100, 10, 1), "c4s8": (300, 30, 12)}


def step_value(wname: str, step_s: float) -> float:
    """Whole-step throughput in the workload's unit."""
    from mlir_edsl_hip.inputs import WORKLOADS
    wl = WORKLOADS[wname]
    if UNITS[wname] == "GB/s":
        return wl.compulsory_bytes / step_s / 1e9
    return wl.flops / step_s / 1e12


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="c3", choices=sorted(UNITS),
                    help="workload of the headline line (default c3, the BASELINE metric's config)")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--secondary", default="c4,c5,c2,c1,c4s8,c3s8",
                    help="comma-separated workloads measured after the headline one")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--host-path", action="store_true",
                    help="also time the memref-ABI entry on host (numpy) buffers for the headline "
                         "workload: H2D copies + kernels + D2H, as the reference GPU path does "
                         "(reported as host_path, never as value)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device-to-device copy of BYTES (3 times) and exit; "
                         "its FETCH_SIZE / WRITE_SIZE counters calibrate the traffic figures")
    args = ap.parse_args()

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
    rotate = SECONDARY_PLAN[head_name][2]
    log(f"[bench] {head_name} {w.description}: warmup {args.warmup}, steps {args.steps}")
    head = measure(head_name, args.steps, args.warmup, rotate=rotate)
    log(f"[bench] {head_name} done: {head['ms_per_step']:.4f} ms/step, kernel "
        f"{head['kernel_ms_mean'] * 1e3:.1f} us [{head['plan']}]")

    secondary = []
    if not args.no_secondary:
        for wname in [x.strip() for x in args.secondary.split(",") if x.strip()]:
            if wname == head_name:
                continue
            steps, warm, rot = SECONDARY_PLAN[wname]
            log(f"[bench] {wname} {WORKLOADS[wname].description}")
            r = measure(wname, steps, warm, rotate=rot)
            wl = WORKLOADS[wname]
            val = step_value(wname, r["ms_per_step"] * 1e-3)
            r.update({"value": round(val, 3), "unit": UNITS[wname],
                      "roofline": roofline_for(wname, r, traffic),
                      "config": {"M": wl.M, "K": wl.K, "N": wl.N, "seed": wl.seed, "dtype": wl.dtype}})
            log(f"[bench] {wname} done: {val:.2f} {UNITS[wname]}, kernel {r['kernel_ms_mean'] * 1e3:.1f} us "
                f"[{r['plan']}]")
            secondary.append(r)

    host = None
    if args.host_path:
        host = measure_host_path(head_name, max(3, args.steps // 5))
        log(f"[bench] host path: {host['value']:.2f} {host['unit']} ({host['ms_per_call']:.3f} ms/call)")

    cpu = None
    if not args.no_cpu_baseline:
        log(f"[bench] cpu baseline (oracle, row sample of {head_name})")
        cpu = cpu_baseline(head_name, args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu['value']} {cpu['unit']} on {cpu['cores']} threads")

    value = step_value(head_name, head["ms_per_step"] * 1e-3)
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": UNITS[head_name],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if w.dtype == "f32" else "i32 (int8 MFMA)",
        "data": "synthetic: numpy PCG64 default_rng(seed); X~N(0,1), W~N(0,1/K), b~U[-0.1,0.1) "
                "(c5: ints in [-8,7], b in [-512,511])",
        "config": {"workload": f"{head_name}: {w.description}", "M": w.M, "N": w.N, "K": w.K,
                   "seed": w.seed, "parallelism": "single GPU", "plan": head["plan"],
                   "w_buffers_rotated": rotate},
        "roofline": roofline_for(head_name, head, traffic),
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    if host is not None:
        line["host_path"] = host
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
