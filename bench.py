#!/usr/bin/env python3
"""Benchmark of the dense hot path on one MI355X.

Headline (BASELINE.json metric): fused fp32 matmul+bias+ReLU at M=N=K=4096
(workload c3), in TFLOP/s and as a fraction of the dense fp32 MFMA peak.
Secondary lines (same run): the M=16, K=N=8192 layer in GB/s (c4, W rotated
over 3 buffers so the 256 MB Infinity Cache cannot serve it), the integer
layer 2048^3 (c5), 1024^3 (c2) and the 256^3 matmul (c1).

A step is one call of the dense layer on device-resident inputs (the
C-ABI launch entry point, enqueued on torch's current stream). W warmup
steps, then K timed steps between two device synchronisations; per-launch
HIP events on the same stream give the kernel time used for the roofline.
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
                "c4": "gemv_f32_kernel", "c5": "narrow_i8_kernel + gemm_i8_kernel"}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


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
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        launch(i)
        ends[i].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    kms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    res = {
        "workload": wname,
        "ms_per_step": (t1 - t0) * 1e3 / steps,
        "kernel_ms_mean": statistics.fmean(kms),
        "kernel_ms_median": statistics.median(kms),
        "plan": plan,
        "rotate_w": rotate,
    }
    del X, W, Ws, Y, dev
    torch.cuda.empty_cache()
    return res


def load_traffic() -> dict:
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f)
    return {}


def roofline_for(wname: str, r: dict, traffic: dict) -> dict:
    from mlir_edsl_hip.inputs import WORKLOADS
    w = WORKLOADS[wname]
    t = r["kernel_ms_mean"] * 1e-3
    tr = traffic.get(wname, {}).get("hbm_bytes_per_launch")
    if wname == "c4":
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
    over 64x64 tiles, 8x8x8 fma micro-kernel, separate bias+ReLU pass) on the
    first R rows of the workload; R is sized so that one run takes about a
    third of the budget, and the median of 3 runs is reported."""
    import oracle
    from mlir_edsl_hip.inputs import WORKLOADS, make_inputs

    w = WORKLOADS[wname]
    X, W, b = make_inputs(w)
    threads = oracle.cpu_threads()
    R = 64
    t0 = time.perf_counter()
    oracle.dense_f32(X[:R], W, b, "relu", threads=threads)
    t_probe = time.perf_counter() - t0
    per_row = t_probe / R
    R = int(max(64, min(w.M, (budget_s / 3) / max(per_row, 1e-9))) // 64 * 64)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        oracle.dense_f32(X[:R], W, b, "relu", threads=threads)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    flops = 2 * R * w.N * w.K
    return {"value": round(flops / t / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"rows 0..{R - 1} of {wname} (X[{R},{w.K}] @ W[{w.K},{w.N}] + b, ReLU), "
                      f"median of 3 runs, {t:.2f} s each",
            "host_cpu": cpu_model()}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--secondary", default="c4,c5,c2,c1",
                    help="comma-separated secondary workloads to measure after c3")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device-to-device copy of BYTES (3 times) and exit; "
                         "its FETCH_SIZE / WRITE_SIZE counters calibrate the traffic figures")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures the dense path on one GPU only: this build has no multi-GPU "
              "path (column-sharding design in DESIGN.md); run with --gpus 1.", file=sys.stderr)
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
    w = WORKLOADS["c3"]
    log(f"[bench] c3 {w.description}: warmup {args.warmup}, steps {args.steps}")
    head = measure("c3", args.steps, args.warmup)
    log(f"[bench] c3 done: {head['ms_per_step']:.3f} ms/step, kernel {head['kernel_ms_mean']:.3f} ms [{head['plan']}]")

    secondary = []
    if not args.no_secondary:
        plan = {"c4": (200, 3), "c5": (100, 1), "c2": (100, 1), "c1": (200, 1)}
        for wname in [w.strip() for w in args.secondary.split(",") if w.strip()]:
            steps, rot = plan[wname]
            log(f"[bench] {wname} {WORKLOADS[wname].description}")
            r = measure(wname, steps, 20, rotate=rot)
            wl = WORKLOADS[wname]
            step_s = r["ms_per_step"] * 1e-3
            if wname == "c4":
                val, unit = wl.compulsory_bytes / step_s / 1e9, "GB/s"
            elif wname == "c5":
                val, unit = wl.flops / step_s / 1e12, "TOP/s"
            else:
                val, unit = wl.flops / step_s / 1e12, "TFLOP/s"
            r.update({"value": round(val, 3), "unit": unit, "roofline": roofline_for(wname, r, traffic),
                      "config": {"M": wl.M, "K": wl.K, "N": wl.N, "seed": wl.seed, "dtype": wl.dtype}})
            log(f"[bench] {wname} done: {val:.2f} {unit}, kernel {r['kernel_ms_mean'] * 1e3:.1f} us [{r['plan']}]")
            secondary.append(r)

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline (oracle, row sample of c3)")
        cpu = cpu_baseline("c3", args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu['value']} TFLOP/s on {cpu['cores']} threads")

    value = w.flops / (head["ms_per_step"] * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: numpy PCG64 default_rng(seed); X~N(0,1), W~N(0,1/K), b~U[-0.1,0.1)",
        "config": {"workload": "c3: fp32 dense relu(X@W+b), M=N=K=4096", "M": w.M, "N": w.N,
                   "K": w.K, "seed": w.seed, "parallelism": "single GPU", "plan": head["plan"]},
        "roofline": roofline_for("c3", head, traffic),
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
