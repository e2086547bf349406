"""bench.py --trace-summary on a synthetic kernel trace (CPU only).

Dispatches of one kernel with different grids (the one-wave 64x64 tile of
the c3 shard, and the same kernel run by another layer before it) must not
be mixed: the summary keys such a kernel by its grid and splits each
workload's own steps into the bench's passes.
"""
from __future__ import annotations

import csv
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNEL = "void edsl::(anonymous namespace)::gemm_f32_direct64_kernel<4, 0, 3>(edsl::GemmF32Args)"
KERNEL_RC = "void edsl::(anonymous namespace)::gemm_f32_direct_rc_kernel<4, 4, 3>(edsl::GemmF32Args)"


def _write_trace(path, blocks):
    """blocks: (kernel, grid, count, duration in us); dispatches back to back."""
    fields = ["Kind", "Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X"]
    t, d = 1_000_000, 0
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for kernel, grid, count, us in blocks:
            for _ in range(count):
                d += 1
                w.writerow({"Kind": "KERNEL_DISPATCH", "Dispatch_Id": d, "Kernel_Name": kernel,
                            "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000), "Grid_Size_X": grid})
                t += int(us * 1000) + 500


def test_shared_kernel_is_split_by_grid(tmp_path):
    # c2: 20 warmup + 3 x 100 steps at 20 us; the c3 shard's kernel at another
    # grid (320 dispatches at 60 us); then c3s8: 100 warmup + 3 x 100 at 120 us
    trace = tmp_path / "trace.csv"
    _write_trace(trace, [(KERNEL_RC, 65536, 320, 20.0), (KERNEL, 65536, 320, 60.0), (KERNEL, 131072, 400, 120.0)])
    def rec(wname, ms, flops):
        achieved = flops / (ms * 1e-3) / 1e12
        return {"workload": wname, "kernel_ms_mean": ms,
                "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": 157.3, "unit": "TFLOP/s",
                             "frac": round(achieved / 157.3, 4), "algorithmic_flops": flops}}
    line = {"config": {"workload": "c3: fp32 dense 4096^3"},
            "secondary": [rec("c2", 0.020, 2 * 1024 ** 3), rec("c3s8", 0.120, 2 * 4096 * 4096 * 512)]}
    line_path = tmp_path / "line.json"
    line_path.write_text(json.dumps(line) + "\n")
    for wname, us in (("c2", 20.0), ("c3s8", 120.0)):
        out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--trace-summary", str(trace),
                              str(line_path), "--summary-workload", wname],
                             capture_output=True, text=True, check=True).stdout
        if wname == "c3s8":
            assert "[grid 131072]" in out and "[grid 65536]" in out, out
        back = [ln for ln in out.splitlines() if ln.startswith("Backlogged pass")][0]
        assert f"mean step of 100: {us:.2f} us" in back, back
