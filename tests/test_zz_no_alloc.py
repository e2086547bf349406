"""edsl_hip_dense_f32_launch_noalloc: the allocation-free f32 launch.

Its kernels take their scratch (the small-M split-K partials) from
a static device array instead of library allocations. Results must equal the
ordinary entry point's bit for bit (same plan, same kernels), on consecutive
calls that reuse the array with different sizes, and plans that need more
scratch than the array holds are rejected on the host. Run under a
global-mode HIP stream capture, where the runtime refuses hipMalloc, as the
first library call of a fresh process, it captures and replays like the
allocating entry; the allocating entry's first split-K call, captured the
same way, is refused (so the capture does catch an allocation).
"""
from __future__ import annotations

import json
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from conftest import assert_f32_parity
from mlir_edsl_hip import _native

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _inputs(M, K, N, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.float32(np.sqrt(K))).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, N).astype(np.float32)
    return X, W, b


def _launch(torch, entry, X, W, b, epi, x_off=0):
    """Runs one C-ABI entry on device copies (X at an element offset when
    x_off > 0, which misaligns its rows); returns (Y, plan)."""
    M, K = X.shape
    N = W.shape[1]
    xbuf = torch.zeros(M * K + x_off, dtype=torch.float32, device="cuda")
    tX = xbuf[x_off:].view(M, K)
    tX.copy_(torch.from_numpy(X))
    tW, tb = torch.from_numpy(W).cuda(), torch.from_numpy(b).cuda()
    tY = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    fn = getattr(_native.lib(), entry)
    rc = fn(tX.data_ptr(), K, tW.data_ptr(), N, tb.data_ptr(), tY.data_ptr(), N, M, N, K, epi, 0.02,
            torch.cuda.current_stream().cuda_stream)
    if rc != 0:
        raise RuntimeError(_native.last_error())
    plan = _native.last_plan()
    torch.cuda.synchronize()
    return tY.cpu().numpy(), plan


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    return torch


# Each pair: a larger call, then a smaller one that reuses the same array.
_PAIRS = [
    # c4 (split-K partials, 2 MiB), then an odd-K layer (unaligned X rows, K tail)
    ((16, 8192, 8192, 0, _native.EPI_BIAS_RELU), (5, 1003, 1024, 1, _native.EPI_BIAS_LEAKY)),
    # four row blocks with misaligned X, then one row block, aligned
    ((64, 4096, 4096, 3, _native.EPI_BIAS), (16, 2048, 2048, 0, _native.EPI_RELU)),
    # a tiled layer (no scratch at all), then the c4 column shard
    ((512, 1024, 768, 0, _native.EPI_BIAS_RELU), (16, 8192, 1024, 0, _native.EPI_BIAS_RELU)),
]


@pytest.mark.parametrize("pair", _PAIRS, ids=["c4-then-oddK", "mb4-then-mb1", "tiled-then-shard"])
def test_noalloc_matches_the_allocating_entry(pair, torch_cuda):
    for i, (M, K, N, x_off, epi) in enumerate(pair):
        X, W, b = _inputs(M, K, N, 100 * i + M + K + N)
        ref, ref_plan = _launch(torch_cuda, "edsl_hip_dense_f32_launch", X, W, b, epi, x_off)
        got, plan = _launch(torch_cuda, "edsl_hip_dense_f32_launch_noalloc", X, W, b, epi, x_off)
        print(f"call {i}: {M}x{K}x{N} x_off={x_off} [{plan}]", flush=True)
        assert plan.replace(" +fixed-scratch", "") == ref_plan, (plan, ref_plan)
        if "+reduce" in plan:
            assert plan.endswith("+fixed-scratch"), plan
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
            f"{np.count_nonzero(got.view(np.uint32) != ref.view(np.uint32))} elements differ"
        act = {_native.EPI_BIAS_RELU: "relu", _native.EPI_RELU: "relu", _native.EPI_BIAS_LEAKY: "leaky",
               _native.EPI_BIAS: "none"}[epi]
        assert_f32_parity(got, oracle.dense_f32_chains(X, W, b if epi & 1 else None, act, 0.02), K)


def test_noalloc_rejects_plans_beyond_its_scratch(torch_cuda):
    """Four row blocks with 16 forced K splits at N = 8192 need 32 MiB of
    partials, twice the static array: rejected before any launch."""
    from mlir_edsl_hip.device import set_gemv_ksplit
    M, K, N = 64, 8192, 8192
    tX = torch_cuda.zeros((M, K), device="cuda")
    tW = torch_cuda.zeros((K, N), device="cuda")
    tY = torch_cuda.full((M, N), 7.0, device="cuda")
    set_gemv_ksplit(16)
    try:
        rc = _native.lib().edsl_hip_dense_f32_launch_noalloc(
            tX.data_ptr(), K, tW.data_ptr(), N, None, tY.data_ptr(), N, M, N, K, _native.EPI_RELU, 0.0,
            torch_cuda.cuda.current_stream().cuda_stream)
    finally:
        set_gemv_ksplit(0)
    code, msg = _native.last_error()
    assert rc == -5 and code == -5, (rc, code, msg)
    assert "needs 33554432 bytes of scratch" in msg and f"holds {_native.NOALLOC_SCRATCH_BYTES}" in msg, msg
    torch_cuda.cuda.synchronize()
    assert bool((tY == 7.0).all())  # nothing ran


_SCRIPT = r'''
import ctypes, json, sys
sys.path.insert(0, %(pkg)r)
import numpy as np
import torch
from mlir_edsl_hip import _native

torch.zeros(1, device="cuda")              # the HIP runtime is up; nothing of the library has run
L = _native.lib()
hip = ctypes.CDLL(next(l.split()[-1] for l in open("/proc/self/maps") if "libamdhip64" in l))
vp, c_int = ctypes.c_void_p, ctypes.c_int
hip.hipStreamCreateWithFlags.argtypes = [ctypes.POINTER(vp), ctypes.c_uint]
hip.hipStreamBeginCapture.argtypes = [vp, c_int]
hip.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, ctypes.c_char_p, ctypes.c_size_t]
hip.hipGraphLaunch.argtypes = [vp, vp]
hip.hipStreamSynchronize.argtypes = [vp]
hip.hipGraphExecDestroy.argtypes = [vp]
hip.hipGraphDestroy.argtypes = [vp]
hip.hipStreamDestroy.argtypes = [vp]
GLOBAL = 0                                  # hipStreamCaptureModeGlobal

stream = vp()
assert hip.hipStreamCreateWithFlags(ctypes.byref(stream), 1) == 0
out = {}
for name, (M, K, N) in (("small_m_split_k", (16, 4096, 4096)), ("tiled", (512, 1024, 768))):
    g = torch.Generator(device="cuda").manual_seed(M + K)
    X = torch.randn(M, K, device="cuda", generator=g)
    W = torch.randn(K, N, device="cuda", generator=g) / K ** 0.5
    b = torch.randn(N, device="cuda", generator=g)
    Yg = torch.full((M, N), float("nan"), device="cuda")
    Ye = torch.full((M, N), float("nan"), device="cuda")
    torch.cuda.synchronize()
    args = (X.data_ptr(), K, W.data_ptr(), N, b.data_ptr())
    assert hip.hipStreamBeginCapture(stream, GLOBAL) == 0
    rc = L.edsl_hip_dense_f32_launch_noalloc(*args, Yg.data_ptr(), N, M, N, K, _native.EPI_BIAS_RELU, 0.0, stream)
    plan = _native.last_plan()
    graph = vp()
    end = hip.hipStreamEndCapture(stream, ctypes.byref(graph))
    res = {"rc": rc, "end": end, "plan": plan, "error": _native.last_error()[1] if rc else ""}
    if rc == 0 and end == 0:
        ex = vp()
        assert hip.hipGraphInstantiate(ctypes.byref(ex), graph, None, None, 0) == 0
        for _ in range(2):                  # two replays, each against the eager run
            assert hip.hipGraphLaunch(ex, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            rce = L.edsl_hip_dense_f32_launch(*args, Ye.data_ptr(), N, M, N, K, _native.EPI_BIAS_RELU, 0.0,
                                              torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            res.setdefault("same", []).append(rce == 0 and bool(torch.equal(Yg.view(torch.int32), Ye.view(torch.int32))))
            Yg.fill_(float("nan"))
            torch.cuda.synchronize()
        hip.hipGraphExecDestroy(ex)
        hip.hipGraphDestroy(graph)
    out[name] = res

# Control: the allocating entry's split-K workspace has never been sized in
# this process (above, only its tiled plan ran eagerly), so a split-K call
# under the same capture needs hipMalloc, which the capture must refuse.
M, K, N = 32, 8192, 8192
X = torch.randn(M, K, device="cuda"); W = torch.randn(K, N, device="cuda"); Y = torch.empty(M, N, device="cuda")
torch.cuda.synchronize()
assert hip.hipStreamBeginCapture(stream, GLOBAL) == 0
rc = L.edsl_hip_dense_f32_launch(X.data_ptr(), K, W.data_ptr(), N, None, Y.data_ptr(), N, M, N, K, _native.EPI_RELU, 0.0,
                                 stream)
graph = vp()
end = hip.hipStreamEndCapture(stream, ctypes.byref(graph))
out["control"] = {"rc": rc, "end": end, "error": _native.last_error()[1] if rc else "", "plan": _native.last_plan()}
if graph.value:
    hip.hipGraphDestroy(graph)
hip.hipStreamDestroy(stream)
print("RESULT " + json.dumps(out), flush=True)
'''


def test_noalloc_entry_allocates_nothing_under_capture():
    code = _SCRIPT % {"pkg": os.path.join(ROOT, "ml-edsl_amd")}
    p = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    print(p.stdout[-3000:], p.stderr[-3000:], flush=True)
    assert p.returncode == 0, p.stderr[-3000:]
    res = json.loads(next(line for line in p.stdout.splitlines() if line.startswith("RESULT "))[7:])
    for name in ("small_m_split_k", "tiled"):
        r = res[name]
        assert r["rc"] == 0 and r["end"] == 0, (name, r)
        assert r["same"] == [True, True], (name, r)
    assert "+fixed-scratch" in res["small_m_split_k"]["plan"], res["small_m_split_k"]
    ctl = res["control"]
    assert ctl["rc"] != 0 or ctl["end"] != 0, ("a hipMalloc under global capture was not refused", ctl)
