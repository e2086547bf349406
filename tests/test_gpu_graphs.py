"""Device entry points captured into HIP graphs (torch.cuda.CUDAGraph) and
replayed. Each replay follows eager work of the program's own (an eager run
of the same layers on new inputs, which uses the same library workspaces)
and a synchronisation, and its outputs must equal that eager run bit for bit:
the captured kernels, plans and summation orders are the eager ones. One
more replay follows eager calls large enough to grow every workspace: the
graph keeps the buffers it was captured with.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import assert_f32_parity
from mlir_edsl_hip import _native
from mlir_edsl_hip.device import dense_launch

pytestmark = pytest.mark.gpu


def _layer(torch, g, dtype, M, K, N, epi):
    if dtype == "f32":
        W = torch.randn(K, N, device="cuda", generator=g) / K ** 0.5
        b = torch.randn(N, device="cuda", generator=g)
    else:
        W = torch.randint(-128, 128, (K, N), device="cuda", dtype=torch.int32, generator=g)
        b = torch.randint(-2**20, 2**20, (N,), device="cuda", dtype=torch.int32, generator=g)
    return W, b, epi


def _inputs(torch, g, dtype, M, K):
    if dtype == "f32":
        return torch.randn(M, K, device="cuda", generator=g)
    return torch.randint(-128, 128, (M, K), device="cuda", dtype=torch.int32, generator=g)


# (name, dtype, M, layer widths, epilogues, plan prefixes): a chain of dense
# layers, each layer's output the next one's input
CASES = [
    ("tiled_f32_chain", "f32", 512, [384, 512, 256, 320], [3, 3, 0], ["gemm_f32"] * 3),
    ("small_m_split_k", "f32", 16, [4096, 2048, 1024], [3, 1], ["gemv_f32"] * 2),
    # K = 4099: X rows copied to aligned rows, then a 3-row K tail; K = 2052: a 4-row tail
    ("small_m_staged_tail", "f32", 16, [4099, 2052, 1028], [3, 1], ["gemv_f32"] * 2),
    ("int8_path", "i32", 256, [384, 256, 512], [3, 3], ["narrow_i8+gemm_i8"] * 2),
]


@pytest.mark.parametrize("name, dtype, M, widths, epis, plans", CASES, ids=[c[0] for c in CASES])
def test_graph_replay_matches_eager(name, dtype, M, widths, epis, plans):
    import torch
    assert torch.cuda.is_available()
    g = torch.Generator(device="cuda").manual_seed(21)
    layers = [_layer(torch, g, dtype, M, widths[i], widths[i + 1], epis[i]) for i in range(len(epis))]
    tdt = torch.float32 if dtype == "f32" else torch.int32
    X = _inputs(torch, g, dtype, M, widths[0])
    outs = [torch.empty(M, widths[i + 1], dtype=tdt, device="cuda") for i in range(len(epis))]
    eager_outs = [torch.empty_like(o) for o in outs]

    def chain(x, ys):
        for (W, b, epi), y in zip(layers, ys):
            dense_launch(x, W, b, y, epi)
            x = y

    chain(X, outs)  # warm-up: sizes the workspaces before capture
    got_plans = []
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            chain(X, outs)
            got_plans.append(_native.last_plan())
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert got_plans[0].startswith(plans[-1]), got_plans

    def grow_workspaces():
        # eager calls with larger shapes than any captured one: every
        # workspace of the device entry points is reallocated
        big = torch.randn(64, 8192, device="cuda", generator=g)
        Wb = torch.randn(8192, 8192, device="cuda", generator=g)
        yb = torch.empty(64, 8192, device="cuda")
        from mlir_edsl_hip.device import set_small_m
        set_small_m(1)  # four row blocks at K = N go to the tiles by default
        try:
            dense_launch(big, Wb, None, yb, 0)
        finally:
            set_small_m(0)
        assert "ksplit=" in _native.last_plan() and "ksplit=1 " not in _native.last_plan()
        xo = torch.randn(64, 8191, device="cuda", generator=g)  # unaligned rows and a K tail
        dense_launch(xo, Wb[:8191], None, yb, 0)
        assert "+xunaligned" in _native.last_plan() and "+ktail" in _native.last_plan()
        xi = torch.randint(-128, 128, (2048, 2048), device="cuda", dtype=torch.int32, generator=g)
        yi = torch.empty(2048, 2048, device="cuda", dtype=torch.int32)
        dense_launch(xi, xi, None, yi, 0)
        assert _native.last_plan().startswith("narrow_i8+gemm_i8")

    for rep in range(4):
        if rep == 3:
            grow_workspaces()
        X.copy_(_inputs(torch, g, dtype, M, widths[0]))
        chain(X, eager_outs)  # eager work between replays, same workspaces
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager_outs)):
            assert torch.equal(o, e), f"{name}: replay {rep}, layer {i}"
    # and the chain itself is right: last layer against the oracle from the
    # eager previous layer's output (float path) or exactly (integer path)
    prev = (X if len(layers) == 1 else eager_outs[-2]).cpu().numpy()
    W, b, epi = layers[-1]
    act = "relu" if epi in (2, 3) else "none"
    bias = b.cpu().numpy() if epi in (1, 3) else None
    if dtype == "f32":
        assert_f32_parity(outs[-1].cpu().numpy(), oracle.dense_f32_chains(prev, W.cpu().numpy(), bias, act), W.shape[0])
    else:
        assert np.array_equal(outs[-1].cpu().numpy(), oracle.dense_i32(prev, W.cpu().numpy(), bias, act))


def _exact_i32(X, W, b):
    y = X.astype(np.int64) @ W.astype(np.int64) + b.astype(np.int64)
    return np.maximum((y + 2**31) % 2**32 - 2**31, 0).astype(np.int32)


def test_int8_range_flags_on_replay():
    """A captured integer layer replayed on inputs that leave int8 and come
    back: out of range, in range, out of range (elsewhere), in range. The
    narrowing pass rewrites every tile's range flag on every call, so each
    replay is exact and none inherits the previous one's fallback."""
    import torch
    M, K, N = 512, 384, 256
    rng = np.random.default_rng(33)
    W = rng.integers(-128, 128, size=(K, N), dtype=np.int32)
    b = rng.integers(-2**20, 2**20, size=(N,), dtype=np.int32)
    tW, tb = torch.from_numpy(W).cuda(), torch.from_numpy(b).cuda()
    tX = torch.zeros((M, K), dtype=torch.int32, device="cuda")
    tY = torch.empty((M, N), dtype=torch.int32, device="cuda")
    good = rng.integers(-128, 128, size=(M, K), dtype=np.int32)
    bad1 = good.copy()
    bad1[3, 5] = 70000          # first 128-row tile only
    bad2 = good.copy()
    bad2[400, 380] = -300       # last row tile, last k tile
    bad2[130, 0] = 2**30        # second row tile
    tX.copy_(torch.from_numpy(good))
    dense_launch(tX, tW, tb, tY, _native.EPI_BIAS_RELU)  # sizes the workspaces
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            dense_launch(tX, tW, tb, tY, _native.EPI_BIAS_RELU)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for step, Xv in enumerate((bad1, good, bad2, good, bad1)):
        tX.copy_(torch.from_numpy(Xv))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(tY.cpu().numpy(), _exact_i32(Xv, W, b)), f"replay {step}"
