"""Device entry points called from several streams at once. The small-M
split-K partials and the packed int8 operands are library scratch shared by
every call on a device; calls from different streams that would overlap on
the device must still give each caller its own result. Each launch is queued
behind a spin kernel on its stream, so the launches of the two streams
would start together if nothing ordered them."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import assert_f32_parity
from mlir_edsl_hip import _native
from mlir_edsl_hip.device import dense_launch

pytestmark = pytest.mark.gpu

SPIN_CYCLES = 200_000  # ~0.1 ms


def _problem(torch, rng, dtype, M, K, N):
    if dtype in ("f32", "f32s"):
        X = rng.standard_normal((M, K), dtype=np.float32)
        W = rng.standard_normal((K, N), dtype=np.float32)
        b = rng.standard_normal(N, dtype=np.float32)
        ref = oracle.dense_f32_chains(X, W, b, "relu")
    else:
        X = rng.integers(-128, 128, size=(M, K), dtype=np.int32)
        W = rng.integers(-128, 128, size=(K, N), dtype=np.int32)
        b = rng.integers(-2**20, 2**20, size=N, dtype=np.int32)
        ref = oracle.dense_i32(X, W, b, "relu")
    t = [torch.from_numpy(a).cuda() for a in (X, W, b)]
    Y = torch.full((M, N), -7, dtype=t[0].dtype, device="cuda")
    return t, Y, ref, K


# f32s: small M with K = 2047, so X rows are unaligned (read with 4-byte
# loads) and the reduce kernel adds a K tail
@pytest.mark.parametrize("kinds", [("f32", "f32"), ("i32", "i32"), ("f32", "i32"), ("f32s", "f32s"),
                                   ("f32s", "i32")])
def test_scratch_users_on_two_streams(kinds):
    import torch
    assert torch.cuda.is_available()
    rng = np.random.default_rng(11)
    shapes = {"f32": (16, 2048, 2048), "i32": (256, 384, 256), "f32s": (16, 2047, 2048)}
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    # four rounds, each stream gets its own problem every round
    probs = [[_problem(torch, rng, kinds[j], *shapes[kinds[j]]) for j in range(2)] for _ in range(4)]
    torch.cuda.synchronize()
    plans = set()
    for rnd in probs:
        for s, ((X, W, b), Y, _, _) in zip(streams, rnd):
            with torch.cuda.stream(s):
                torch.cuda._sleep(SPIN_CYCLES)
                dense_launch(X, W, b, Y, _native.EPI_BIAS_RELU, stream=s)
                plans.add(_native.last_plan())
    torch.cuda.synchronize()
    # both scratch users are exercised
    for k in set(kinds):
        want = {"f32": "ksplit=", "f32s": "+ktail", "i32": "narrow_i8+gemm_i8"}[k]
        assert any(want in p and ("ksplit=1 " not in p) for p in plans), plans
    for r, rnd in enumerate(probs):
        for j, (_, Y, ref, K) in enumerate(rnd):
            got = Y.cpu().numpy()
            if got.dtype == np.int32:
                assert np.array_equal(got, ref), f"round {r} stream {j}"
            else:
                assert_f32_parity(got, ref, K)


def test_launch_without_a_stream_uses_the_current_one():
    """dense_launch without a stream argument enqueues on torch's current
    stream, read through torch's raw-handle accessor: the same handle as
    torch.cuda.current_stream(), inside and outside a stream context."""
    import torch
    from mlir_edsl_hip import device
    device._torch_module()
    assert device._raw_stream() == torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(12)
    (X, W, b), Y, ref, K = _problem(torch, rng, "f32", 64, 256, 128)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        assert device._raw_stream() == s.cuda_stream
        torch.cuda._sleep(SPIN_CYCLES)
        dense_launch(X, W, b, Y, _native.EPI_BIAS_RELU)
        done = torch.cuda.Event()
        done.record()
    done.synchronize()
    assert_f32_parity(Y.cpu().numpy(), ref, K)
    assert device._raw_stream() == torch.cuda.current_stream().cuda_stream


def test_dense_launch_operand_errors_name_the_operand():
    import torch
    d = "cuda"
    X, W, b, Y = (torch.zeros(4, 8, device=d), torch.zeros(8, 16, device=d), torch.zeros(16, device=d),
                  torch.zeros(4, 16, device=d))
    cases = [
        ((X, W.int(), b, Y), TypeError, "W has dtype"),
        ((X, W, b, Y.cpu()), ValueError, "Y must be a GPU tensor"),
        ((X, torch.zeros(16, 8, device=d).t(), b, Y), ValueError, "W must have unit inner stride"),
        ((X, W, b, torch.zeros(4, 15, device=d)), ValueError, "shape mismatch"),
        ((X, torch.zeros(7, 16, device=d), b, Y), ValueError, "shape mismatch"),
        ((X, W, torch.zeros(15, device=d), Y), ValueError, "bias shape"),
        ((X, W, torch.zeros(32, device=d)[::2], Y), ValueError, "b must have unit inner stride"),
        ((X.reshape(4, 8, 1), W, b, Y), ValueError, "2-D"),
    ]
    for args, exc, msg in cases:
        with pytest.raises(exc, match=msg):
            dense_launch(*args, _native.EPI_BIAS_RELU)
    dense_launch(X, W, b, Y, _native.EPI_BIAS_RELU)  # the same operands, correct, still launch
    torch.cuda.synchronize()
    assert torch.equal(Y, torch.zeros_like(Y))
