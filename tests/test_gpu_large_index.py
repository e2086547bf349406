"""Outputs beyond 2^31 elements: every kernel family indexes with 64-bit
offsets where a 32-bit product would overflow. Each case builds device
operands directly (8 GiB outputs, or 8 GiB weights for the small-M
streaming kernel), runs one launch through the C ABI,
and checks sampled rows / columns -- always including the last ones, where
the offsets are largest -- against the oracle on the same slices.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import assert_f32_parity
from mlir_edsl_hip import _native

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    return torch


def _rows(torch, M):
    return torch.from_numpy(np.unique(np.r_[0, 1, M // 2, M - 2, M - 1])).cuda()


def test_tiled_f32_output_beyond_2_31(torch_cuda):
    torch = torch_cuda
    from mlir_edsl_hip.device import dense_launch
    M, K, N = 65536, 64, 32768 + 256  # Y: 2.16e9 elements
    g = torch.Generator(device="cuda").manual_seed(5)
    X = torch.randn(M, K, device="cuda", generator=g)
    W = torch.randn(K, N, device="cuda", generator=g)
    b = torch.randn(N, device="cuda", generator=g)
    Y = torch.empty(M, N, device="cuda")
    dense_launch(X, W, b, Y, _native.EPI_BIAS_RELU)
    torch.cuda.synchronize()
    plan = _native.last_plan()
    assert plan.startswith("gemm_f32"), plan
    rows = _rows(torch, M)
    ref = oracle.dense_f32_chains(X.index_select(0, rows).cpu().numpy(), W.cpu().numpy(), b.cpu().numpy(), "relu")
    assert_f32_parity(Y.index_select(0, rows).cpu().numpy(), ref, K)
    del X, W, b, Y
    torch.cuda.empty_cache()


def test_int8_output_beyond_2_31(torch_cuda):
    torch = torch_cuda
    from mlir_edsl_hip.device import dense_launch
    M, K, N = 65536, 128, 32768 + 128
    g = torch.Generator(device="cuda").manual_seed(6)
    X = torch.randint(-128, 128, (M, K), device="cuda", dtype=torch.int32, generator=g)
    W = torch.randint(-128, 128, (K, N), device="cuda", dtype=torch.int32, generator=g)
    b = torch.randint(-2**20, 2**20, (N,), device="cuda", dtype=torch.int32, generator=g)
    Y = torch.empty(M, N, device="cuda", dtype=torch.int32)
    dense_launch(X, W, b, Y, _native.EPI_BIAS_RELU)
    torch.cuda.synchronize()
    plan = _native.last_plan()
    assert plan.startswith("narrow_i8+gemm_i8"), plan
    rows = _rows(torch, M)
    ref = oracle.dense_i32(X.index_select(0, rows).cpu().numpy(), W.cpu().numpy(), b.cpu().numpy(), "relu")
    assert np.array_equal(Y.index_select(0, rows).cpu().numpy(), ref)
    del X, W, b, Y
    torch.cuda.empty_cache()


def test_small_m_weights_beyond_2_31(torch_cuda):
    torch = torch_cuda
    from mlir_edsl_hip.device import dense_launch
    M, K, N = 16, 256, 2**23 + 128  # W: 2.15e9 elements
    g = torch.Generator(device="cuda").manual_seed(7)
    X = torch.randn(M, K, device="cuda", generator=g)
    W = torch.randn(K, N, device="cuda", generator=g)
    b = torch.randn(N, device="cuda", generator=g)
    Y = torch.empty(M, N, device="cuda")
    from mlir_edsl_hip.device import set_small_m
    set_small_m(1)  # K = 256 alone would give the layer to the tiles
    try:
        dense_launch(X, W, b, Y, _native.EPI_BIAS_RELU)
        torch.cuda.synchronize()
    finally:
        set_small_m(0)
    plan = _native.last_plan()
    assert plan.startswith("gemv_f32"), plan
    cols = torch.from_numpy(np.unique(np.r_[0, 1, 4096, N // 2, N - 129, N - 4, N - 1])).cuda()
    Wc = W.index_select(1, cols).cpu().numpy()
    ref = oracle.dense_f32_chains(X.cpu().numpy(), Wc, b.index_select(0, cols).cpu().numpy(), "relu")
    assert_f32_parity(Y.index_select(1, cols).cpu().numpy(), ref, K)
    del X, W, b, Y
    torch.cuda.empty_cache()
