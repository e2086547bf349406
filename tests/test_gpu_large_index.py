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


# The one-wave fp32 tiles address A and B through buffer descriptors with
# 32-bit byte offsets from the tile's first row (A) and first column (B); the
# planner gives them a layer only when 128 * lda * 4 + 64 and
# (K + 16) * ldb * 4 + 1024 fit in 2^31 - 1 (gemm_f32_direct_offsets_fit).
ONE_WAVE_TILES = ["f32_128x128x16_direct", "f32_128x128x16_direct_edge", "f32_64x64x16_direct",
                  "f32_64x64x64_direct_k4", "f32_64x64x64_direct_k4_edge", "f32_16x16x64_direct_k4",
                  "f32_32x32x64_direct_rc"]
LDA_LIMIT = (2**31 - 1 - 64) // 512 // 4 * 4          # 4,194,300 elements
LDB_LIMIT_K256 = (2**31 - 1 - 1024) // (272 * 4) // 4 * 4  # 1,973,788 elements at K = 256


def _one_wave_case(torch, lda, ldb, seed):
    """A 128 x 256 x 256 layer whose X (row pitch lda) or W (row pitch ldb) is a
    view into a ~2 GiB buffer filled with NaN past the operand's columns; run
    under each one-wave tile forced and under the automatic plan."""
    from mlir_edsl_hip.device import dense_launch, set_f32_config
    M, K, N = 128, 256, 256
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.float32(16.0)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, N).astype(np.float32)
    ref = oracle.dense_f32_chains(X, W, b, "relu")
    tX = torch.full((M, lda), float("nan"), device="cuda")[:, :K]
    tW = torch.full((K, ldb), float("nan"), device="cuda")[:, :N]
    tX.copy_(torch.from_numpy(X))
    tW.copy_(torch.from_numpy(W))
    tb = torch.from_numpy(b).cuda()
    names = _native.f32_config_names()
    plans = {}
    try:
        for name in ONE_WAVE_TILES + [None]:
            set_f32_config(names.index(name) if name else -1)
            tY = torch.full((M, N), float("nan"), device="cuda")
            dense_launch(tX, tW, tb, tY, _native.EPI_BIAS_RELU)
            torch.cuda.synchronize()
            plans[name] = _native.last_plan()
            assert_f32_parity(tY.cpu().numpy(), ref, K)
    finally:
        set_f32_config(-1)
    del tX, tW
    torch.cuda.empty_cache()
    return plans


@pytest.mark.parametrize("side", ["lda", "ldb"])
def test_one_wave_tiles_at_the_32_bit_offset_limit(side, torch_cuda):
    """At the largest row pitch the bound admits, each forced one-wave tile
    runs, its last rows read at byte offsets just under 2^31."""
    lda, ldb = (LDA_LIMIT, 256) if side == "lda" else (256, LDB_LIMIT_K256)
    plans = _one_wave_case(torch_cuda, lda, ldb, 31)
    for name in ONE_WAVE_TILES:
        assert f"cfg={name} " in plans[name], (name, plans[name])


@pytest.mark.parametrize("side", ["lda", "ldb"])
def test_one_wave_tiles_refused_past_the_32_bit_offset_limit(side, torch_cuda):
    """One row pitch step (4 elements) past the bound, a forced one-wave tile
    is not taken: the layer goes to a tile with 64-bit addressing."""
    lda, ldb = (LDA_LIMIT + 4, 256) if side == "lda" else (256, LDB_LIMIT_K256 + 4)
    plans = _one_wave_case(torch_cuda, lda, ldb, 32)
    for name, plan in plans.items():
        assert plan.startswith("gemm_f32"), plan
        assert "_direct" not in plan, (name, plan)
