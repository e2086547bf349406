"""Seeded random parity cases for the dense path through the C ABI.

Each case draws a shape (including K = 0 and sizes that are no multiple of
any tile; a second set draws multiples of 4 up to 1100 with 16-byte aligned
views, the shapes the edge tiles and padded int8 tiles serve), a dtype, a
pattern, host or device operands, and for device operands a padded row stride
and an element offset (a third set: small M with X misaligned on its own and K
often not a multiple of 16; a fourth: small M with W and Y misaligned on their
own, N often not a multiple of 4; a fifth: sizes 2048..4096, aligned or
not), then compares the HIP result with the
oracle: i32 bit-exact (int8-range values take the int8 MFMA path, wider ones
the exact i32 fallback), f32 within relative Frobenius 1e-5 and max|delta| <=
1e-4*sqrt(K).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import assert_f32_parity
from mlir_edsl_hip import _native
from mlir_edsl_hip.device import dense_launch

pytestmark = pytest.mark.gpu

_PATTERNS = {"matmul": (False, "none"), "matmul_relu": (False, "relu"), "matmul_bias": (True, "none"),
             "dense_relu": (True, "relu"), "dense_leaky": (True, "leaky")}
_EPI = {"none": 0, "relu": 1, "leaky": 2}


_SMALL_DIMS = [1, 2, 3, 7, 16, 17, 31, 32, 33, 63, 64, 65, 96, 127, 128, 129, 200, 256, 300]
# Multiples of 4 that divide no tile, up to 1100: with 16-byte aligned views
# these take the fp32 edge tiles, partial small-M column blocks and the padded
# int8 tiles on grids of many workgroups.
_EDGE_DIMS = [4, 8, 12, 20, 36, 60, 100, 132, 260, 500, 516, 1000, 1028, 1100]


def _case(seed, dims=_SMALL_DIMS, pads=(0, 0, 1, 3, 4, 9), offs=(0, 0, 1, 2, 4), k_zero=True):
    rng = np.random.default_rng(seed)
    M, N = (int(rng.choice(dims)) for _ in range(2))
    K = int(rng.choice(dims + [0] if k_zero else dims))
    dtype = "i32" if rng.random() < 0.4 else "f32"
    pats = [p for p in _PATTERNS if not (dtype == "i32" and p == "dense_leaky")]
    pattern = pats[int(rng.integers(len(pats)))]
    device = bool(rng.random() < 0.6)
    pad = int(rng.choice(list(pads))) if device else 0
    off = int(rng.choice(list(offs))) if device else 0
    wide = dtype == "i32" and rng.random() < 0.3
    return rng, M, K, N, dtype, pattern, device, pad, off, wide


def _draw(rng, shape, dtype, wide):
    if dtype == "f32":
        return rng.standard_normal(shape, dtype=np.float32)
    lim = 2**31 if wide else 128
    return rng.integers(-lim, lim, size=shape, dtype=np.int64).astype(np.int32)


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    return torch


def _device_view(torch, a, pad, off):
    """a copied to the device as a view with row stride cols + pad and an
    element offset off."""
    if a.ndim == 1:
        buf = torch.empty(a.shape[0] + off, dtype=torch.float32 if a.dtype == np.float32 else torch.int32,
                          device="cuda")
        v = buf[off:off + a.shape[0]]
        v.copy_(torch.from_numpy(a))
        return v
    rows, cols = a.shape
    buf = torch.empty(rows * (cols + pad) + off + 1, dtype=torch.float32 if a.dtype == np.float32 else torch.int32,
                      device="cuda")
    v = buf[off:off + rows * (cols + pad)].view(rows, cols + pad)[:, :cols]
    v.copy_(torch.from_numpy(a))
    return v


@pytest.mark.parametrize("seed", range(60))
def test_random_case(seed, torch_cuda):
    _check_case(seed, _case(seed), torch_cuda)


@pytest.mark.parametrize("seed", range(1000, 1040))
def test_random_edge_case(seed, torch_cuda):
    _check_case(seed, _case(seed, _EDGE_DIMS, pads=(0, 4, 8), offs=(0, 4), k_zero=False), torch_cuda)


# Layers of at least one 128x128 tile per CU, some 16-byte aligned, some not
# (odd pads and offsets). These seeds reach the 16x16-block tiles (64x64 edge,
# eight-wave 128x128 and the 128x128 any-shape twin), the 256x256 and 64x64
# any-shape tiles, the host pipeline's row chunks, and the padded int8 tiles
# with some tiles out of int8 range; the 128x256 and four-wave 128x128
# layouts are checked on fixed shapes in test_gpu_edge_tiles.py.
_LARGE_DIMS = [2048, 2052, 2100, 2176, 2500, 3000, 3072, 4000, 4096]


@pytest.mark.parametrize("seed", range(4000, 4016))
def test_random_large_case(seed, torch_cuda):
    _check_case(seed, _case(seed, _LARGE_DIMS, pads=(0, 0, 4, 1, 3), offs=(0, 0, 4, 1), k_zero=False),
                torch_cuda)


# Layers of whole 16-, 48-, 64-, 80- and 128-row tiles on 16-byte aligned
# views, fp32: the one-wave tiles of gemm_f32_direct.hip (16x16, 64x64 and
# R x C with K split over four waves, 64x64 unsplit, 128x128), each seed
# checked against the oracle and the set of seeds required to reach every one
# of them.
_ONE_WAVE_MN = [256, 320, 720, 768, 1024, 1088, 1440, 1536, 2048, 2560, 4096]
_ONE_WAVE_K = [64, 256, 448, 512, 1024, 1536]


def test_random_one_wave_tiles(torch_cuda):
    """24 seeds; EDSL_ONE_WAVE_SWEEP=N adds N more (progress every 100 with -s)."""
    import os
    extra = int(os.environ.get("EDSL_ONE_WAVE_SWEEP", "0"))
    plans = []
    for seed in range(5000, 5024 + extra):
        if seed >= 5024 and (seed - 5024) % 100 == 0:
            print(f"one-wave sweep: {seed - 5024} of {extra} extra seeds passed", flush=True)
        rng = np.random.default_rng(seed)
        M, N = (int(rng.choice(_ONE_WAVE_MN)) for _ in range(2))
        K = int(rng.choice(_ONE_WAVE_K))
        if seed == 5000:
            M, N, K = 256, 256, 256      # the 16x16 tile
        elif seed == 5001:
            M, N, K = 2048, 2048, 512    # 64x64 unsplit
        elif seed == 5002:
            M, N, K = 4096, 4096, 256    # 128x128
        elif seed == 5003:
            M, N, K = 768, 768, 768      # 48x48, K split four ways
        elif seed == 5004:
            M, N, K = 1200, 1200, 1024   # 80x80
        elif seed == 5005:
            M, N, K = 1536, 1536, 512    # 96x96
        pattern = list(_PATTERNS)[int(rng.integers(len(_PATTERNS)))]
        pad, off = ((0, 0), (4, 4), (8, 0))[seed % 3]
        case = (rng, M, K, N, "f32", pattern, True, pad, off, False)
        _check_case(seed, case, torch_cuda)
        plans.append(_native.last_plan())
    for tile in ("f32_16x16x64_direct_k4", "f32_64x64x64_direct_k4", "f32_64x64x16_direct ", "f32_128x128x16_direct ",
                 "f32_48x48x64_direct_rc", "f32_80x80x64_direct_rc", "f32_96x96x64_direct_rc"):
        assert any(tile in p + " " for p in plans), (tile, plans)


def _check_case(seed, case, torch):
    rng, M, K, N, dtype, pattern, device, pad, off, wide = case
    bias, act = _PATTERNS[pattern]
    X = _draw(rng, (M, K), dtype, wide)
    W = _draw(rng, (K, N), dtype, wide)
    b = _draw(rng, (N,), dtype, wide) if bias else None
    alpha = float(np.float32(rng.uniform(0.01, 0.5)))
    if dtype == "f32":
        ref = oracle.dense_f32_chains(X, W, b, act, alpha)
    else:
        ref = oracle.dense_i32(X, W, b, act)
    epi = (1 if bias else 0) | (_EPI[act] << 1)
    if device:
        tX, tW = _device_view(torch, X, pad, off), _device_view(torch, W, pad, off)
        tb = _device_view(torch, b, 0, off) if bias else None
        tY = _device_view(torch, np.zeros((M, N), X.dtype), pad, off)
        dense_launch(tX, tW, tb, tY, epi, alpha)
        torch.cuda.synchronize()
        got = tY.cpu().numpy()
    else:
        from mlir_edsl_hip import backend
        args = [X, W] + ([b] if bias else [])
        got = backend.run(pattern, *args, alpha=alpha)
    what = f"seed={seed} {dtype} {pattern} M={M} K={K} N={N} device={device} pad={pad} off={off} " \
           f"wide={wide} [{_native.last_plan()}]"
    if dtype == "i32":
        assert np.array_equal(got, ref), what
    else:
        try:
            assert_f32_parity(got, ref, K)
        except AssertionError as e:
            raise AssertionError(f"{what}: {e}") from None


# Small M with X's own row pad and element offset (often misaligned) while W,
# b and Y stay 16-byte aligned, and K often not a multiple of 16: the
# small-M kernel reading unaligned X rows in place and the K tail added by
# the reduce kernel, at one to four row blocks.
_SMALL_M = [1, 5, 16, 17, 32, 48, 64]
_SMALL_M_K = [1003, 2047, 4099, 4096, 8191]
_SMALL_M_N = [64, 1000, 1028, 2048, 4100]


def _check_small_m(seed, torch):
    rng = np.random.default_rng(seed)
    M, K, N = int(rng.choice(_SMALL_M)), int(rng.choice(_SMALL_M_K)), int(rng.choice(_SMALL_M_N))
    pattern = str(rng.choice(list(_PATTERNS)))
    bias, act = _PATTERNS[pattern]
    x_pad, x_off = int(rng.choice([0, 1, 2, 3, 5])), int(rng.choice([0, 1, 2, 3]))
    w_pad, w_off = int(rng.choice([0, 4])), int(rng.choice([0, 4]))
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.float32(np.sqrt(K))).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, N).astype(np.float32) if bias else None
    alpha = float(np.float32(rng.uniform(0.01, 0.5)))
    tX = _device_view(torch, X, x_pad, x_off)
    tW = _device_view(torch, W, w_pad, w_off)
    tb = _device_view(torch, b, 0, w_off) if bias else None
    tY = _device_view(torch, np.zeros((M, N), np.float32), w_pad, w_off)
    from mlir_edsl_hip.device import set_small_m
    set_small_m(1)  # aligned short-K layers would otherwise go to the tiles
    try:
        dense_launch(tX, tW, tb, tY, (1 if bias else 0) | (_EPI[act] << 1), alpha)
        torch.cuda.synchronize()
    finally:
        set_small_m(0)
    plan = _native.last_plan()
    what = f"seed={seed} {pattern} M={M} K={K} N={N} x_pad={x_pad} x_off={x_off} w_pad={w_pad} " \
           f"w_off={w_off} [{plan}]"
    assert plan.startswith("gemv_f32"), what
    try:
        assert_f32_parity(tY.cpu().numpy(), oracle.dense_f32_chains(X, W, b, act, alpha), K)
    except AssertionError as e:
        raise AssertionError(f"{what}: {e}") from None


@pytest.mark.parametrize("seed", range(2000, 2030))
def test_random_small_m_case(seed, torch_cuda):
    _check_small_m(seed, torch_cuda)


# Small M with W (and Y, which shares W's pitch and offset) misaligned by its
# own pad and offset, N not a multiple of 4 as often as not, and W large
# enough that the plan streams it realigned (or per column) through the
# small-M kernel rather than the any-shape tile.
_UW_M = [1, 3, 16, 17, 33, 48, 64]
_UW_K = [1003, 2047, 2048, 4099, 8191]
_UW_N = [1001, 2047, 2048, 4097, 4100, 8191]


def _check_small_m_unaligned_w(seed, torch):
    rng = np.random.default_rng(seed)
    M, K, N = int(rng.choice(_UW_M)), int(rng.choice(_UW_K)), int(rng.choice(_UW_N))
    pattern = str(rng.choice(list(_PATTERNS)))
    bias, act = _PATTERNS[pattern]
    x_pad, x_off = int(rng.choice([0, 1, 4])), int(rng.choice([0, 2]))
    w_pad, w_off = int(rng.choice([0, 1, 2, 3, 5])), int(rng.choice([0, 1, 2, 3]))
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.float32(np.sqrt(K))).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, N).astype(np.float32) if bias else None
    alpha = float(np.float32(rng.uniform(0.01, 0.5)))
    tX = _device_view(torch, X, x_pad, x_off)
    tW = _device_view(torch, W, w_pad, w_off)
    tb = _device_view(torch, b, 0, w_off) if bias else None
    tY = _device_view(torch, np.zeros((M, N), np.float32), w_pad, w_off)
    dense_launch(tX, tW, tb, tY, (1 if bias else 0) | (_EPI[act] << 1), alpha)
    torch.cuda.synchronize()
    what = f"seed={seed} {pattern} M={M} K={K} N={N} x_pad={x_pad} x_off={x_off} w_pad={w_pad} " \
           f"w_off={w_off} [{_native.last_plan()}]"
    try:
        assert_f32_parity(tY.cpu().numpy(), oracle.dense_f32_chains(X, W, b, act, alpha), K)
    except AssertionError as e:
        raise AssertionError(f"{what}: {e}") from None
    return _native.last_plan()


def test_random_small_m_unaligned_w_cases(torch_cuda):
    plans = [_check_small_m_unaligned_w(seed, torch_cuda) for seed in range(3000, 3040)]
    # The seeds reach the realigned small-M kernel, its 4-byte column loads
    # and the any-shape tile.
    assert any("+wrealigned" in p for p in plans), plans
    assert any("_anyshape" in p for p in plans), plans


def test_random_sweep(torch_cuda):
    """Opt-in wide sweep: EDSL_RANDOM_SWEEP=N runs N more seeds of both case
    sets (and two small-M cases, aligned and misaligned W, every tenth seed)
    in this one test. N = 20000
    takes about eleven minutes on one MI355X; run it with -s to see a
    progress line every 1000 seeds."""
    import os
    n = int(os.environ.get("EDSL_RANDOM_SWEEP", "0"))
    if n <= 0:
        pytest.skip("set EDSL_RANDOM_SWEEP=N to run N more seeds")
    for seed in range(10000, 10000 + n):
        _check_case(seed, _case(seed), torch_cuda)
        _check_case(seed, _case(seed, _EDGE_DIMS, pads=(0, 4, 8), offs=(0, 4), k_zero=False), torch_cuda)
        if seed % 10 == 0:
            _check_small_m(seed, torch_cuda)
        if seed % 10 == 5:
            _check_small_m_unaligned_w(seed, torch_cuda)
        if (seed - 9999) % 1000 == 0:  # progress, visible with pytest -s
            print(f"random sweep: {seed - 9999} of {n} seeds passed", flush=True)
