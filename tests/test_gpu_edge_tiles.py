"""GPU parity for shapes that are not multiples of the tile.

The fp32 tiles have edge variants (partial tiles at the M, N and K edges,
16-byte vector loads at clamped addresses, masked stores) for 16-byte aligned
operands whose K, N and row strides are multiples of 4, and any-shape variants
(element-checked 4-byte loads and stores) for every other layout; the small-M kernel
spreads K over its wave slices in 16-row chunks, so K need only be a multiple
of 16, and its last column block may be partial, so N need only be a multiple
of 4. Every case is checked against the oracle on the full output.
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


def _inputs(M, K, N, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.float32(np.sqrt(K))).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, N).astype(np.float32)
    return X, W, b


def _view(torch, a, pad=0, off=0):
    """Device copy of `a` as a view with row pitch cols + pad, `off` elements in."""
    rows, cols = a.shape
    buf = torch.zeros(rows * (cols + pad) + off, dtype=torch.float32, device="cuda")
    v = buf[off:].view(rows, cols + pad)[:, :cols]
    v.copy_(torch.from_numpy(a))
    return v


def _run(torch, X, W, b, pad=0, off=0):
    from mlir_edsl_hip.device import dense_launch
    M, N = X.shape[0], W.shape[1]
    tX, tW = _view(torch, X, pad, off), _view(torch, W, pad, off)
    tb = torch.from_numpy(b).cuda()
    tY = _view(torch, np.full((M, N), np.nan, dtype=np.float32), pad, off)
    dense_launch(tX, tW, tb, tY, _native.EPI_BIAS_RELU)
    torch.cuda.synchronize()
    return tY.cpu().numpy(), _native.last_plan()


# M > 64 or K < 16 throughout: smaller M with K >= 16 takes the small-M kernel.
EDGE_SHAPES = [(300, 100, 260), (257, 68, 132), (65, 20, 36), (97, 1000, 1028), (1, 4, 4)]


def test_every_edge_config_on_odd_shapes(torch_cuda):
    from mlir_edsl_hip.device import set_f32_config
    names = _native.f32_config_names()
    edge = [(c, n) for c, n in enumerate(names) if n.endswith("_edge")]
    assert len(edge) >= 5
    try:
        for cfg, name in edge:
            set_f32_config(cfg)
            for i, (M, K, N) in enumerate(EDGE_SHAPES):
                X, W, b = _inputs(M, K, N, 100 + i)
                ref = oracle.dense_f32_chains(X, W, b, "relu")
                # contiguous, then a padded row pitch with an element offset
                # (both keep 16-byte aligned rows)
                for pad, off in ((0, 0), (8, 4)):
                    got, plan = _run(torch_cuda, X, W, b, pad, off)
                    assert name in plan, (name, plan)
                    assert_f32_parity(got, ref, K)
    finally:
        set_f32_config(-1)


@pytest.mark.parametrize("shape, tile", [
    ((1000, 1000, 1000), "f32_64x64x64_direct_k4_edge"),
    ((4000, 256, 4000), "f32_128x128x16_direct_edge"),
    # 33 x 32 tiles of 128x128 would give 32 CUs a fifth tile
    ((4097, 256, 4096), "f32_64x64x64_mfma16_edge"),
    # K = 1000 leaves a partial last K step on every tile
    ((512, 1000, 512), "f32_32x32x64_direct_rc_edge"),
], ids=["1000^3", "4000x256x4000", "4097x256x4096", "512x1000x512"])
def test_auto_plan_takes_edge_tiles(shape, tile, torch_cuda):
    M, K, N = shape
    X, W, b = _inputs(M, K, N, M + K + N)
    got, plan = _run(torch_cuda, X, W, b)
    assert f"cfg={tile} " in plan, plan
    assert_f32_parity(got, oracle.dense_f32_chains(X, W, b, "relu"), K)


def test_aligned_shapes_keep_their_tiles(torch_cuda):
    """Shapes the tiles divide still take the unguarded configurations."""
    for (M, K, N), tile in (((1024, 1024, 1024), "f32_64x64x64_direct_rc"),
                            ((2048, 2048, 2048), "f32_64x64x16_direct"),
                            ((4096, 1024, 4096), "f32_128x128x16_direct"),
                            ((3072, 512, 3072), "f32_64x64x64_direct_k4"),
                            ((2048, 128, 2048), "f32_128x128x32_mfma16_w8"),
                            ((1024, 128, 1024), "f32_64x64x64_mfma16"),
                            ((256, 256, 256), "f32_16x16x64_direct_k4"),
                            ((512, 512, 512), "f32_32x32x64_direct_rc"),
                            ((768, 768, 768), "f32_48x48x64_direct_rc"),
                            ((1536, 512, 1536), "f32_96x96x64_direct_rc")):
        X, W, b = _inputs(M, K, N, 7)
        got, plan = _run(torch_cuda, X, W, b)
        assert f"cfg={tile} " in plan, plan
        assert_f32_parity(got, oracle.dense_f32_chains(X, W, b, "relu"), K)


def test_unaligned_k_takes_an_any_shape_tile(torch_cuda):
    """K not a multiple of 4 leaves rows unaligned: an element-checked tile."""
    X, W, b = _inputs(70, 37, 50, 9)
    got, plan = _run(torch_cuda, X, W, b)
    assert "anyshape" in plan, plan
    assert_f32_parity(got, oracle.dense_f32_chains(X, W, b, "relu"), 37)


# K and N of every residue mod 4, M past and below the tiles; with an odd row
# pitch and an element offset no row is 16-byte aligned.
ODD_SHAPES = [(300, 101, 259), (257, 37, 133), (65, 3, 7), (97, 1001, 1029), (1, 1, 1), (130, 2002, 66)]


def test_every_any_shape_config_on_odd_shapes(torch_cuda):
    from mlir_edsl_hip.device import set_f32_config
    names = _native.f32_config_names()
    anyshape = [(c, n) for c, n in enumerate(names) if n.endswith("_anyshape")]
    assert len(anyshape) == 5
    try:
        for cfg, name in anyshape:
            set_f32_config(cfg)
            for i, (M, K, N) in enumerate(ODD_SHAPES):
                X, W, b = _inputs(M, K, N, 200 + i)
                ref = oracle.dense_f32_chains(X, W, b, "relu")
                for pad, off in ((0, 0), (3, 1)):
                    got, plan = _run(torch_cuda, X, W, b, pad, off)
                    assert name in plan, (name, plan, (M, K, N))
                    assert_f32_parity(got, ref, K)
    finally:
        set_f32_config(-1)


@pytest.mark.parametrize("shape, pad_off, tile", [
    ((2001, 2001, 2001), (0, 0), "f32_128x128x32_mfma16_anyshape"),
    ((1025, 1025, 1025), (0, 0), "f32_64x64x64_w2x2_k2_pf2_anyshape"),
    # K = N = 2048 but every row misaligned by an element offset
    ((2048, 2048, 2048), (0, 1), "f32_128x128x32_mfma16_anyshape"),
    ((4001, 1001, 4001), (0, 0), "f32_256x256x16_w4x4_anyshape"),
], ids=["2001^3", "1025^3", "2048^3-offset", "4001x1001x4001"])
def test_auto_plan_takes_any_shape_tiles(shape, pad_off, tile, torch_cuda):
    M, K, N = shape
    X, W, b = _inputs(M, K, N, M + 3 * K + N)
    got, plan = _run(torch_cuda, X, W, b, *pad_off)
    assert f"cfg={tile} " in plan, plan
    assert_f32_parity(got, oracle.dense_f32_chains(X, W, b, "relu"), K)


def _run_small_m(torch, X, W, b, pad=0, off=0):
    """_run with the small-M kernel taken wherever it can plan the layer (the
    automatic choice gives short-K layers to the tiles)."""
    from mlir_edsl_hip.device import set_small_m
    set_small_m(1)
    try:
        return _run(torch, X, W, b, pad, off)
    finally:
        set_small_m(0)


@pytest.mark.parametrize("M, K, N", [(16, 8000, 8192), (16, 8000, 1024), (3, 4112, 2048), (40, 1040, 512)])
def test_small_m_uneven_k_slices(M, K, N, torch_cuda):
    X, W, b = _inputs(M, K, N, M * 3 + K)
    got, plan = _run_small_m(torch_cuda, X, W, b)
    assert plan.startswith("gemv_f32"), plan
    assert_f32_parity(got, oracle.dense_f32_chains(X, W, b, "relu"), K)


# Small M with W, Y and bias rows that are not 16-byte aligned or N not a
# multiple of 4: W realigned from two 16-byte chunks per row (N >= 4, four
# columns per lane) or read per column, Y and the bias per element, columns
# past N never stored; the last row of W and any odd K go through the reduce
# kernel's tail. One to four row blocks, each column width the plan picks,
# contiguous and misaligned views (pad 0 puts W's last element at the end of
# its buffer).
@pytest.mark.parametrize("M, K, N", [(16, 8192, 8191), (16, 4096, 5003), (5, 1003, 1029), (64, 2048, 1023),
                                     (33, 512, 7), (1, 512, 3), (48, 4096, 4097)])
def test_small_m_unaligned_w(M, K, N, torch_cuda):
    """The automatic plan (the small-M kernel or the 32x32 any-shape tile,
    whichever measured faster for the shape), then the small-M kernel itself
    under a forced split of 2."""
    from mlir_edsl_hip.device import set_gemv_ksplit
    X, W, b = _inputs(M, K, N, M * 7 + K + N)
    ref = oracle.dense_f32_chains(X, W, b, "relu")
    for pad, off in ((0, 0), (3, 1)):
        got, plan = _run(torch_cuda, X, W, b, pad, off)
        assert "+wunaligned" in plan or "+wrealigned" in plan or "32x32x64" in plan, plan
        assert_f32_parity(got, ref, K)
        try:
            set_gemv_ksplit(2)
            got, plan = _run(torch_cuda, X, W, b, pad, off)
        finally:
            set_gemv_ksplit(0)
        assert plan.startswith("gemv_f32") and "ksplit=2" in plan, plan
        assert ("+wrealigned" if N >= 4 and "cols=32 " not in plan else "+wunaligned") in plan, plan
        assert_f32_parity(got, ref, K)


# Realigned W rows at every offset of a row within its 16-byte chunk: row
# pitches N + pad and element offsets chosen so that the offset of row k
# cycles with k when the pitch is odd; N such that the last lane of a lane
# group (the one that loads its own second chunk) holds a column below N,
# straddles N or lies past it, on every column width; one to three row blocks
# (second chunk from the neighbouring lane) and four (both chunks loaded by
# every lane). K = 1029: the last rows, the last one always, go to the tail.
@pytest.mark.parametrize("cols", [64, 128, 256])
@pytest.mark.parametrize("M", [1, 17, 40, 64])
def test_realigned_w_rows(M, cols, torch_cuda):
    from mlir_edsl_hip.device import set_gemv_cols, set_gemv_ksplit
    K = 1029
    checked = 0
    for N in (5, 61, 62, 63, 64 + 58, 64 + 60, 128 + 1, 128 + 63, 256 + 2, 256 + 62, 511):
        X, W, b = _inputs(M, K, N, M * 1000 + N)
        ref = oracle.dense_f32_chains(X, W, b, "relu")
        for pad, off in ((0, 0), (1, 0), (2, 1), (3, 3), (0, 2)):
            try:
                set_gemv_cols(cols)
                set_gemv_ksplit(2)
                got, plan = _run(torch_cuda, X, W, b, pad, off)
            finally:
                set_gemv_ksplit(0)
                set_gemv_cols(0)
            what = f"M={M} K={K} N={N} pad={pad} off={off} [{plan}]"
            vector_rows = N % 4 == 0 and pad % 4 == 0 and off % 4 == 0
            assert plan.startswith("gemv_f32") and f"cols={cols} " in plan, what
            assert ("+wrealigned" in plan) != vector_rows, what
            try:
                assert_f32_parity(got, ref, K)
            except AssertionError as e:
                raise AssertionError(f"{what}: {e}") from None
            checked += 1
    assert checked == 55


# The automatic choice between the small-M kernel and the tiles for aligned
# operands: short K goes to the tiles (32x32 tiles read W once up to 32 rows,
# twice up to 64), long K to the small-M kernel.
@pytest.mark.parametrize("M, K, N, kernel", [
    (16, 512, 512, "gemv_f32"), (1, 256, 256, "gemm_f32"), (16, 256, 4096, "gemm_f32"),
    (32, 2048, 1024, "gemv_f32"), (32, 512, 512, "gemm_f32"), (48, 2048, 2048, "gemv_f32"),
    (48, 1024, 4096, "gemm_f32"), (64, 256, 256, "gemm_f32"), (64, 4096, 1024, "gemv_f32"),
    (64, 4096, 8192, "gemv_f32"), (64, 2048, 8192, "gemm_f32"), (64, 2048, 2048, "gemm_f32"),
])
def test_auto_choice_small_m_or_tile(M, K, N, kernel, torch_cuda):
    X, W, b = _inputs(M, K, N, M + 5 * K + N)
    got, plan = _run(torch_cuda, X, W, b)
    assert plan.startswith(kernel), plan
    assert_f32_parity(got, oracle.dense_f32_chains(X, W, b, "relu"), K)


def test_small_m_forced_splits_on_uneven_k(torch_cuda):
    from mlir_edsl_hip.device import set_gemv_cols, set_gemv_ksplit
    M, K, N = 16, 8000, 1024
    X, W, b = _inputs(M, K, N, 5)
    ref = oracle.dense_f32_chains(X, W, b, "relu")
    try:
        set_gemv_cols(128)
        for ks in (1, 2, 3, 5, 16):
            set_gemv_ksplit(ks)
            got, plan = _run(torch_cuda, X, W, b)
            assert f"ksplit={ks} cols=128" in plan, plan
            assert_f32_parity(got, ref, K)
    finally:
        set_gemv_ksplit(0)
        set_gemv_cols(0)


@pytest.mark.parametrize("M, K, N", [(16, 4096, 50256), (16, 8192, 8100), (8, 4096, 4100), (1, 4096, 1000),
                                     (33, 1040, 36), (64, 2048, 4)])
def test_small_m_partial_column_blocks(M, K, N, torch_cuda):
    """N a multiple of 4 but not of the column block: the last block is
    partial (its lanes read the last columns and store nothing)."""
    X, W, b = _inputs(M, K, N, M + K + N)
    got, plan = _run_small_m(torch_cuda, X, W, b)
    assert plan.startswith("gemv_f32"), plan
    assert_f32_parity(got, oracle.dense_f32_chains(X, W, b, "relu"), K)


def test_small_m_every_width_on_a_partial_block(torch_cuda):
    from mlir_edsl_hip.device import set_gemv_cols, set_gemv_ksplit
    M, K, N = 16, 8000, 1000
    X, W, b = _inputs(M, K, N, 11)
    ref = oracle.dense_f32_chains(X, W, b, "relu")
    try:
        for cols in (32, 64, 128, 256):
            for ks in (1, 3):
                set_gemv_cols(cols)
                set_gemv_ksplit(ks)
                got, plan = _run(torch_cuda, X, W, b, 8, 4)
                assert f"ksplit={ks} cols={cols}" in plan, plan
                assert_f32_parity(got, ref, K)
    finally:
        set_gemv_ksplit(0)
        set_gemv_cols(0)


def _run_x_view(torch, X, W, b, x_pad, x_off, ksplit=None, epi=_native.EPI_BIAS_RELU, alpha=0.0):
    """Only X is a (possibly misaligned) view; W, b and Y are contiguous."""
    from mlir_edsl_hip.device import dense_launch, set_gemv_ksplit
    M, K = X.shape
    N = W.shape[1]
    buf = torch.zeros(M * (K + x_pad) + x_off, dtype=torch.float32, device="cuda")
    tX = buf[x_off:].view(M, K + x_pad)[:, :K]
    tX.copy_(torch.from_numpy(X))
    tW, tb = torch.from_numpy(W).cuda(), torch.from_numpy(b).cuda()
    tY = torch.full((M, N), float("nan"), device="cuda")
    if ksplit is not None:
        set_gemv_ksplit(ksplit)
    try:
        dense_launch(tX, tW, tb if epi & 1 else None, tY, epi, alpha)
        torch.cuda.synchronize()
    finally:
        set_gemv_ksplit(0)
    return tY.cpu().numpy(), _native.last_plan()


@pytest.mark.parametrize("M, K, N, x_pad, x_off, tags", [
    (16, 8191, 8192, 0, 0, ("+xunaligned", "+ktail")),   # contiguous X, odd K: unaligned rows
    (16, 8192, 2048, 0, 1, ("+xunaligned",)),             # misaligned X base, K % 16 == 0
    (33, 4100, 512, 0, 0, ("+ktail",)),                   # aligned X, K % 16 == 4
    (5, 1003, 1024, 2, 3, ("+xunaligned", "+ktail")),
], ids=["odd-K", "misaligned-X", "aligned-tail", "both"])
def test_small_m_k_tail_and_unaligned_x(M, K, N, x_pad, x_off, tags, torch_cuda):
    X, W, b = _inputs(M, K, N, M + K + N)
    got, plan = _run_x_view(torch_cuda, X, W, b, x_pad, x_off)
    assert plan.startswith("gemv_f32"), plan
    for t in tags:
        assert t in plan, plan
    if "+ktail" not in tags:
        assert "+ktail" not in plan, plan
    assert_f32_parity(got, oracle.dense_f32_chains(X, W, b, "relu"), K)


_TAIL_EPIS = {"none": (_native.EPI_NONE, None, "none"), "bias": (_native.EPI_BIAS, "b", "none"),
              "leaky": (_native.EPI_BIAS_LEAKY, "b", "leaky"), "relu_nobias": (_native.EPI_RELU, None, "relu")}


@pytest.mark.parametrize("epi_name", sorted(_TAIL_EPIS))
@pytest.mark.parametrize("M", [1, 32, 64])
@pytest.mark.parametrize("K, x_pad, x_off", [(2047, 0, 0), (4099, 3, 1), (1003, 0, 2)],
                         ids=["odd-K", "padded-offset", "offset"])
def test_small_m_tail_and_unaligned_x_per_row_block_and_epilogue(M, K, x_pad, x_off, epi_name, torch_cuda):
    """Unaligned X rows (read with 4-byte loads) and the K tail for one, two
    and four row blocks, with every epilogue the reduce kernel applies after
    adding the tail."""
    epi, use_b, act = _TAIL_EPIS[epi_name]
    N = 1024
    X, W, b = _inputs(M, K, N, 7 * M + K)
    got, plan = _run_x_view(torch_cuda, X, W, b, x_pad, x_off, epi=epi, alpha=0.05)
    assert plan.startswith(f"gemv_f32 mb={(M + 15) // 16}"), plan
    assert "+ktail" in plan and "+xunaligned" in plan, plan
    ref = oracle.dense_f32_chains(X, W, b if use_b else None, act, 0.05)
    assert_f32_parity(got, ref, K)


@pytest.mark.parametrize("K", [8191, 1001, 4096])
def test_single_row_x_with_any_row_stride(K, torch_cuda):
    """A (1, K) view of a column vector has row stride 1 (and a broadcast view
    0): with a single row the stride is never used, so any value must work."""
    from mlir_edsl_hip.device import dense_launch
    N = 2048
    X, W, b = _inputs(1, K, N, K)
    tX = torch_cuda.from_numpy(np.ascontiguousarray(X.reshape(K, 1))).cuda().T  # shape (1, K), strides (1, 1)
    assert tX.stride() == (1, 1)
    tW, tb = torch_cuda.from_numpy(W).cuda(), torch_cuda.from_numpy(b).cuda()
    tY = torch_cuda.full((1, N), float("nan"), device="cuda")
    dense_launch(tX, tW, tb, tY, _native.EPI_BIAS_RELU)
    torch_cuda.cuda.synchronize()
    assert _native.last_plan().startswith("gemv_f32"), _native.last_plan()
    assert_f32_parity(tY.cpu().numpy(), oracle.dense_f32_chains(X, W, b, "relu"), K)
    # Row stride 0 through the C ABI directly (torch reports the view's own
    # stride; a broadcast (1, K) row from expand() has stride 0 on dim 0).
    tY2 = torch_cuda.full((1, N), float("nan"), device="cuda")
    rc = _native.lib().edsl_hip_dense_f32_launch(tX.data_ptr(), 0, tW.data_ptr(), N, tb.data_ptr(),
                                                 tY2.data_ptr(), 0, 1, N, K, _native.EPI_BIAS_RELU, 0.0,
                                                 torch_cuda.cuda.current_stream().cuda_stream)
    assert rc == 0, _native.last_error()
    torch_cuda.cuda.synchronize()
    assert np.array_equal(tY2.cpu().numpy(), tY.cpu().numpy())


def test_small_m_k_tail_forces_the_reduce(torch_cuda):
    """A forced single split becomes two when there is a K tail: the reduce
    kernel adds the tail rows."""
    X, W, b = _inputs(16, 4100, 1024, 3)
    got, plan = _run_x_view(torch_cuda, X, W, b, 0, 0, ksplit=1)
    assert "ksplit=2" in plan and "+ktail" in plan, plan
    assert_f32_parity(got, oracle.dense_f32_chains(X, W, b, "relu"), 4100)


# ------------------------------------------------------------ integer path
# The int8 path pads its packed copies with zeros to multiples of 128 in M, N
# and K, so every shape runs on the matrix cores; results must equal the exact
# wrapping i32 sums.
def _exact_i32(X, W, b):
    y = X.astype(np.int64) @ W.astype(np.int64) + b.astype(np.int64)
    y = (y + 2**31) % 2**32 - 2**31
    return np.maximum(y, 0).astype(np.int32)


@pytest.mark.parametrize("M, K, N", [(1, 1, 1), (130, 129, 131), (257, 300, 129), (1000, 1000, 1000),
                                     (2000, 2000, 200)])
def test_int8_path_on_odd_shapes(M, K, N, torch_cuda):
    from mlir_edsl_hip.device import dense_launch, set_i8_variant
    rng = np.random.default_rng(M + 3 * K + 7 * N)
    X = rng.integers(-128, 128, size=(M, K), dtype=np.int32)
    W = rng.integers(-128, 128, size=(K, N), dtype=np.int32)
    b = rng.integers(-2**20, 2**20, size=(N,), dtype=np.int32)
    exp = _exact_i32(X, W, b)
    tX, tW, tb = (torch_cuda.from_numpy(a).cuda() for a in (X, W, b))
    n = _native.lib().edsl_hip_i8_variant_count()
    try:
        for v in range(n):
            set_i8_variant(v)
            tY = torch_cuda.full((M, N), -7, dtype=torch_cuda.int32, device="cuda")
            dense_launch(tX, tW, tb, tY, _native.EPI_BIAS_RELU)
            torch_cuda.cuda.synchronize()
            plan = _native.last_plan()
            assert plan.startswith(f"narrow_i8+gemm_i8 variant={v}"), plan
            assert np.array_equal(tY.cpu().numpy(), exp), plan
    finally:
        set_i8_variant(-1)
    if M * K * N <= 10**7:
        assert np.array_equal(tY.cpu().numpy(), oracle.dense_i32(X, W, b, "relu"))


def test_int8_path_odd_shapes_strided_and_out_of_range(torch_cuda):
    """Padded, offset device views (the narrowing pass's unaligned loads on
    edge tiles), then a value outside int8 (the exact i32 fallback on the
    original tensors), then in range again."""
    from mlir_edsl_hip.device import dense_launch
    M, K, N = 300, 250, 190
    rng = np.random.default_rng(21)
    X = rng.integers(-128, 128, size=(M, K), dtype=np.int32)
    W = rng.integers(-128, 128, size=(K, N), dtype=np.int32)
    b = rng.integers(-1000, 1000, size=(N,), dtype=np.int32)

    def view(a, pad, off):
        rows, cols = a.shape
        buf = torch_cuda.zeros(rows * (cols + pad) + off, dtype=torch_cuda.int32, device="cuda")
        v = buf[off:].view(rows, cols + pad)[:, :cols]
        v.copy_(torch_cuda.from_numpy(a))
        return v

    for Xc, path in ((X, "narrow_i8+gemm_i8"), (np.where(np.arange(K) == 17, 5000, X).astype(np.int32),
                                                 "narrow_i8+gemm_i8"), (X, "narrow_i8+gemm_i8")):
        tX, tW = view(Xc, 3, 1), view(W, 5, 2)
        tY = view(np.full((M, N), -7, dtype=np.int32), 2, 3)
        dense_launch(tX, tW, torch_cuda.from_numpy(b).cuda(), tY, _native.EPI_BIAS_RELU)
        torch_cuda.cuda.synchronize()
        assert _native.last_plan().startswith(path)
        assert np.array_equal(tY.cpu().numpy(), _exact_i32(Xc, W, b))


# The tiles on 16x16 MFMA blocks (gemm_f32_m16.hip): K steps of 32 (128x128)
# or 64 (64x64) with loads two steps ahead and each step's last group of MFMAs
# deferred past its barrier. One, two and three K steps cover the ring's
# remainder paths and the final deferred group in both parities; the long K
# and the tall and wide shapes cover many steps and tile orders. The one-wave
# 128x128 tile (gemm_f32_direct.hip) walks K in 16-deep groups, two register
# sets: one, two and three groups cover its loop and its odd remainder; its
# 64x64 twin runs three register sets per wave over the wave's share of K.
MFMA16_SHAPES = {
    "f32_128x128x16_direct": [(128, 16, 128), (256, 32, 128), (128, 48, 384), (384, 2048, 256),
                              (1024, 160, 128), (128, 208, 1024)],
    # the 64x64 tile: one to seven groups per wave, K unsplit and split four ways
    "f32_64x64x16_direct": [(64, 16, 64), (128, 32, 64), (64, 48, 192), (192, 2048, 128), (1024, 160, 64),
                            (64, 208, 1024)],
    # the 16x16 tile for small layers: one to eight groups per wave, every load up front
    "f32_16x16x64_direct_k4": [(80, 64, 48), (256, 256, 256), (96, 512, 160), (1024, 128, 32), (128, 448, 16)],
    "f32_64x64x64_direct_k4": [(64, 64, 64), (128, 128, 64), (64, 192, 192), (192, 2048, 128),
                               (1024, 320, 64), (64, 448, 1024), (1024, 1024, 1024)],
    # the R x C tiles with K split four ways: one to 32 groups per wave (K / 16
    # groups shared as evenly as they go), B in pieces of 64, 32 and 16
    # columns (3 = 2 + 1, 5 = 4 + 1, 6 = 4 + 2)
    "f32_32x32x64_direct_rc": [(96, 64, 32), (128, 128, 96), (512, 512, 512), (96, 1024, 64), (160, 2048, 256),
                               (96, 80, 64), (128, 208, 96)],
    "f32_48x48x64_direct_rc": [(96, 64, 48), (144, 128, 144), (768, 768, 768), (144, 2048, 48), (96, 320, 480),
                               (144, 112, 96), (768, 784, 768)],
    "f32_80x80x64_direct_rc": [(80, 64, 80), (160, 192, 240), (400, 1024, 160), (1280, 256, 1280)],
    "f32_96x96x64_direct_rc": [(96, 64, 96), (192, 128, 288), (96, 2048, 192), (1536, 384, 1536), (192, 1040, 96)],
    "f32_48x96x64_direct_rc": [(96, 64, 96), (144, 256, 192), (768, 512, 3072)],
    "f32_96x48x64_direct_rc": [(96, 64, 48), (192, 256, 96), (3072, 512, 768)],
    "f32_64x64x64_direct_rc": [(64, 64, 64), (128, 128, 64), (64, 192, 192), (192, 2048, 128),
                               (1024, 320, 64), (1024, 1024, 1024)],
    "f32_128x128x32_mfma16": [(128, 32, 128), (256, 64, 128), (128, 96, 384), (384, 2048, 256),
                              (1024, 160, 128), (128, 224, 1024)],
    "f32_128x128x32_mfma16_w8": [(128, 32, 128), (256, 64, 256), (384, 96, 128), (128, 1056, 384)],
    "f32_128x256x32_mfma16": [(128, 32, 256), (256, 64, 512), (128, 96, 768), (384, 1056, 256)],
    "f32_64x64x64_mfma16": [(64, 64, 64), (128, 128, 64), (64, 192, 192), (192, 2048, 128),
                            (1024, 320, 64), (64, 448, 1024), (1024, 1024, 1024)],
}


@pytest.mark.parametrize("tile", sorted(MFMA16_SHAPES))
def test_mfma16_tiles_across_k_steps_shapes_and_epilogues(tile, torch_cuda):
    from mlir_edsl_hip.device import dense_launch, set_f32_config
    torch = torch_cuda
    names = _native.f32_config_names()
    cfg = names.index(tile)
    acts = [(_native.EPI_BIAS_RELU, "relu", True), (_native.EPI_NONE, "none", False),
            (_native.EPI_BIAS, "none", True), (_native.EPI_RELU, "relu", False),
            (_native.EPI_BIAS_LEAKY, "leaky", True), (_native.EPI_LEAKY, "leaky", False)]
    try:
        set_f32_config(cfg)
        for i, (M, K, N) in enumerate(MFMA16_SHAPES[tile]):
            X, W, b = _inputs(M, K, N, 300 + i)
            epi, act, has_bias = acts[i % len(acts)]
            ref = oracle.dense_f32_chains(X, W, b if has_bias else None, act, alpha=0.125)
            # contiguous, then padded rows with an element offset (16-byte aligned)
            for pad, off in ((0, 0), (4, 8)):
                tX, tW = _view(torch, X, pad, off), _view(torch, W, pad, off)
                tb = torch.from_numpy(b).cuda()
                tY = _view(torch, np.full((M, N), np.nan, dtype=np.float32), pad, off)
                dense_launch(tX, tW, tb if has_bias else None, tY, epi, 0.125)
                torch.cuda.synchronize()
                assert f"cfg={tile} " in _native.last_plan(), _native.last_plan()
                assert_f32_parity(tY.cpu().numpy(), ref, K)
    finally:
        set_f32_config(-1)


def test_mfma16_edge_tiles_on_random_shapes(torch_cuda):
    """The edge twins of the 16x16-block tiles on random sizes (M, N up to
    2600, K up to 900, multiples of 4, so both partial tiles and a partial
    last K step occur), contiguous and as padded views with an offset, each
    forced and by the automatic plan, against the oracle on the full output."""
    from mlir_edsl_hip.device import set_f32_config
    torch = torch_cuda
    names = _native.f32_config_names()
    forced = [names.index("f32_128x128x32_mfma16_edge"), names.index("f32_64x64x64_mfma16_edge"),
              names.index("f32_128x128x16_direct_edge"), names.index("f32_64x64x64_direct_k4_edge"),
              names.index("f32_48x48x64_direct_rc_edge"), names.index("f32_96x96x64_direct_rc_edge")]
    rng = np.random.default_rng(77)
    try:
        for case in range(12):
            M, N = (int(v) for v in 4 * rng.integers(1, 651, size=2))
            K = int(4 * rng.integers(1, 226))
            X, W, b = _inputs(M, K, N, 400 + case)
            ref = oracle.dense_f32_chains(X, W, b, "relu")
            pad, off = ((0, 0), (4, 8), (8, 4))[case % 3]
            for cfg in forced + [-1]:
                set_f32_config(cfg)
                got, plan = _run(torch, X, W, b, pad, off)
                if cfg >= 0:
                    assert f"cfg={names[cfg]} " in plan, (plan, (M, K, N))
                assert_f32_parity(got, ref, K)
    finally:
        set_f32_config(-1)


@pytest.mark.parametrize("tile", ["f32_128x128x16_direct_edge", "f32_128x128x16_direct",
                                  "f32_64x64x64_direct_k4_edge",
                                  "f32_64x64x64_direct_k4", "f32_128x128x32_mfma16_edge",
                                  "f32_48x48x64_direct_rc", "f32_96x96x64_direct_rc",
                                  "f32_80x80x64_direct_rc", "f32_48x96x64_direct_rc",
                                  "f32_48x48x64_direct_rc_edge", "f32_96x96x64_direct_rc_edge"])
def test_values_past_the_operands_never_reach_the_output(tile, torch_cuda):
    """Edge tiles read past K, N and M only in ways whose values are zeroed or
    never stored: with NaN and Inf in every padding element of A and B (the
    row pitch past K and N, and the rows after the last), every output
    element still matches the oracle. The one-wave tiles' partial last K
    group sends A chunks past K out of range and the B rows that pair with
    them read zero, so an Inf past K cannot become 0 x Inf; with K split over
    four waves, K = 4 and 20 leave some waves no group at all."""
    from mlir_edsl_hip.device import dense_launch, set_f32_config
    torch = torch_cuda
    names = _native.f32_config_names()
    bm, bn = (int(v) for v in tile.split("_")[1].split("x")[:2])
    shapes = [(384, 2048, 256), (256, 1024, 384)] if 128 % bm == 0 and 128 % bn == 0 else \
        [(3 * bm, 2048, 2 * bn), (2 * bm, 1024, 3 * bn)]
    if tile.endswith("_edge"):
        shapes = [(300, 100, 260), (257, 68, 132), (129, 1028, 260), (65, 20, 36), (1, 4, 4)]
    try:
        set_f32_config(names.index(tile))
        for i, (M, K, N) in enumerate(shapes):
            X, W, b = _inputs(M, K, N, 700 + i)
            ref = oracle.dense_f32_chains(X, W, b, "relu")
            views = []
            for a, fill in ((X, np.nan), (W, np.inf)):
                rows, cols = a.shape
                pitch = cols + 8
                buf = torch.full(((rows + 2) * pitch + 4,), fill, dtype=torch.float32, device="cuda")
                v = buf[4:4 + rows * pitch].view(rows, pitch)[:, :cols]
                v.copy_(torch.from_numpy(a))
                views.append(v)
            tb = torch.from_numpy(b).cuda()
            tY = _view(torch, np.full((M, N), np.nan, dtype=np.float32), 8, 4)
            dense_launch(views[0], views[1], tb, tY, _native.EPI_BIAS_RELU)
            torch.cuda.synchronize()
            assert f"cfg={tile} " in _native.last_plan(), _native.last_plan()
            assert_f32_parity(tY.cpu().numpy(), ref, K)
    finally:
        set_f32_config(-1)
