"""GPU parity: the HIP path, called through the C ABI, against the pinned
oracle, the exact golden vectors and the reference's known answers.

Bar: i32 bit-exact; f32 relative Frobenius error <= 1e-5 and
max|delta| <= 1e-4*sqrt(K) against both rounding chains the reference can
take, element by element (tests/conftest.py: assert_f32_parity).
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle
from conftest import assert_f32_parity
from mlir_edsl_hip import _native, backend
from mlir_edsl_hip.inputs import WORKLOADS, make_inputs

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_PATTERN = {"matmul": (False, "none"), "matmul_relu": (False, "relu"),
            "matmul_bias": (True, "none"), "dense_relu": (True, "relu"),
            "dense_leaky": (True, "leaky"), "dense_if_relu": (True, "if_relu"),
            "matmul_if_relu": (False, "if_relu")}
_EPI_TAG = {"none": "matmul", "bias": "matmul_bias", "relu": "dense_relu", "leaky": "dense_leaky",
            "relu_nobias": "matmul_relu", "if_relu": "dense_if_relu", "if_relu_nobias": "matmul_if_relu"}


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available()
    return torch


def to_dev(torch, arrays):
    return [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrays]


def gpu_run(pattern, arrays, alpha=0.01, device=False):
    if device:
        import torch
        out = backend.run(pattern, *to_dev(torch, arrays), alpha=alpha)
        torch.cuda.synchronize()
        return out.cpu().numpy()
    return backend.run(pattern, *arrays, alpha=alpha)


def oracle_run(pattern, arrays, alpha=0.01):
    bias, act = _PATTERN[pattern]
    X, W = arrays[0], arrays[1]
    b = arrays[2] if bias else None
    if X.dtype == np.int32:
        return oracle.dense_i32(X, W, b, act)
    return oracle.dense_f32_chains(X, W, b, act, alpha)


def check(got, ref, K):
    if isinstance(ref, oracle.F32Chains):
        assert_f32_parity(got, ref, K)
    else:
        assert ref.dtype == np.int32 and got.dtype == np.int32
        assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches"


# ------------------------------------------------------------ known answers
def _known():
    with open(os.path.join(GOLDEN, "reference_known_answers.json")) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("device", [False, True], ids=["host", "device"])
@pytest.mark.parametrize("case", _known(), ids=lambda c: c["name"])
def test_reference_known_answers(case, device, torch_cuda):
    dt = np.float32 if case["dtype"] == "f32" else np.int32
    ins = [np.asarray(x, dtype=dt) for x in case["inputs"]]
    got = gpu_run(case["pattern"], ins, alpha=case["alpha"], device=device)
    exp = np.asarray(case["expected"], dtype=dt)
    if dt == np.int32:
        assert np.array_equal(got, exp)
    else:
        np.testing.assert_allclose(got, exp, rtol=case["rtol"], atol=case["atol"])


def test_chained_matmul_known_answer(torch_cuda):
    # reference tests/linalg/test_matmul_execution.py:110-122: (I @ B) @ I == B
    I = np.eye(2, dtype=np.float32)
    B = np.array([[1, 2], [3, 4]], np.float32)
    np.testing.assert_allclose(backend.matmul(backend.matmul(I, B), I), B, rtol=1e-4)


# ----------------------------------------------------------- golden vectors
def _golden_cases():
    with open(os.path.join(GOLDEN, "dense_golden.json")) as f:
        meta = json.load(f)["cases"]
    return [(c, tag) for c in meta for tag in c["epilogues"]]


@pytest.fixture(scope="module")
def golden_data():
    return np.load(os.path.join(GOLDEN, "dense_golden.npz"), allow_pickle=False)


@pytest.mark.parametrize("case,tag", _golden_cases(), ids=lambda v: v["name"] if isinstance(v, dict) else v)
def test_golden_vectors(case, tag, golden_data, torch_cuda):
    n = case["name"]
    X, W, b = golden_data[f"{n}/X"], golden_data[f"{n}/W"], golden_data[f"{n}/b"]
    pattern = _EPI_TAG[tag]
    arrays = [X, W, b] if _PATTERN[pattern][0] else [X, W]
    if case["dtype"] == "f32":
        exp = oracle.F32Chains(golden_data[f"{n}/Y_{tag}_fma"], golden_data[f"{n}/Y_{tag}_muladd"])
    else:
        exp = golden_data[f"{n}/Y_{tag}"]
    for device in (False, True):
        got = gpu_run(pattern, arrays, alpha=case.get("alpha", 0.01), device=device)
        check(got, exp, case["K"])


# ------------------------------------------- the reference's GPU test shapes
@pytest.mark.parametrize("pattern,size", [
    ("matmul", 8), ("matmul", 16), ("matmul", 48), ("matmul", 64), ("matmul", 96), ("matmul", 128),
    ("dense_relu", 32), ("dense_relu", 64), ("dense_relu", 96), ("matmul_bias", 64),
    ("matmul", 256), ("dense_relu", 128)])
def test_reference_gpu_and_multicore_shapes(pattern, size, torch_cuda):
    # reference tests/gpu/test_gpu_execution.py:52-210, tests/core/test_multicore.py:19-123
    rng = np.random.default_rng(1000 + size)
    arrays = [rng.random((size, size), dtype=np.float32), rng.random((size, size), dtype=np.float32)]
    if _PATTERN[pattern][0]:
        arrays.append(rng.random(size, dtype=np.float32))
    ref = oracle_run(pattern, arrays)
    for device in (False, True):
        check(gpu_run(pattern, arrays, device=device), ref, size)


# ------------------------------------------------------- BASELINE workloads
def test_c1_matmul_256(torch_cuda):
    w = WORKLOADS["c1"]
    A, B = make_inputs(w)
    check(gpu_run("matmul", [A, B], device=True), oracle.dense_f32_chains(A, B), w.K)


def test_c2_dense_1024(torch_cuda):
    w = WORKLOADS["c2"]
    X, W, b = make_inputs(w)
    ref = oracle.dense_f32_chains(X, W, b, "relu")
    check(gpu_run("dense_relu", [X, W, b], device=True), ref, w.K)
    check(gpu_run("dense_relu", [X, W, b], device=False), ref, w.K)


def test_c3_dense_4096_full(torch_cuda):
    """The headline layer, every one of its 4096 x 4096 outputs against the
    oracle (about a second of CPU time on 16 threads)."""
    w = WORKLOADS["c3"]
    X, W, b = make_inputs(w)
    got = gpu_run("dense_relu", [X, W, b], device=True)
    assert _native.last_plan().startswith("gemm_f32")
    check(got, oracle.dense_f32_chains(X, W, b, "relu"), w.K)


def test_c4_dense_small_m(torch_cuda):
    w = WORKLOADS["c4"]
    X, W, b = make_inputs(w)
    ref = oracle.dense_f32_chains(X, W, b, "relu")
    for _ in range(2):  # the split-K counters must re-arm between calls
        got = gpu_run("dense_relu", [X, W, b], device=True)
        assert _native.last_plan().startswith("gemv_f32")
        check(got, ref, w.K)


def test_c4_column_shard(torch_cuda):
    """One GPU's share of c4 column-sharded 8 ways, full output."""
    w = WORKLOADS["c4s8"]
    X, W, b = make_inputs(w)
    got = gpu_run("dense_relu", [X, W, b], device=True)
    assert _native.last_plan().startswith("gemv_f32")
    check(got, oracle.dense_f32_chains(X, W, b, "relu"), w.K)


def test_c3_column_shard_full(torch_cuda):
    """One GPU's share of c3 column-sharded 8 ways, full output."""
    w = WORKLOADS["c3s8"]
    X, W, b = make_inputs(w)
    got = gpu_run("dense_relu", [X, W, b], device=True)
    assert _native.last_plan().startswith("gemm_f32")
    check(got, oracle.dense_f32_chains(X, W, b, "relu"), w.K)


def test_column_shards_reassemble_the_layer(torch_cuda):
    """Column sharding needs no exchange: the 8 shards of c4, each run on a
    strided column slice of W (row stride 8192) and of b, written into the
    matching columns of one Y, give the layer's output."""
    import torch
    from mlir_edsl_hip.device import dense_launch
    w = WORKLOADS["c4"]
    X, W, b = make_inputs(w)
    tX, tW, tb = to_dev(torch, [X, W, b])
    Y = torch.full((w.M, w.N), float("nan"), device="cuda")
    n = w.N // 8
    for g in range(8):
        cols = slice(g * n, (g + 1) * n)
        dense_launch(tX, tW[:, cols], tb[cols], Y[:, cols], _native.EPI_BIAS_RELU)
        assert _native.last_plan().startswith("gemv_f32")
    torch.cuda.synchronize()
    check(Y.cpu().numpy(), oracle.dense_f32_chains(X, W, b, "relu"), w.K)


def test_c5_int_dense_bit_exact(torch_cuda):
    w = WORKLOADS["c5"]
    X, W, b = make_inputs(w)
    got = gpu_run("dense_relu", [X, W, b], device=True)
    assert _native.last_plan().startswith("narrow_i8+gemm_i8")
    exact = X.astype(np.float64) @ W.astype(np.float64) + b  # |sum| < 2^53: exact
    exp = np.maximum(exact, 0).astype(np.int32)
    assert np.array_equal(got, exp)
    assert np.array_equal(got, oracle.dense_i32(X, W, b, "relu"))


# ------------------------------------------------------------ integer path
def test_int8_path_falls_back_when_values_leave_int8(torch_cuda):
    rng = np.random.default_rng(9)
    n = 256
    X = rng.integers(-2**31, 2**31, size=(n, n), dtype=np.int64).astype(np.int32)
    W = rng.integers(-2**31, 2**31, size=(n, n), dtype=np.int64).astype(np.int32)
    b = rng.integers(-2**31, 2**31, size=(n,), dtype=np.int64).astype(np.int32)
    with np.errstate(over="ignore"):
        exp = (X.astype(np.int64) @ W.astype(np.int64) + b).astype(np.int32)
    got = gpu_run("matmul_bias", [X, W, b], device=True)
    assert np.array_equal(got, exp)
    # one value out of range among int8 ones
    X2 = rng.integers(-128, 128, size=(n, n), dtype=np.int32)
    W2 = rng.integers(-128, 128, size=(n, n), dtype=np.int32)
    W2[17, 201] = 300
    exp2 = (X2.astype(np.int64) @ W2.astype(np.int64) + b.astype(np.int64) + 2**31) % 2**32 - 2**31
    got2 = gpu_run("dense_relu", [X2, W2, b], device=True)
    assert np.array_equal(got2, np.maximum(exp2, 0).astype(np.int32))
    # the next in-range call takes the int8 path again and is still exact
    W2[17, 201] = 5
    got3 = gpu_run("matmul", [X2, W2], device=True)
    assert np.array_equal(got3, (X2.astype(np.int64) @ W2.astype(np.int64)).astype(np.int32))


def test_int8_fallback_is_per_tile(torch_cuda):
    """Values outside int8 in a few 64x64 tiles of X and W: the tiles whose
    panels hold them take the exact i32 path, the others the int8 path, and
    every output is exact, for every variant."""
    from mlir_edsl_hip.device import set_i8_variant
    rng = np.random.default_rng(16)
    M, K, N = 640, 768, 896
    X = rng.integers(-128, 128, size=(M, K), dtype=np.int32)
    W = rng.integers(-128, 128, size=(K, N), dtype=np.int32)
    b = rng.integers(-2**20, 2**20, size=(N,), dtype=np.int32)
    X[200, 700] = 129
    X[639, 0] = -2**31
    W[64, 895] = 2**20
    exact = X.astype(np.int64) @ W.astype(np.int64) + b
    exp = np.maximum((exact + 2**31) % 2**32 - 2**31, 0).astype(np.int32)
    try:
        for v in range(_native.lib().edsl_hip_i8_variant_count()):
            set_i8_variant(v)
            got = gpu_run("dense_relu", [X, W, b], device=True)
            assert _native.last_plan().startswith(f"narrow_i8+gemm_i8 variant={v}")
            assert np.array_equal(got, exp), f"variant {v}"
    finally:
        set_i8_variant(-1)


def test_every_int8_variant(torch_cuda):
    from mlir_edsl_hip.device import set_i8_variant
    rng = np.random.default_rng(15)
    M, K, N = 256, 512, 384
    X = rng.integers(-128, 128, size=(M, K), dtype=np.int32)
    W = rng.integers(-128, 128, size=(K, N), dtype=np.int32)
    b = rng.integers(-2**20, 2**20, size=(N,), dtype=np.int32)
    Xbig = X.copy()
    Xbig[5, 7] = 1000  # forces the exact i32 fallback inside the same kernel
    n = _native.lib().edsl_hip_i8_variant_count()
    try:
        for v in range(n):
            set_i8_variant(v)
            for Xc in (X, Xbig):
                got = gpu_run("dense_relu", [Xc, W, b], device=True)
                assert f"variant={v}" in _native.last_plan()
                assert np.array_equal(got, oracle.dense_i32(Xc, W, b, "relu"))
    finally:
        set_i8_variant(-1)


@pytest.mark.parametrize("K", [128, 384, 1152])
def test_int8_depth_fallback_and_strided_sources(K, torch_cuda):
    """K/32 = 4, 12, 36 steps: prefetch depth 8 does not divide them, so every
    variant runs at depth 4 or 2 (the plan names the depth). The sources are
    device views with an odd row pitch and an element offset, so the
    narrowing pass takes its unaligned 4-byte loads."""
    import torch
    from mlir_edsl_hip.device import dense_launch, set_i8_variant
    rng = np.random.default_rng(K)
    M, N = 256, 128
    X = rng.integers(-128, 128, size=(M, K), dtype=np.int32)
    W = rng.integers(-128, 128, size=(K, N), dtype=np.int32)
    b = rng.integers(-2**20, 2**20, size=(N,), dtype=np.int32)
    exp = oracle.dense_i32(X, W, b, "relu")

    def view(a, pad, off):
        rows, cols = a.shape
        buf = torch.zeros(rows * (cols + pad) + off, dtype=torch.int32, device="cuda")
        v = buf[off:].view(rows, cols + pad)[:, :cols]
        v.copy_(torch.from_numpy(a))
        return v

    tX, tW = view(X, 3, 1), view(W, 5, 2)
    tb = torch.from_numpy(b).cuda()
    n = _native.lib().edsl_hip_i8_variant_count()
    try:
        for v in range(n):
            set_i8_variant(v)
            tY = torch.full((M, N), -7, dtype=torch.int32, device="cuda")
            dense_launch(tX, tW, tb, tY, _native.EPI_BIAS_RELU)
            torch.cuda.synchronize()
            plan = _native.last_plan()
            assert f"variant={v}" in plan and "depth=8" not in plan, plan
            assert np.array_equal(tY.cpu().numpy(), exp), plan
    finally:
        set_i8_variant(-1)


@pytest.mark.parametrize("K, path", [(2**17 - 128, "narrow_i8+gemm_i8"), (2**17 - 1, "narrow_i8+gemm_i8"),
                                     (2**17, "gemm_i32_valu")])
def test_int8_exactness_boundary(K, path, torch_cuda):
    """Every product is (-128)(-128) = 16384, so every output is 16384*K,
    exact in i32 up to K = 2^17 - 1 (the int8 path runs; K = 2^17 - 1 also
    pads the packed K to 2^17 with zeros) and 2^31 at K = 2^17, which wraps
    to -2^31 (arith.addi semantics; the exact i32 path runs, as it does for
    every K >= 2^17). ReLU of the wrapped value is 0."""
    import torch
    from mlir_edsl_hip.device import dense_launch
    M = N = 128
    X = torch.full((M, K), -128, dtype=torch.int32, device="cuda")
    W = torch.full((K, N), -128, dtype=torch.int32, device="cuda")
    exp = (16384 * K + 2**31) % 2**32 - 2**31
    for epi, want in ((_native.EPI_NONE, exp), (_native.EPI_RELU, max(exp, 0))):
        Y = torch.full((M, N), 7, dtype=torch.int32, device="cuda")
        dense_launch(X, W, None, Y, epi)
        torch.cuda.synchronize()
        plan = _native.last_plan()
        assert plan.startswith(path), plan
        got = Y.cpu().numpy()
        assert (got == want).all(), (plan, int(got.min()), int(got.max()), want)


@pytest.mark.parametrize("shape", [(1, 1, 1), (3, 5, 7), (65, 33, 17), (130, 128, 128), (128, 256, 384)])
def test_int_shapes(shape, torch_cuda):
    M, K, N = shape
    rng = np.random.default_rng(M * 7 + K)
    X = rng.integers(-100, 100, size=(M, K), dtype=np.int32)
    W = rng.integers(-100, 100, size=(K, N), dtype=np.int32)
    b = rng.integers(-1000, 1000, size=(N,), dtype=np.int32)
    for pattern in ("matmul", "matmul_relu", "matmul_bias", "dense_relu"):
        arrays = [X, W, b] if _PATTERN[pattern][0] else [X, W]
        check(gpu_run(pattern, arrays, device=True), oracle_run(pattern, arrays), K)


# ------------------------------------------------------ shapes and layouts
@pytest.mark.parametrize("shape", [(1, 1, 1), (3, 5, 7), (65, 33, 17), (100, 200, 300),
                                   (257, 129, 511), (64, 4, 64)])
def test_f32_odd_shapes(shape, torch_cuda):
    M, K, N = shape
    rng = np.random.default_rng(M + 3 * K + 7 * N)
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = rng.standard_normal((K, N), dtype=np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    for pattern in ("matmul", "dense_relu", "dense_leaky"):
        arrays = [X, W, b] if _PATTERN[pattern][0] else [X, W]
        check(gpu_run(pattern, arrays, alpha=0.2), oracle_run(pattern, arrays, alpha=0.2), K)


def test_k_zero_gives_activation_of_bias(torch_cuda):
    X = np.zeros((4, 0), np.float32)
    W = np.zeros((0, 8), np.float32)
    b = np.linspace(-1, 1, 8, dtype=np.float32)
    got = gpu_run("dense_relu", [X, W, b])
    assert np.array_equal(got, np.tile(np.maximum(b, 0), (4, 1)))
    gi = gpu_run("matmul_bias", [X.astype(np.int32), W.astype(np.int32), np.arange(8, dtype=np.int32)])
    assert np.array_equal(gi, np.tile(np.arange(8, dtype=np.int32), (4, 1)))


def test_empty_output(torch_cuda):
    got = gpu_run("matmul", [np.zeros((0, 5), np.float32), np.zeros((5, 3), np.float32)])
    assert got.shape == (0, 3)


def test_strided_and_misaligned_device_operands(torch_cuda):
    torch = torch_cuda
    rng = np.random.default_rng(11)
    M, K, N = 192, 256, 320
    big_x = rng.standard_normal((M, K + 9), dtype=np.float32)
    big_w = rng.standard_normal((K, N + 3), dtype=np.float32)
    b = rng.standard_normal(N + 1, dtype=np.float32)
    tx, tw, tb = to_dev(torch, [big_x, big_w, b])
    X, W, bias = tx[:, 1:K + 1], tw[:, :N], tb[1:]        # row stride > cols, offset 1
    Y = torch.empty((M, N + 5), device="cuda")[:, 2:N + 2]  # strided, misaligned output
    from mlir_edsl_hip.device import dense_launch
    dense_launch(X, W, bias, Y, _native.EPI_BIAS_RELU)
    torch.cuda.synchronize()
    ref = oracle.dense_f32_chains(big_x[:, 1:K + 1], big_w[:, :N], b[1:], "relu")
    check(Y.cpu().numpy(), ref, K)
    # aligned views with a padded row stride keep the fast path
    X2, W2 = tx[:, :K], tw[:, :N - 64]
    Y2 = torch.empty((M, N - 64 + 4), device="cuda")[:, :N - 64]
    dense_launch(X2, W2, None, Y2, _native.EPI_NONE)
    torch.cuda.synchronize()
    check(Y2.cpu().numpy(), oracle.dense_f32_chains(big_x[:, :K], big_w[:, :N - 64]), K)


def test_memref_offset_is_honoured(torch_cuda):
    """aligned + offset addressing of the descriptor (host operands)."""
    rng = np.random.default_rng(12)
    A = rng.standard_normal(8 * 8 + 3, dtype=np.float32)
    B = rng.standard_normal((8, 8), dtype=np.float32)
    C = np.zeros((8, 8), np.float32)
    L = _native.lib()
    L.edsl_hip_matmul_f32(A.ctypes.data, A.ctypes.data, 3, 8, 8, 8, 1,
                          B.ctypes.data, B.ctypes.data, 0, 8, 8, 8, 1,
                          C.ctypes.data, C.ctypes.data, 0, 8, 8, 8, 1)
    _native.raise_on_error("matmul")
    check(C, oracle.dense_f32_chains(A[3:].reshape(8, 8), B), 8)


@pytest.mark.parametrize("M", [1, 2, 16, 17, 31, 48, 64])
@pytest.mark.parametrize("ksplit", [1, 2, 4, 8])
def test_small_m_kernel(M, ksplit, torch_cuda):
    from mlir_edsl_hip.device import set_gemv_ksplit
    rng = np.random.default_rng(M * 10 + ksplit)
    K, N = 1024, 512
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.float32(32)).astype(np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    set_gemv_ksplit(ksplit)
    try:
        for _ in range(2):
            got = gpu_run("dense_relu", [X, W, b], device=True)
            assert _native.last_plan().startswith(f"gemv_f32 mb={(M + 15) // 16} ksplit={ksplit}")
            check(got, oracle.dense_f32_chains(X, W, b, "relu"), K)
    finally:
        set_gemv_ksplit(0)


@pytest.mark.parametrize("cols", [32, 64, 128, 256])
@pytest.mark.parametrize("ksplit", [1, 2, 4, 8, 16])
def test_small_m_column_blocks_and_splits(cols, ksplit, torch_cuda):
    """Every column-block width and K split, on back-to-back calls with
    different inputs and row counts (the partial buffer is reused)."""
    from mlir_edsl_hip.device import set_gemv_cols, set_gemv_ksplit
    K, N = 4096, 1024
    set_gemv_cols(cols)
    set_gemv_ksplit(ksplit)
    try:
        for trial, M in enumerate((16, 5, 33, 64)):
            rng = np.random.default_rng(1000 * cols + 10 * ksplit + trial)
            X = rng.standard_normal((M, K), dtype=np.float32)
            W = (rng.standard_normal((K, N), dtype=np.float32) / np.float32(64)).astype(np.float32)
            b = rng.standard_normal(N, dtype=np.float32)
            got = gpu_run("dense_relu", [X, W, b], device=True)
            plan = _native.last_plan()
            assert f"ksplit={ksplit} cols={cols}" in plan, plan
            check(got, oracle.dense_f32_chains(X, W, b, "relu"), K)
    finally:
        set_gemv_cols(0)
        set_gemv_ksplit(0)


def test_every_f32_tile_config(torch_cuda):
    from mlir_edsl_hip.device import set_f32_config
    rng = np.random.default_rng(13)
    M, K, N = 512, 256, 512
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = rng.standard_normal((K, N), dtype=np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    ref = oracle.dense_f32_chains(X, W, b, "relu")
    names = _native.f32_config_names()
    try:
        for cfg, name in enumerate(names):
            if "guard" in name:
                continue
            set_f32_config(cfg)
            bm, bn, bk = (int(v) for v in name.split("_")[1].split("x"))
            if M % bm == 0 and N % bn == 0 or name.endswith(("_edge", "_anyshape")):
                Mc, Nc, Xc, Wc, bc, refc = M, N, X, W, b, ref
            else:
                # exact tiles that do not divide 512 (48, 80, 96): the next
                # multiples of the tile
                Mc, Nc = -(-M // bm) * bm, -(-N // bn) * bn
                Xc = rng.standard_normal((Mc, K), dtype=np.float32)
                Wc = rng.standard_normal((K, Nc), dtype=np.float32)
                bc = rng.standard_normal(Nc, dtype=np.float32)
                refc = oracle.dense_f32_chains(Xc, Wc, bc, "relu")
            got = gpu_run("dense_relu", [Xc, Wc, bc], device=True)
            assert name in _native.last_plan()
            check(got, refc, K)
            # Seven K steps: the loop remainder after every group of prefetch
            # steps (1 for depths 2 and 3, 3 for depth 4) and the ring wrap.
            # Four: at depth 4 only the load-free tail runs (no loop group).
            for steps in (7, 4):
                Ks = steps * bk
                Xs = rng.standard_normal((Mc, Ks), dtype=np.float32)
                Ws = rng.standard_normal((Ks, Nc), dtype=np.float32)
                got = gpu_run("dense_relu", [Xs, Ws, bc], device=True)
                assert name in _native.last_plan()
                check(got, oracle.dense_f32_chains(Xs, Ws, bc, "relu"), Ks)
    finally:
        set_f32_config(-1)


def test_nan_and_inf_propagate_like_maximumf(torch_cuda):
    rng = np.random.default_rng(14)
    M, K, N = 128, 128, 128
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = rng.standard_normal((K, N), dtype=np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    X[3, 5] = np.nan
    b[7] = np.inf
    b[9] = -np.inf
    for pattern in ("dense_relu", "dense_leaky", "matmul_bias"):
        ref = oracle_run(pattern, [X, W, b], alpha=0.1)
        got = gpu_run(pattern, [X, W, b], alpha=0.1, device=True)
        assert np.isnan(got[3]).all()  # fmaxf semantics would give 0 after ReLU
        check(got, ref, K)


@pytest.mark.parametrize("shape", [(16, 1024, 512), (256, 256, 256), (300, 101, 259), (1, 64, 8)],
                         ids=["small-M", "tiles", "any-shape", "one-row"])
def test_if_relu_maps_nan_and_negative_zero_to_zero(shape, torch_cuda):
    """The f32 If(v > 0.0, v, 0.0) epilogue on every kernel family: NaN
    inputs and -0 sums give +0 (cmpf ogt), where maximumf keeps the NaN;
    every element against the oracle's If epilogue on both chains."""
    import torch
    from mlir_edsl_hip.device import dense_launch
    M, K, N = shape
    rng = np.random.default_rng(M + K + N)
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = (rng.standard_normal((K, N), dtype=np.float32) / np.float32(np.sqrt(K))).astype(np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    X[0, K // 2] = np.nan                 # row 0: NaN sums
    b[N // 2] = np.nan                    # one NaN column
    b[-1] = -0.0
    if M > 1:
        X[M - 1, :] = 0.0                 # last row: +0 + -0 = +0 in the last column
    tX, tW, tb = to_dev(torch, [X, W, b])
    for epi, bias in ((_native.EPI_BIAS_IF_RELU, b), (_native.EPI_IF_RELU, None)):
        Y = torch.full((M, N), 7.0, device="cuda")
        dense_launch(tX, tW, tb if bias is not None else None, Y, epi)
        torch.cuda.synchronize()
        got = Y.cpu().numpy()
        assert not np.isnan(got).any() and not np.signbit(got).any(), _native.last_plan()
        assert np.array_equal(got[0], np.zeros(N, np.float32))
        check(got, oracle.dense_f32_chains(X, W, bias, "if_relu"), K)


def test_execute_gpu_function_host_entry(torch_cuda):
    be = backend.get_backend()
    w = WORKLOADS["c2"]
    X, W, b = make_inputs(w, M=256, K=512, N=384)
    be.compile_dense("dense_host_entry", "dense_relu",
                     [backend.tensor_type_of(a) for a in (X, W, b)])
    got = be.execute_gpu_function("dense_host_entry", X, W, b)
    check(got, oracle.dense_f32_chains(X, W, b, "relu"), 512)
    with pytest.raises(TypeError):
        be.execute_gpu_function("dense_host_entry", X.astype(np.float64), W, b)
