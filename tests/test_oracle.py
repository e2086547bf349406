"""Pins the CPU oracle (oracle/oracle.c) before anything is compared with it.

Checks, each chosen so that a plausible mistake in the oracle fails one:
  * the reference's own known answers (tests/golden/reference_known_answers.json);
  * golden vectors from exact rational arithmetic (tests/golden/make_golden.py):
    both fp32 rounding chains (fma, and mulf+addf) and the wrapping i32 sums,
    bit for bit;
  * the fp64 forward-error bound |fl(x.w) - x.w| <= gamma_K * sum|x||w| at
    sizes too large for rational arithmetic;
  * exact wrapping i32 arithmetic via int64 products at larger sizes;
  * IEEE special values through the ReLU (maximumf: NaN propagates), If-ReLU
    (cmpf ogt: NaN and -0 give +0) and leaky epilogues;
  * planted mistakes (oracle.mutation) are each caught by the checks above.
"""
from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _known_answers():
    with open(os.path.join(GOLDEN, "reference_known_answers.json")) as f:
        return json.load(f)["cases"]


def _golden():
    with open(os.path.join(GOLDEN, "dense_golden.json")) as f:
        meta = json.load(f)["cases"]
    data = np.load(os.path.join(GOLDEN, "dense_golden.npz"), allow_pickle=False)
    return meta, data


_EPI = {"none": (False, "none"), "bias": (True, "none"), "relu": (True, "relu"),
        "leaky": (True, "leaky"), "relu_nobias": (False, "relu"), "if_relu": (True, "if_relu"),
        "if_relu_nobias": (False, "if_relu")}
CHAINS = ("fma", "muladd")
_PATTERN = {"matmul": (False, "none"), "matmul_relu": (False, "relu"),
            "matmul_bias": (True, "none"), "dense_relu": (True, "relu"),
            "dense_leaky": (True, "leaky")}


def run_oracle(dtype, X, W, b, act, alpha=0.01, chain="fma"):
    if dtype == "f32":
        return oracle.dense_f32(X, W, b, act, alpha, chain=chain)
    return oracle.dense_i32(X, W, b, act)


# ------------------------------------------------------------ the checks
def check_known_answers():
    failures = []
    for c in _known_answers():
        dt = np.float32 if c["dtype"] == "f32" else np.int32
        ins = [np.asarray(x, dtype=dt) for x in c["inputs"]]
        bias, act = _PATTERN[c["pattern"]]
        exp = np.asarray(c["expected"], dtype=dt)
        for chain in CHAINS if c["dtype"] == "f32" else ("exact",):
            got = run_oracle(c["dtype"], ins[0], ins[1], ins[2] if bias else None, act, c["alpha"], chain)
            if c["dtype"] == "i32":
                ok = np.array_equal(got, exp)
            else:
                ok = np.allclose(got, exp, rtol=c["rtol"], atol=c["atol"])
            if not ok:
                failures.append(f"known answer {c['name']} ({c['source']}) chain {chain}")
    return failures


def check_golden():
    meta, data = _golden()
    failures = []
    for c in meta:
        n = c["name"]
        X, W, b = data[f"{n}/X"], data[f"{n}/W"], data[f"{n}/b"]
        for tag in c["epilogues"]:
            use_b, act = _EPI[tag]
            if c["dtype"] == "i32":
                got = run_oracle("i32", X, W, b if use_b else None, act)
                if not np.array_equal(got, data[f"{n}/Y_{tag}"]):
                    failures.append(f"golden {n}/{tag}")
                continue
            for chain in c["chains"]:
                got = run_oracle("f32", X, W, b if use_b else None, act, c["alpha"], chain)
                exp = data[f"{n}/Y_{tag}_{chain}"]
                if not np.array_equal(got.view(np.uint32), exp.view(np.uint32)):
                    failures.append(f"golden {n}/{tag} chain {chain}")
    return failures


def check_special_values():
    """bias injects NaN / inf / signed values into the epilogue directly."""
    failures = []
    vals = np.array([np.nan, -np.inf, np.inf, -1.0, 2.0, -0.0, 0.5, -3.0], dtype=np.float32)
    N = vals.size
    X = np.zeros((1, 8), np.float32)
    W = np.zeros((8, N), np.float32)
    for chain in CHAINS:
        y = oracle.dense_f32(X, W, vals, "relu", chain=chain)[0]
        exp = np.array([np.nan, 0, np.inf, 0, 2, 0, 0.5, 0], np.float32)
        if not (np.isnan(y[0]) and np.array_equal(y[1:], exp[1:]) and not np.signbit(y[5])):
            failures.append(f"relu special values {y}")
        # If(v > 0.0, v, 0.0): NaN and -0 both select the constant +0.
        yi = oracle.dense_f32(X, W, vals, "if_relu", chain=chain)[0]
        expi = np.array([0, 0, np.inf, 0, 2, 0, 0.5, 0], np.float32)
        if not (np.array_equal(yi, expi) and not np.signbit(yi).any()):
            failures.append(f"if_relu special values {yi}")
        yl = oracle.dense_f32(X, W, vals, "leaky", alpha=0.25, chain=chain)[0]
        expl = np.array([np.nan, -np.inf, np.inf, -0.25, 2, 0, 0.5, -0.75], np.float32)
        if not (np.isnan(yl[0]) and np.array_equal(yl[1:], expl[1:])):
            failures.append(f"leaky special values {yl}")
    # -0 reaching the activation from the sums themselves: on the fma chain
    # fma(-1e-30, 1e-30, +0) underflows to -0 and -0 + (-0 bias) stays -0;
    # on the mulf+addf chain the product underflows to -0 but +0 + -0 = +0.
    # If(v > 0.0, v, 0.0) turns the -0 into +0.
    Xz = np.array([[-1e-30]], np.float32)
    Wz = np.array([[1e-30, 1.0]], np.float32)
    bz = np.array([-0.0, -0.0], np.float32)
    yn = oracle.dense_f32(Xz, Wz, bz, "none", chain="fma")[0]
    ym = oracle.dense_f32(Xz, Wz, bz, "none", chain="muladd")[0]
    yi = [oracle.dense_f32(Xz, Wz, bz, "if_relu", chain=c)[0] for c in CHAINS]
    if not (yn[0] == 0 and np.signbit(yn[0]) and ym[0] == 0 and not np.signbit(ym[0])
            and all(np.array_equal(y, [0.0, 0.0]) and not np.signbit(y).any() for y in yi)):
        failures.append(f"-0 through if_relu: {yn}, {ym} -> {yi}")
    return failures


def check_i32_wrap():
    rng = np.random.default_rng(5)
    failures = []
    for (M, K, N) in [(64, 96, 80), (7, 33, 5)]:
        X = rng.integers(-2**31, 2**31, size=(M, K), dtype=np.int64).astype(np.int32)
        W = rng.integers(-2**31, 2**31, size=(K, N), dtype=np.int64).astype(np.int32)
        b = rng.integers(-2**31, 2**31, size=(N,), dtype=np.int64).astype(np.int32)
        # int64 products / sums wrap modulo 2^64; reducing to 32 bits is exact.
        with np.errstate(over="ignore"):
            exp = (X.astype(np.int64) @ W.astype(np.int64) + b.astype(np.int64)).astype(np.int32)
        got = oracle.dense_i32(X, W, b, "none")
        if not np.array_equal(got, exp):
            failures.append(f"i32 wrap {M}x{K}x{N}")
        got_r = oracle.dense_i32(X, W, b, "relu")
        if not np.array_equal(got_r, np.maximum(exp, 0)):
            failures.append(f"i32 wrap relu {M}x{K}x{N}")
    return failures


def check_fp64_bound():
    """|fl - exact| <= gamma_K * (sum|x||w|) elementwise (+ one rounding for
    the bias add), at shapes on both the fma and the mulf+addf paths."""
    rng = np.random.default_rng(6)
    failures = []
    u = 2.0 ** -24
    for (M, K, N) in [(128, 128, 64), (96, 96, 96), (64, 256, 192), (40, 100, 30)]:
        X = rng.standard_normal((M, K), dtype=np.float32)
        W = rng.standard_normal((K, N), dtype=np.float32)
        b = rng.standard_normal(N, dtype=np.float32)
        x64, w64 = X.astype(np.float64), W.astype(np.float64)
        exact = x64 @ w64 + b.astype(np.float64)
        # mulf+addf rounds twice per step: gamma_{2K} bounds both chains.
        gamma = 2 * K * u / (1 - 2 * K * u)
        bound = gamma * (np.abs(x64) @ np.abs(w64)) + u * (np.abs(exact) + np.abs(b)) + 1e-30
        for chain in CHAINS:
            got = oracle.dense_f32(X, W, b, "none", chain=chain).astype(np.float64)
            if not np.all(np.abs(got - exact) <= bound * 1.0001):
                failures.append(f"fp64 bound {M}x{K}x{N} chain {chain}")
    return failures


ALL_CHECKS = [check_known_answers, check_golden, check_special_values, check_i32_wrap,
              check_fp64_bound]


def all_failures():
    out = []
    for chk in ALL_CHECKS:
        out += chk()
    return out


# ------------------------------------------------------------- the tests
@pytest.mark.parametrize("chk", ALL_CHECKS, ids=lambda f: f.__name__)
def test_oracle_pinned(chk):
    assert chk() == []


def test_golden_vectors_hold_both_chains():
    """Every f32 golden case and epilogue holds both chains, and on most cases
    the two differ, so the golden check pins each chain separately."""
    meta, data = _golden()
    differ = 0
    f32 = [c for c in meta if c["dtype"] == "f32"]
    for c in f32:
        assert c["chains"] == list(CHAINS)
        a, b = data[f"{c['name']}/Y_none_fma"], data[f"{c['name']}/Y_none_muladd"]
        differ += not np.array_equal(a.view(np.uint32), b.view(np.uint32))
        for tag in c["epilogues"]:
            assert f"{c['name']}/Y_{tag}_fma" in data and f"{c['name']}/Y_{tag}_muladd" in data
    assert differ >= len(f32) // 2, differ


def test_fma_and_muladd_chains_differ_somewhere():
    """The two rounding paths are distinguishable on the golden inputs, so the
    golden check really pins which one the oracle takes."""
    import exact
    _, data = _golden()
    X, W = data["f32_32x32x32/X"], data["f32_32x32x32/W"]
    a = exact.dense_f32_exact(X[:4], W, None, "none", 0.0, fma_path=True)
    b = exact.dense_f32_exact(X[:4], W, None, "none", 0.0, fma_path=False)
    assert not np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_chain_argument_is_checked():
    X = np.ones((2, 2), np.float32)
    with pytest.raises(KeyError):
        oracle.dense_f32(X, X, chain="fmaf")
    with pytest.raises(TypeError):
        oracle.dense_f32(X, X)  # the chain is never implied


@pytest.mark.parametrize("mutation", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11])
def test_planted_mistake_is_caught(mutation):
    assert all_failures() == []
    with oracle.mutation(mutation):
        caught = all_failures()
    assert caught, f"planted mistake {mutation} went unnoticed"
    assert all_failures() == []


def test_threads_do_not_change_results():
    rng = np.random.default_rng(7)
    X = rng.standard_normal((192, 128), dtype=np.float32)
    W = rng.standard_normal((128, 256), dtype=np.float32)
    b = rng.standard_normal(256, dtype=np.float32)
    for chain in CHAINS:
        y1 = oracle.dense_f32(X, W, b, "relu", chain=chain, threads=1)
        y4 = oracle.dense_f32(X, W, b, "relu", chain=chain, threads=4)
        assert np.array_equal(y1.view(np.uint32), y4.view(np.uint32))


def test_rows_are_independent():
    """A row subset gives the same bits as the full product (the GPU parity
    tests rely on this to check large shapes on sampled rows)."""
    rng = np.random.default_rng(8)
    X = rng.standard_normal((256, 128), dtype=np.float32)
    W = rng.standard_normal((128, 128), dtype=np.float32)
    b = rng.standard_normal(128, dtype=np.float32)
    rows = np.array([0, 5, 64, 200, 255])
    for chain in CHAINS:
        full = oracle.dense_f32(X, W, b, "relu", chain=chain)
        part = oracle.dense_f32(X[np.concatenate([rows, np.arange(64 - rows.size) + 1])], W, b, "relu",
                                chain=chain)
        assert np.array_equal(full[rows].view(np.uint32), part[:rows.size].view(np.uint32))
        assert math.isfinite(float(full.sum()))


# ------------------------------------------------ vectorised timing twin
@pytest.mark.parametrize("M, K, N", [(8, 8, 8), (64, 64, 64), (16, 256, 512), (192, 96, 40), (256, 1024, 192)])
@pytest.mark.parametrize("act", ["none", "relu", "leaky", "if_relu"])
def test_vector_twin_is_bit_identical(M, K, N, act):
    """oracle_dense_f32_vec (the bench's CPU baseline: the reference JIT's
    8x8x8 schedule on 8-wide FMA vectors) must round exactly like the scalar
    restatement of the fma chain it times, special values included."""
    rng = np.random.default_rng(M + K + N)
    X = rng.standard_normal((M, K), dtype=np.float32)
    W = rng.standard_normal((K, N), dtype=np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    X[0, 0] = np.nan
    if M > 1:
        X[1, 1] = np.inf
    b[-1] = -np.inf
    for bias in (b, None):
        ref = oracle.dense_f32(X, W, bias, act, 0.07, chain="fma")
        got = oracle.dense_f32_vec(X, W, bias, act, 0.07)
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("M, K, N", [(65, 8, 8), (8, 8, 9), (64, 12, 64)])
def test_vector_twin_needs_whole_tiles(M, K, N):
    with pytest.raises(ValueError, match="whole 8x8x8 tiles"):
        oracle.dense_f32_vec(np.ones((M, K), np.float32), np.ones((K, N), np.float32))
