"""mlir_edsl_hip.wire: FunctionDef bytes written without the front end.

Pinned byte for byte against the bytes the reference front end serialized
for the same programs (tests/golden/wire/, recorded by
tests/golden/make_wire_fixtures.py), and decoded by the module's own
FunctionDef reader to the expected dense form at the benchmark shapes.
"""
from __future__ import annotations

import json
import os

import pytest

from mlir_edsl_hip import wire
from mlir_edsl_hip._mlir_backend import MLIRCompiler

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
L = wire.Layer

# fixture -> the same program written with the encoder, given the mangled
# function name the front end chose (f"{name}_{id}", the id from a
# process-wide counter; recorded in the fixture index)
PROGRAMS = {
    "dense_relu_f32": lambda n: wire.dense_layer(n, 16, 64, 32),
    "matmul_bias_f32": lambda n: wire.dense_layer(n, 8, 24, 40, act="none"),
    "matmul_f32": lambda n: wire.dense_layer(n, 32, 48, 16, bias=False, act="none"),
    "matmul_i32": lambda n: wire.dense_layer(n, 4, 4, 4, "i32", bias=False, act="none"),
    "matmul_relu_f32": lambda n: wire.dense_layer(n, 64, 64, 64, bias=False),
    "dense_leaky_f32": lambda n: wire.dense_layer(n, 16, 32, 64, act="leaky", alpha=0.2),
    "dense_leaky_default_f32": lambda n: wire.dense_layer(n, 16, 32, 64, act="leaky"),
    "dense_relu_f32_1024": lambda n: wire.dense_layer(n, 1024, 1024, 1024),
    "chain_two_layer_net": lambda n: wire.dense_program(
        n, ("X", 2, 4), [L("W1", 8, "b1", "relu"), L("W2", 3, "b2", "relu")]),
    "chain_three_layer_net": lambda n: wire.dense_program(
        n, ("X", 4, 8), [L("W1", 16, "b1", "relu"), L("W2", 8, "b2", "relu"), L("W3", 4, "b3", "relu")]),
    "chain_relu_no_bias": lambda n: wire.dense_program(
        n, ("X", 4, 4), [L("W1", 4, None, "relu"), L("W2", 4, None, "relu")]),
    "chain_relu_then_leaky": lambda n: wire.dense_program(
        n, ("X", 64, 128), [L("W1", 256, "b1", "relu"), L("W2", 64, None, "leaky", 0.1)]),
}


def _fixture(name):
    with open(os.path.join(GOLDEN, "wire_fixtures.json")) as f:
        case = next(c for c in json.load(f)["cases"] if c["fixture"] == name)
    with open(os.path.join(GOLDEN, case["file"]), "rb") as f:
        return case, f.read()


@pytest.mark.parametrize("fixture", sorted(PROGRAMS))
def test_encoder_writes_the_front_end_bytes(fixture):
    case, data = _fixture(fixture)
    assert PROGRAMS[fixture](case["function"]) == data, case["source"]


@pytest.mark.parametrize("M, K, N, bias, act, form", [
    (16, 8192, 8192, True, "relu", "relu(X @ W + b)"),
    (4096, 4096, 4096, True, "relu", "relu(X @ W + b)"),
    (256, 256, 256, False, "none", "A @ B"),
    (2048, 2048, 2048, True, "none", "X @ W + b"),
])
def test_benchmark_shapes_decode_to_their_form(M, K, N, bias, act, form):
    comp = MLIRCompiler()
    comp.compile_function(wire.dense_layer("f", M, K, N, bias=bias, act=act))
    got = comp.function_form("f")
    assert got["form"] == form and got["dtype"] == "f32"
    assert f"tensor<{M}x{K}xf32>" in comp.get_module_ir()
    comp.clear()


def test_integer_relu_is_not_written_as_an_activation():
    with pytest.raises(ValueError, match="tensor_map"):
        wire.dense_layer("f", 4, 4, 4, "i32", act="relu")
