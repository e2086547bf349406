"""FunctionDef bytes for the dense-path programs, without the front end.

``MLIRCompiler.compile_function`` takes a serialized ``mlir_edsl.FunctionDef``
(reference cpp/schemas/ast.proto:473-478). The reference front end writes
one from a decorated Python function; this module writes the same bytes
directly from shapes, for callers that drive the compiler on their own (the
benchmark's host-path workloads, tools, C++ embedders' tests). The encoding
follows the schema's field numbers and proto3's rules (default scalars are
omitted, repeated int64 is packed) in the order the front end emits fields,
so for the forms it supports the result is byte-identical to what the front
end produces (checked against recorded front-end bytes in the tests).

Supported: ``A @ B``, ``X @ W + b``, ``relu(...)`` and ``leaky_relu(...,
alpha)`` of either (f32), and chains of such layers whose input is the
previous layer. Field numbers used (cpp/schemas/ast.proto): TypeSpec.tensor 3,
ScalarTypeSpec.kind 1, TensorTypeSpec.shape 1 / element_type 2, ASTNode.function
4 / linalg 7, FunctionNode.parameter 1, Parameter.name 1 / type 2,
LinalgNode.matmul 2 / binary_op 8 / activation 9, LinalgMatmul lhs 1 / rhs 2 /
out_type 3, LinalgBinaryOp lhs 1 / rhs 2 / op_type 3 / broadcast 4 / out_type 5,
LinalgActivation input 1 / act_type 2 / alpha 3 / out_type 4,
FunctionParameter name 1 / type 2, FunctionDef name 1 / params 2 /
return_type 3 / body 4; enums ScalarTypeSpec.Kind (I32 0, F32 1),
ActivationType (RELU 0, LEAKY_RELU 1), BroadcastMode.TENSOR_BIAS_RIGHT 3.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from typing import Sequence

_KIND = {"i32": 0, "f32": 1}


def _varint(v: int) -> bytes:
    v &= (1 << 64) - 1  # negative int64 values take ten bytes, as in proto3
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _len(field: int, payload: bytes) -> bytes:
    return _varint(field << 3 | 2) + _varint(len(payload)) + payload


def _int(field: int, v: int) -> bytes:
    return b"" if v == 0 else _varint(field << 3) + _varint(v)


def _f32(field: int, v: float) -> bytes:
    return b"" if v == 0.0 else _varint(field << 3 | 5) + struct.pack("<f", v)


def tensor_type(shape: Sequence[int], dtype: str) -> bytes:
    """TypeSpec{tensor: TensorTypeSpec{shape, element_type: TypeSpec{scalar}}}."""
    packed = b"".join(_varint(int(d)) for d in shape)
    elem = _len(1, _int(1, _KIND[dtype]))  # TypeSpec.scalar = ScalarTypeSpec{kind}
    return _len(3, (_len(1, packed) if packed else b"") + _len(2, elem))


def _param_node(name: str, ttype: bytes) -> bytes:
    """ASTNode{function: FunctionNode{parameter: Parameter{name, type}}}."""
    return _len(4, _len(1, _len(1, name.encode()) + _len(2, ttype)))


def _linalg(field: int, payload: bytes) -> bytes:
    return _len(7, _len(field, payload))


@dataclass
class Layer:
    """One dense layer: h = act(input @ W (+ b)); `w` / `b` name parameters."""
    w: str
    n: int
    b: str | None = None
    act: str = "none"      # "none" | "relu" | "leaky"
    alpha: float = 0.01


def dense_program(name: str, x: tuple[str, int, int], layers: Sequence[Layer], dtype: str = "f32") -> bytes:
    """FunctionDef of ``act_n(... act_1(X @ W1 + b1) ... @ Wn + bn)``.

    x = (parameter name, M, K). Parameters are declared in the order X, then
    each layer's weight and bias, as a function written
    ``def f(X, W1, b1, W2, b2, ...)`` would declare them."""
    xname, M, K = x
    if dtype not in _KIND:
        raise ValueError(f"dtype {dtype!r}: f32 or i32")
    params = [(xname, tensor_type((M, K), dtype))]
    body = _param_node(xname, params[0][1])
    k = K
    for L in layers:
        if L.act != "none" and dtype != "f32":
            raise ValueError("the i32 ReLU is written with tensor_map(If), which this encoder does not emit")
        wt = tensor_type((k, L.n), dtype)
        out = tensor_type((M, L.n), dtype)
        params.append((L.w, wt))
        node = _linalg(2, _len(1, body) + _len(2, _param_node(L.w, wt)) + _len(3, out))
        if L.b is not None:
            bt = tensor_type((L.n,), dtype)
            params.append((L.b, bt))
            # op_type ADD (0) is the proto3 default and is omitted
            node = _linalg(8, _len(1, node) + _len(2, _param_node(L.b, bt)) + _int(4, 3) + _len(5, out))
        if L.act in ("relu", "leaky"):
            node = _linalg(9, _len(1, node) + _int(2, 1 if L.act == "leaky" else 0) +
                           (_f32(3, L.alpha) if L.act == "leaky" else b"") + _len(4, out))
        elif L.act != "none":
            raise ValueError(f"activation {L.act!r}")
        body = node
        k = L.n
    out = _len(1, name.encode())
    for pname, ptype in params:
        out += _len(2, _len(1, pname.encode()) + _len(2, ptype))
    out += _len(3, tensor_type((M, k), dtype)) + _len(4, body)
    return out


def dense_layer(name: str, M: int, K: int, N: int, dtype: str = "f32", bias: bool = True,
                act: str = "relu", alpha: float = 0.01) -> bytes:
    """FunctionDef of ``act(X @ W + b)`` (parameters X, W, b) or, without a
    bias, ``act(A @ B)`` (parameters A, B)."""
    if bias:
        return dense_program(name, ("X", M, K), [Layer("W", N, "b", act, alpha)], dtype)
    return dense_program(name, ("A", M, K), [Layer("B", N, None, act, alpha)], dtype)
