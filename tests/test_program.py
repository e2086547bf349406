"""FunctionDef front end (include/edsl_hip_program.h), host side only.

The fixtures are the exact bytes the reference Python front end serializes
(tests/golden/make_wire_fixtures.py drove it end to end); each must decode to
the dense form its program spells, or be rejected with a reason. Nothing here
touches a GPU: decoding, matching, descriptor and shape validation all happen
before any device call.
"""
from __future__ import annotations

import ctypes
import json
import os

import numpy as np
import pytest

from mlir_edsl_hip import _native
from mlir_edsl_hip._mlir_backend import MLIRCompiler

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _cases():
    with open(os.path.join(GOLDEN, "wire_fixtures.json")) as f:
        return json.load(f)["cases"]


def _bytes(case) -> bytes:
    with open(os.path.join(GOLDEN, case["file"]), "rb") as f:
        return f.read()


DENSE = [c for c in _cases() if "reject" not in c["expected"]]
REJECT = [c for c in _cases() if "reject" in c["expected"]]


@pytest.fixture
def compiler():
    c = MLIRCompiler()
    c.set_target("gpu")  # as the front end does for a target="gpu" function
    yield c
    c.clear()


@pytest.mark.parametrize("case", DENSE, ids=lambda c: c["fixture"])
def test_reference_front_end_bytes_decode_to_their_dense_form(case, compiler):
    compiler.compile_function(_bytes(case))
    assert compiler.has_function(case["function"])
    got = compiler.function_form(case["function"])
    exp = case["expected"]
    for key in ("form", "dtype", "x", "w", "b", "epilogue"):
        if key in exp:
            assert got[key] == exp[key], (key, got, exp)
    if "alpha" in exp:
        assert got["alpha"] == pytest.approx(exp["alpha"], rel=1e-7)
    if "layers" in exp:
        assert len(got["layers"]) == len(exp["layers"])
        for g, e in zip(got["layers"], exp["layers"]):
            assert {k: g[k] for k in e} == e, (got["layers"], exp["layers"])
    else:
        assert len(got["layers"]) == 1
    assert compiler.get_function_pointer(case["function"]) != 0


@pytest.mark.parametrize("case", REJECT, ids=lambda c: c["fixture"])
def test_programs_outside_the_dense_path_are_rejected(case, compiler):
    with pytest.raises(RuntimeError, match=case["expected"]["reject"]):
        compiler.compile_function(_bytes(case))
    assert not compiler.has_function(case["function"])
    assert case["expected"]["reject"] in compiler.get_failure_ir()


def test_leaky_default_alpha_is_the_front_end_default(compiler):
    case = next(c for c in DENSE if c["fixture"] == "dense_leaky_default_f32")
    compiler.compile_function(_bytes(case))
    assert compiler.function_form(case["function"])["alpha"] == pytest.approx(0.01, rel=1e-7)


def test_registry_semantics(compiler):
    for c in DENSE[:4]:
        compiler.compile_function(_bytes(c))
    names = compiler.list_functions()
    assert names == sorted(c["function"] for c in DENSE[:4])
    with pytest.raises(RuntimeError, match="already compiled"):
        compiler.compile_function(_bytes(DENSE[0]))
    ptrs = {compiler.get_function_pointer(n) for n in names}
    assert len(ptrs) == len(names)
    ir = compiler.get_module_ir()
    assert all(f"func @{n}(" in ir for n in names)
    compiler.clear()
    assert compiler.list_functions() == [] and not compiler.has_function(names[0])


def test_unknown_function_pointer(compiler):
    with pytest.raises(RuntimeError, match="Function not compiled: nope"):
        compiler.get_function_pointer("nope")


def test_injected_failure_like_the_reference(compiler):
    # reference tests/core/test_ir_inspection.py:22-36
    case = DENSE[0]
    compiler.compile_function(_bytes(case))
    assert compiler.get_failure_ir() == ""
    compiler.inject_test_failure()
    with pytest.raises(RuntimeError, match="Lowering pipeline failed"):
        compiler.get_function_pointer(case["function"])
    fir = compiler.get_failure_ir()
    assert "__test_failure_inject__" in fir and case["function"] in fir
    assert case["function"] in compiler.get_module_ir()
    compiler.clear()
    assert compiler.get_failure_ir() == ""


def test_every_truncation_is_an_error_never_a_crash(compiler):
    data = _bytes(next(c for c in DENSE if c["fixture"] == "dense_relu_i32_tensor_map"))
    for n in range(len(data)):
        try:
            compiler.compile_function(data[:n])
        except RuntimeError:
            pass
        compiler.clear()


def test_random_corruption_is_an_error_never_a_crash(compiler):
    rng = np.random.default_rng(0)
    cases = [_bytes(c) for c in _cases()]
    for trial in range(3000):
        data = bytearray(cases[trial % len(cases)])
        for _ in range(1 + trial % 3):
            data[rng.integers(len(data))] = rng.integers(256)
        try:
            compiler.compile_function(bytes(data))
        except RuntimeError:
            pass
        compiler.clear()


def _varint(v: int) -> bytes:
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        out.append(b | (0x80 if v else 0))
        if not v:
            return bytes(out)


def test_unknown_fields_are_skipped(compiler):
    case = next(c for c in DENSE if c["fixture"] == "dense_relu_f32")
    data = _bytes(case)
    extra = (_varint(15 << 3 | 0) + _varint(123456789)           # varint
             + _varint(16 << 3 | 1) + bytes(8)                    # fixed64
             + _varint(17 << 3 | 2) + _varint(3) + b"abc"         # length-delimited
             + _varint(18 << 3 | 5) + bytes(4))                   # fixed32
    compiler.compile_function(extra + data)
    assert compiler.function_form(case["function"])["form"] == case["expected"]["form"]


def test_group_wire_type_is_rejected(compiler):
    with pytest.raises(RuntimeError, match="wire type"):
        compiler.compile_function(_varint(15 << 3 | 3) + _bytes(DENSE[0]))


def test_execute_checks_shapes_before_any_device_call(compiler):
    case = next(c for c in DENSE if c["fixture"] == "dense_relu_f32")
    compiler.compile_function(_bytes(case))
    X = np.zeros((16, 64), np.float32)
    W = np.zeros((64, 33), np.float32)  # compiled for 64 x 32
    b = np.zeros(32, np.float32)
    with pytest.raises(RuntimeError, match="shape"):
        compiler.execute_gpu_function(case["function"], [(a.ctypes.data, list(a.shape)) for a in (X, W, b)],
                                      [16, 32], 4)
    with pytest.raises(RuntimeError, match="element_size"):
        compiler.execute_gpu_function(case["function"], [(a.ctypes.data, list(a.shape)) for a in (X, X, b)],
                                      [16, 32], 8)
    with pytest.raises(RuntimeError, match="takes 3 inputs"):
        compiler.execute_gpu_function(case["function"], [(X.ctypes.data, [16, 64])], [16, 32], 4)


def _descriptor(a):
    return [a.ctypes.data, a.ctypes.data, 0] + list(a.shape) + [s // a.itemsize for s in a.strides]


def test_function_pointer_validates_descriptors_before_any_device_call(compiler):
    case = next(c for c in DENSE if c["fixture"] == "dense_relu_f32")
    compiler.compile_function(_bytes(case))
    ptr = compiler.get_function_pointer(case["function"])
    X = np.zeros((16, 64), np.float32)
    W = np.zeros((64, 40), np.float32)  # wrong N
    b = np.zeros(32, np.float32)
    Y = np.zeros((16, 32), np.float32)
    args = _descriptor(X) + _descriptor(W) + _descriptor(b) + _descriptor(Y)
    assert len(args) == 26
    ctypes.CFUNCTYPE(None, *([ctypes.c_int64] * 26))(ptr)(*args)
    code, msg = _native.last_error()
    assert code == -1 and "compiled for 32" in msg


def test_stale_function_pointer_after_clear(compiler):
    case = next(c for c in DENSE if c["fixture"] == "matmul_f32")
    compiler.compile_function(_bytes(case))
    ptr = compiler.get_function_pointer(case["function"])
    compiler.clear()
    A = np.zeros((32, 48), np.float32)
    B = np.zeros((48, 16), np.float32)
    C = np.zeros((32, 16), np.float32)
    ctypes.CFUNCTYPE(None, *([ctypes.c_int64] * 21))(ptr)(*(_descriptor(A) + _descriptor(B) + _descriptor(C)))
    code, msg = _native.last_error()
    assert code == -8 and "no longer bound" in msg


def _ld(field: int, payload: bytes) -> bytes:
    return _varint(field << 3 | 2) + _varint(len(payload)) + payload


def _tensor_type(shape, kind) -> bytes:
    # TypeSpec{tensor: TensorTypeSpec{shape (packed int64), element_type: TypeSpec{scalar{kind}}}}
    packed = b"".join(_varint(d & ((1 << 64) - 1)) for d in shape)
    scalar = _ld(1, _varint(1 << 3 | 0) + _varint(kind)) if kind else _ld(1, b"")
    return _ld(3, _ld(1, packed) + _ld(2, scalar))


def _param_node(name, shape, kind) -> bytes:
    # ASTNode{function: FunctionNode{parameter: Parameter{name, type}}}
    return _ld(4, _ld(1, _ld(1, name.encode()) + _ld(2, _tensor_type(shape, kind))))


def _matmul_def(name, a_shape, b_shape, out_shape, kind=1) -> bytes:
    body = _ld(7, _ld(2, _ld(1, _param_node("A", a_shape, kind)) + _ld(2, _param_node("B", b_shape, kind))
                      + _ld(3, _tensor_type(out_shape, kind))))
    return (_ld(1, name.encode())
            + _ld(2, _ld(1, b"A") + _ld(2, _tensor_type(a_shape, kind)))
            + _ld(2, _ld(1, b"B") + _ld(2, _tensor_type(b_shape, kind)))
            + _ld(3, _tensor_type(out_shape, kind)) + _ld(4, body))


def test_hand_encoded_matmul_decodes(compiler):
    """Cross-check of the field layout with an encoder written from the
    schema (not the reference front end): same result as the fixtures."""
    compiler.compile_function(_matmul_def("hand_mm", [8, 4], [4, 2], [8, 2]))
    f = compiler.function_form("hand_mm")
    assert (f["form"], f["dtype"], f["x"], f["w"], f["b"]) == ("A @ B", "f32", 0, 1, -1)
    compiler.compile_function(_matmul_def("hand_mm_i32", [8, 4], [4, 2], [8, 2], kind=0))
    assert compiler.function_form("hand_mm_i32")["dtype"] == "i32"


def test_dynamic_dimensions_are_rejected_like_the_reference(compiler):
    # reference cpp/src/MLIRBuilder.cpp:478-486
    with pytest.raises(RuntimeError, match="Dynamic tensor dimensions not supported"):
        compiler.compile_function(_matmul_def("dyn_mm", [-1, 4], [4, 2], [-1, 2]))


def test_shape_mismatches_are_rejected(compiler):
    with pytest.raises(RuntimeError, match="inner dimensions must match"):
        compiler.compile_function(_matmul_def("bad_k", [8, 4], [5, 2], [8, 2]))
    with pytest.raises(RuntimeError, match="return type"):
        compiler.compile_function(_matmul_def("bad_ret", [8, 4], [4, 2], [8, 3]))
    with pytest.raises(RuntimeError, match="f32 or i32"):
        compiler.compile_function(_matmul_def("bad_elem", [8, 4], [4, 2], [8, 2], kind=2))


# ------------------------------------------------ coexistence with the reference
class _StubReferenceCompiler:
    """Stands in for the reference's pybind MLIRCompiler (reference
    cpp/src/python_bindings.cpp:8-98): records what it is handed."""

    def __init__(self):
        self.fns: dict[str, str] = {}
        self.target = "cpu"
        self.injected = False
        self.opt = None
        self.capture = False

    def compile_function(self, data):
        assert data[0] == 0x0A  # FunctionDef.name, field 1
        name = bytes(data[2:2 + data[1]]).decode()
        if name in self.fns:
            raise RuntimeError(f"duplicate {name}")
        self.fns[name] = self.target

    def get_function_pointer(self, name):
        if self.injected:
            raise RuntimeError("Lowering pipeline failed: stub")
        return 0x5000 + sorted(self.fns).index(name)

    def has_function(self, name):
        return name in self.fns

    def list_functions(self):
        return sorted(self.fns)

    def get_module_ir(self):
        return "module { // stub reference }\n"

    def clear(self):
        self.fns.clear()
        self.injected = False

    def get_lowering_snapshots(self):
        return [("stub-pass", "ir")] if self.capture else []

    def enable_snapshot_capture(self):
        self.capture = True

    def get_failure_ir(self):
        return "func.func @__test_failure_inject__" if self.injected else ""

    def inject_test_failure(self):
        self.injected = True

    def set_optimization_level(self, level):
        self.opt = level

    def set_target(self, target):
        self.target = target

    def execute_gpu_function(self, name, inputs, output_shape, element_size):
        return b"stub:" + name.encode()


class _StubReferenceModule:
    MLIRCompiler = _StubReferenceCompiler


@pytest.fixture
def with_reference():
    from mlir_edsl_hip import _mlir_backend as mb
    mb.set_reference_backend(_StubReferenceModule)
    try:
        c = MLIRCompiler()
        yield c
        c.clear()
    finally:
        mb._reference_override = mb._UNSET


def _case(fixture):
    return next(c for c in _cases() if c["fixture"] == fixture)


def test_scalar_and_dense_functions_in_one_session(with_reference):
    """Routing is by target: target="gpu" programs compile on the HIP module,
    anything compiled for target="cpu" goes to the reference compiler (even a
    dense program); later calls are routed by name."""
    c = with_reference
    dense, scalar, mm = _case("dense_relu_f32"), _case("reject_scalar_function"), _case("matmul_f32")
    c.set_target("gpu")
    c.compile_function(_bytes(dense))
    assert c.backend_of(dense["function"]) == "hip"
    c.set_target("cpu")
    c.compile_function(_bytes(scalar))  # CPU JIT requested -> reference
    c.compile_function(_bytes(mm))  # CPU JIT requested -> reference, although it is dense
    assert c.backend_of(scalar["function"]) == "reference" and c.reference.fns[scalar["function"]] == "cpu"
    assert c.backend_of(mm["function"]) == "reference" and c.reference.fns[mm["function"]] == "cpu"
    assert c.list_functions() == sorted([dense["function"], scalar["function"], mm["function"]])
    assert all(c.has_function(n) for n in c.list_functions())
    assert c.get_function_pointer(scalar["function"]) == 0x5000 + sorted(c.reference.fns).index(scalar["function"])
    hip_ptr = c.get_function_pointer(dense["function"])
    assert hip_ptr and hip_ptr < 0x5000 or hip_ptr > 0x6000
    assert c.execute_gpu_function(mm["function"], [], [1], 4) == b"stub:" + mm["function"].encode()
    ir = c.get_module_ir()
    assert f"func @{dense['function']}(" in ir and "stub reference" in ir
    c.set_optimization_level(3)
    assert c.reference.opt == 3
    c.clear()
    assert c.list_functions() == [] and c.reference.fns == {}


def test_rejected_gpu_program_raises_the_decoder_message(with_reference):
    """A target="gpu" program outside the dense path is not handed to the
    reference module (built without GPU support on this host, reference
    cpp/src/MLIRCompiler.cpp:456-461): the HIP decoder's own message is
    raised at compile time and the reference compiler sees nothing."""
    c = with_reference
    c.set_target("gpu")
    for fixture in ("reject_scalar_function", "reject_layer_as_rhs"):
        case = _case(fixture)
        with pytest.raises(RuntimeError, match=case["expected"]["reject"]) as e:
            c.compile_function(_bytes(case))
        assert "is not a dense-path program" in str(e.value)
        assert not c.has_function(case["function"])
    assert c.reference.fns == {}
    assert c.list_functions() == []


def test_dense_errors_are_not_delegated(with_reference):
    """A duplicate dense function is an error of the HIP module, not a reason
    to hand the program to the reference compiler."""
    c = with_reference
    c.set_target("gpu")
    dense = _case("dense_relu_f32")
    c.compile_function(_bytes(dense))
    with pytest.raises(RuntimeError, match="already compiled"):
        c.compile_function(_bytes(dense))
    assert c.reference.fns == {}


def test_injected_failure_goes_to_the_reference_compiler(with_reference):
    # reference tests/core/test_ir_inspection.py:22-36: the scalar function runs on the reference
    c = with_reference
    c.set_target("cpu")
    scalar = _case("reject_scalar_function")
    c.compile_function(_bytes(scalar))
    c.inject_test_failure()
    with pytest.raises(RuntimeError, match="Lowering pipeline failed"):
        c.get_function_pointer(scalar["function"])
    assert "__test_failure_inject__" in c.get_failure_ir()


def test_snapshots_are_what_the_module_did(with_reference):
    c = with_reference
    c.set_target("gpu")
    c.enable_snapshot_capture()
    dense = _case("chain_relu_then_leaky")
    c.compile_function(_bytes(dense))
    c.get_function_pointer(dense["function"])
    snaps = dict(c.get_lowering_snapshots())
    text = snaps[f"match:{dense['function']}"]
    assert "leaky_relu(relu(X @ W1 + b1) @ W2, 0.1)" in text and "layer 1: x=-1 w=3 b=-1 epilogue=4" in text
    assert snaps["stub-pass"] == "ir"


def test_without_a_reference_module_other_programs_are_rejected():
    from mlir_edsl_hip import _mlir_backend as mb
    mb.set_reference_backend(None)
    try:
        c = MLIRCompiler()
        assert c.reference is None
        with pytest.raises(RuntimeError, match=_case("reject_scalar_function")["expected"]["reject"]):
            c.compile_function(_bytes(_case("reject_scalar_function")))
        c.set_target("cpu")  # no CPU JIT to hand it to: dense functions run on the HIP kernels
        c.compile_function(_bytes(_case("matmul_f32")))
        assert c.backend_of(_case("matmul_f32")["function"]) == "hip"
    finally:
        mb._reference_override = mb._UNSET


def test_module_text_describes_the_match(compiler):
    case = _case("chain_relu_then_leaky")
    compiler.compile_function(_bytes(case))
    ir = compiler.get_module_ir()
    assert "// form: leaky_relu(relu(X @ W1 + b1) @ W2, 0.1) (f32, 2 layers)" in ir
    assert "// layer 0: X @ W1 + b1, then relu" in ir and "// layer 1: h0 @ W2, then leaky_relu" in ir


# -------------------------------------------- binding: argument validation
def test_bind_parameter_validates_before_any_device_call(compiler):
    case = _case("dense_relu_f32")  # X[16,64], W[64,32], b[32]
    compiler.compile_function(_bytes(case))
    name = case["function"]
    with pytest.raises(RuntimeError, match=r"W: shape\[1\] = 33, the function was compiled for 32"):
        compiler.bind_parameter(name, "W", np.zeros((64, 33), np.float32))
    with pytest.raises(RuntimeError, match="no parameter 7"):
        compiler.bind_parameter(name, 7, np.zeros((64, 32), np.float32))
    with pytest.raises(RuntimeError, match="has no parameter 'Q'"):
        compiler.bind_parameter(name, "Q", np.zeros((64, 32), np.float32))
    with pytest.raises(RuntimeError, match="rank 2, the function was compiled for rank 1"):
        compiler.bind_parameter(name, "b", np.zeros((1, 32), np.float32))
    with pytest.raises(ValueError, match="C-contiguous"):
        compiler.bind_parameter(name, "W", np.zeros((32, 64), np.float32).T)
    with pytest.raises(TypeError, match="element size 8"):
        compiler.bind_parameter(name, "W", np.zeros((64, 32), np.float64))
    with pytest.raises(RuntimeError, match="Function not compiled: nope"):
        compiler.bind_parameter("nope", 0, np.zeros((64, 32), np.float32))
    compiler.unbind_parameter(name)  # nothing bound: a no-op
    with pytest.raises(RuntimeError, match="no parameter 5"):
        compiler.unbind_parameter(name, 5)


# ------------------------------------------- DYN-declared functions
def test_dyn_specialisations_compile_side_by_side(compiler):
    """A function declared with DYN dimensions is compiled once per call
    shape, under its name with the shapes appended (reference
    mlir_edsl/functions/signature.py:98-104, decorator.py:79-107). Both
    specialisations the front end serialized live in one compiler, each with
    its own concrete types and the dense form of the body."""
    for base in ("dyn_dense_relu_f32", "dyn_matmul_f32", "dyn_dense_relu_i32"):
        cases = [c for c in _cases() if c["fixture"].startswith(base + "__")]
        assert len(cases) == 2 and all(c.get("declared_dyn") for c in cases)
        stems = {c["function"].split("__")[0] for c in cases}
        assert len(stems) == 1, stems  # one DSL function, two variants
        for c in cases:
            compiler.compile_function(_bytes(c))
        ir = compiler.get_module_ir()
        for c in cases:
            form = compiler.function_form(c["function"])
            assert form["form"] == c["expected"]["form"] and form["dtype"] == c["expected"]["dtype"]
            (M, K), N = c["param_shapes"][0], c["param_shapes"][1][1]
            assert c["function"].endswith("__" + "__".join("_".join(map(str, s)) for s in c["param_shapes"]))
            dt = c["expected"]["dtype"]
            assert f"tensor<{M}x{K}x{dt}>" in ir and f"tensor<{M}x{N}x{dt}>" in ir
    assert len(compiler.list_functions()) == 6


def test_inner_dimension_mismatch_is_rejected_like_the_front_end(compiler):
    """The front end refuses a DYN matmul called with mismatched inner
    dimensions before serializing anything (reference
    tests/linalg/test_linalg_dyn.py:72-80, message recorded by the fixture
    generator). A FunctionDef that carries such shapes anyway (written here
    field by field) is refused by the decoder with the same words."""
    from mlir_edsl_hip import wire
    with open(os.path.join(GOLDEN, "wire_fixtures.json")) as f:
        rej = json.load(f)["front_end_rejections"]
    case = next(r for r in rej if r["case"] == "dyn_matmul_inner_mismatch")
    assert case["error"] == "TypeError" and not case["serialized"]
    assert "inner dimensions must match" in case["message"]
    tA, tB, tC = wire.tensor_type((2, 3), "f32"), wire.tensor_type((4, 2), "f32"), wire.tensor_type((2, 2), "f32")
    node = wire._linalg(2, wire._len(1, wire._param_node("A", tA)) + wire._len(2, wire._param_node("B", tB)) +
                        wire._len(3, tC))
    fdef = (wire._len(1, b"mismatch_0__2_3__4_2") + wire._len(2, wire._len(1, b"A") + wire._len(2, tA)) +
            wire._len(2, wire._len(1, b"B") + wire._len(2, tB)) + wire._len(3, tC) + wire._len(4, node))
    with pytest.raises(RuntimeError, match="inner dimensions must match"):
        compiler.compile_function(fdef)
    assert compiler.list_functions() == []


def test_f32_if_relu_forms_decode_by_their_float_semantics(compiler):
    """tensor_map If bodies over f32: v > 0 ? v : 0 is the If-ReLU epilogue
    (NaN and -0 give +0), v <= 0 ? 0 : v is arith.maximumf exactly, and the
    forms that keep -0 are refused."""
    got = {}
    for fx in ("matmul_if_relu_f32", "dense_if_relu_f32", "dense_relu_f32_tensor_map_le"):
        c = _case(fx)
        compiler.compile_function(_bytes(c))
        got[fx] = compiler.function_form(c["function"])["epilogue"]
    assert got == {"matmul_if_relu_f32": 6, "dense_if_relu_f32": 7, "dense_relu_f32_tensor_map_le": 3}
    c = _case("reject_f32_if_ge_relu")
    with pytest.raises(RuntimeError, match="keeps -0"):
        compiler.compile_function(_bytes(c))


def test_bound_array_is_held_until_unbound(compiler, monkeypatch):
    """The facade keeps the bound object alive while its snapshot is matched
    by address, and lets go on unbind, rebind and clear. (The device copy is
    stubbed out: this checks the facade's bookkeeping only.)"""
    import gc
    import weakref
    from mlir_edsl_hip import _mlir_backend as mb
    L = mb._L()
    monkeypatch.setattr(L, "edsl_hip_module_bind_parameter", lambda *a: 0)
    case = _case("dense_relu_f32")
    compiler.compile_function(_bytes(case))
    name = case["function"]

    def bound(param):
        a = np.ones(case["param_shapes"][compiler._param_index(name, param)], np.float32)
        compiler.bind_parameter(name, param, a)
        return weakref.ref(a)

    w, b = bound("W"), bound("b")
    gc.collect()
    assert w() is not None and b() is not None
    compiler.unbind_parameter(name, "W")
    gc.collect()
    assert w() is None and b() is not None
    b2 = bound("b")  # rebinding releases the previous object
    gc.collect()
    assert b() is None and b2() is not None
    compiler.clear()
    gc.collect()
    assert b2() is None
