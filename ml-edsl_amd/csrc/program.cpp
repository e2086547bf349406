// FunctionDef front end of the HIP dense path: compile a serialized
// mlir_edsl.FunctionDef (reference cpp/schemas/ast.proto:473-478) that the
// reference Python front end produced, recognise the dense-path program it
// spells, and bind it to the gfx950 kernels.
//
// This stands in for the reference's MLIRCompiler (cpp/src/MLIRCompiler.cpp:
// compileFunction :184-216, getFunctionPointer :277-280, hasFunction /
// listFunctions :314-320, clear, executeGPUFunction :352-461), restricted to
// the programs the HIP kernels implement:
//
//   matmul(A, B)                          A @ B
//   relu(A @ B)
//   X @ W + b        (bias on either side of the +)
//   relu(X @ W + b)  leaky_relu(X @ W + b, alpha)          (f32)
//   tensor_map(X @ W + b, lambda v: If(v > 0, v, 0))       (i32 ReLU, and
//                     tensor_map(A @ B, ...))
//
// with X, W, b function parameters. The wire format is decoded directly (no
// libprotobuf): proto3 varint / fixed32 / fixed64 / length-delimited fields,
// packed or unpacked repeated scalars, last-one-wins oneofs, unknown fields
// skipped. Field numbers and enum values are those of the reference schema
// (cpp/schemas/ast.proto: TypeSpec / ScalarTypeSpec / MemRefTypeSpec /
// TensorTypeSpec :13-54, enums :61-116, ASTNode :123-133, ScalarNode :136-143,
// ControlFlowNode :166-173, FunctionNode :176-181, BindingNode :184-189,
// Constant :196-203, Parameter :206-209, CompareOp :220-225, IfOp :228-233,
// LinalgNode :341-353, LinalgMatmul :364-368, LinalgBinaryOp :377-383,
// LinalgMap :387-392, LinalgMapElement :396-398, LinalgActivation :424-429,
// LetBinding :447-450, ValueReference :453-455, FunctionParameter :467-470,
// FunctionDef :473-478).
//
// get_function_pointer returns, per compiled function, an entry point with
// the reference JIT symbol's calling convention for THAT function: its
// parameters' expanded memref descriptors in the FunctionDef's parameter
// order followed by the out-param descriptor, void return
// (reference mlir_edsl/backend.py:162-198). Every such argument is a pointer
// or an int64 (the x86-64 SysV INTEGER class), so one trampoline taking N
// int64 arguments serves every parameter order of an N-argument function.

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/edsl_hip.h"
#include "../../include/edsl_hip_device.h"
#include "../../include/edsl_hip_program.h"
#include "runtime_internal.hpp"

namespace edsl {
namespace rt {
namespace {

// ============================================================ wire reader
struct Wire {
  const uint8_t* p;
  const uint8_t* end;

  bool done() const { return p >= end; }

  uint64_t varint() {
    uint64_t v = 0;
    for (int shift = 0;; shift += 7) {
      if (p >= end) fail(kErrProgram, "FunctionDef: truncated varint");
      if (shift > 63) fail(kErrProgram, "FunctionDef: varint longer than 10 bytes");
      const uint8_t b = *p++;
      v |= (uint64_t)(b & 0x7f) << shift;
      if (!(b & 0x80)) return v;
    }
  }
  uint32_t fixed32() {
    if (end - p < 4) fail(kErrProgram, "FunctionDef: truncated fixed32");
    uint32_t v;
    memcpy(&v, p, 4);
    p += 4;
    return v;
  }
  Wire sub() {
    const uint64_t n = varint();
    if (n > (uint64_t)(end - p)) fail(kErrProgram, "FunctionDef: length-delimited field overruns its message");
    Wire w{p, p + n};
    p += n;
    return w;
  }
  void skip(int wire_type) {
    switch (wire_type) {
      case 0: varint(); break;
      case 1:
        if (end - p < 8) fail(kErrProgram, "FunctionDef: truncated fixed64");
        p += 8;
        break;
      case 2: sub(); break;
      case 5: fixed32(); break;
      default: fail(kErrProgram, "FunctionDef: unsupported wire type %d", wire_type);
    }
  }
};

struct Field {
  int number;
  int wire_type;
};

Field next_field(Wire& w) {
  const uint64_t key = w.varint();
  const uint64_t number = key >> 3;
  if (number == 0 || number > 536870911u) fail(kErrProgram, "FunctionDef: bad field number");
  return Field{(int)number, (int)(key & 7)};
}

void expect(const Field& f, int wire_type, const char* what) {
  if (f.wire_type != wire_type)
    fail(kErrProgram, "FunctionDef: %s has wire type %d, expected %d", what, f.wire_type, wire_type);
}

std::string read_string(Wire& w) {
  Wire s = w.sub();
  return std::string(reinterpret_cast<const char*>(s.p), (size_t)(s.end - s.p));
}

float read_float(Wire& w) {
  const uint32_t bits = w.fixed32();
  float v;
  memcpy(&v, &bits, 4);
  return v;
}

// ================================================================== types
// ScalarTypeSpec.Kind
enum : int { kI32 = 0, kF32 = 1, kI1 = 2, kIndex = 3 };
// BinaryOpType, ActivationType, BroadcastMode, ComparisonPredicate values
enum : int { kOpAdd = 0 };
enum : int { kActRelu = 0, kActLeaky = 1 };
enum : int { kBcastNone = 0, kBiasRight = 3, kBiasLeft = 4 };
enum : int { kGT = 0, kLT = 1, kGE = 4, kLE = 5, kSLT = 6, kSLE = 7, kSGT = 8, kSGE = 9,
             kOLT = 14, kOLE = 15, kOGT = 16, kOGE = 17 };

struct TypeSpec {
  int kind = 0;  // 0 unset, 1 scalar, 2 memref, 3 tensor
  int scalar = kI32;             // kind 1
  std::vector<int64_t> shape;    // kind 2, 3
  int elem = -1;                 // kind 2, 3: scalar kind of the element, -1 if not a scalar
};

constexpr int kMaxDepth = 200;

TypeSpec read_type(Wire w, int depth);

void read_shape_and_elem(Wire w, TypeSpec& t, int depth) {
  while (!w.done()) {
    const Field f = next_field(w);
    if (f.number == 1) {  // repeated int64 shape, packed or not
      if (f.wire_type == 2) {
        Wire packed = w.sub();
        while (!packed.done()) t.shape.push_back((int64_t)packed.varint());
      } else {
        expect(f, 0, "shape");
        t.shape.push_back((int64_t)w.varint());
      }
    } else if (f.number == 2) {
      expect(f, 2, "element_type");
      const TypeSpec e = read_type(w.sub(), depth + 1);
      t.elem = e.kind == 1 ? e.scalar : -1;
    } else {
      w.skip(f.wire_type);
    }
  }
}

TypeSpec read_type(Wire w, int depth) {
  if (depth > kMaxDepth) fail(kErrProgram, "FunctionDef: type nesting too deep");
  TypeSpec t;
  while (!w.done()) {
    const Field f = next_field(w);
    if (f.number >= 1 && f.number <= 3) {
      expect(f, 2, "TypeSpec kind");
      Wire s = w.sub();
      t = TypeSpec{};
      t.kind = f.number;
      if (f.number == 1) {
        while (!s.done()) {
          const Field g = next_field(s);
          if (g.number == 1) {
            expect(g, 0, "ScalarTypeSpec.kind");
            t.scalar = (int)s.varint();
          } else {
            s.skip(g.wire_type);
          }
        }
      } else {
        read_shape_and_elem(s, t, depth);
      }
    } else {
      w.skip(f.wire_type);
    }
  }
  return t;
}

const char* scalar_name(int k) {
  switch (k) {
    case kI32: return "i32";
    case kF32: return "f32";
    case kI1: return "i1";
    case kIndex: return "index";
    default: return "?";
  }
}

std::string type_str(const TypeSpec& t) {
  if (t.kind == 1) return scalar_name(t.scalar);
  if (t.kind == 0) return "<none>";
  std::string s = t.kind == 2 ? "memref<" : "tensor<";
  for (int64_t d : t.shape) s += (d < 0 ? std::string("?") : std::to_string(d)) + "x";
  s += t.elem >= 0 ? scalar_name(t.elem) : "?";
  return s + ">";
}

// ================================================================ AST
enum class K {
  Empty, Other, Parameter, Constant, Compare, If, Matmul, BinaryOp, Activation, Map, MapElement, Let, Ref,
};

struct Node {
  K k = K::Empty;
  std::string text;   // Parameter: name; Other: what it is
  TypeSpec type;      // Parameter type, Constant type, result / out type
  int a = -1, b = -1, c = -1;  // children
  int64_t ival = 0;   // Constant int / bool
  float fval = 0.0f;  // Constant float, Activation alpha
  int cvalue = 0;     // Constant: 0 unset, 1 int, 2 float, 3 bool
  int op = 0;         // predicate, op_type, act_type
  int bcast = 0;
  int64_t id = 0;     // Let / Ref / MapElement node id, Map element_node_id
};

struct Ast {
  std::vector<Node> nodes;
  std::map<int64_t, int> lets;  // LetBinding node_id -> value node

  int add(Node n) {
    nodes.push_back(std::move(n));
    return (int)nodes.size() - 1;
  }
  int other(const char* what) {
    Node n;
    n.k = K::Other;
    n.text = what;
    return add(std::move(n));
  }

  int read_node(Wire w, int depth);
  int read_scalar(Wire w, int depth);
  int read_control(Wire w, int depth);
  int read_function(Wire w, int depth);
  int read_binding(Wire w, int depth);
  int read_linalg(Wire w, int depth);
};

// Reads a message whose fields are (child ASTNode | TypeSpec | varint |
// fixed32 float) by field number, into node n. `children` maps field numbers
// to the child slots a, b, c.
struct Layout {
  int child[3] = {0, 0, 0};   // field numbers of a, b, c (0 = none)
  int type_field = 0;
  int op_field = 0;           // varint -> n.op
  int bcast_field = 0;        // varint -> n.bcast
  int id_field = 0;           // varint -> n.id
  int float_field = 0;        // fixed32 -> n.fval
};

void read_with_layout(Ast& ast, Wire w, int depth, Node& n, const Layout& L) {
  while (!w.done()) {
    const Field f = next_field(w);
    int slot = -1;
    for (int i = 0; i < 3; ++i)
      if (L.child[i] && f.number == L.child[i]) slot = i;
    if (slot >= 0) {
      expect(f, 2, "child node");
      const int c = ast.read_node(w.sub(), depth + 1);
      (slot == 0 ? n.a : slot == 1 ? n.b : n.c) = c;
    } else if (L.type_field && f.number == L.type_field) {
      expect(f, 2, "type");
      n.type = read_type(w.sub(), depth + 1);
    } else if (L.op_field && f.number == L.op_field) {
      expect(f, 0, "enum");
      n.op = (int)w.varint();
    } else if (L.bcast_field && f.number == L.bcast_field) {
      expect(f, 0, "broadcast");
      n.bcast = (int)w.varint();
    } else if (L.id_field && f.number == L.id_field) {
      expect(f, 0, "node id");
      n.id = (int64_t)w.varint();
    } else if (L.float_field && f.number == L.float_field) {
      expect(f, 5, "float");
      n.fval = read_float(w);
    } else {
      w.skip(f.wire_type);
    }
  }
}

int Ast::read_node(Wire w, int depth) {
  if (depth > kMaxDepth) fail(kErrProgram, "FunctionDef: expression nesting too deep");
  int result = -1;
  while (!w.done()) {
    const Field f = next_field(w);
    if (f.number < 1 || f.number > 7) {
      w.skip(f.wire_type);
      continue;
    }
    expect(f, 2, "ASTNode");
    Wire s = w.sub();
    switch (f.number) {  // oneof node: the last one present wins
      case 1: result = read_scalar(s, depth); break;
      case 2: result = other("array (memref) operation"); break;
      case 3: result = read_control(s, depth); break;
      case 4: result = read_function(s, depth); break;
      case 5: result = read_binding(s, depth); break;
      case 6: result = other("tensor element operation"); break;
      case 7: result = read_linalg(s, depth); break;
    }
  }
  if (result < 0) {
    Node n;
    n.k = K::Empty;
    result = add(std::move(n));
  }
  return result;
}

int Ast::read_scalar(Wire w, int depth) {
  int result = other("empty scalar node");
  while (!w.done()) {
    const Field f = next_field(w);
    if (f.number < 1 || f.number > 4) {
      w.skip(f.wire_type);
      continue;
    }
    expect(f, 2, "ScalarNode");
    Wire s = w.sub();
    if (f.number == 1) {  // Constant
      Node n;
      n.k = K::Constant;
      while (!s.done()) {
        const Field g = next_field(s);
        if (g.number == 1) {
          expect(g, 0, "Constant.int_value");
          n.ival = (int64_t)(int32_t)(uint32_t)s.varint();
          n.cvalue = 1;
        } else if (g.number == 2) {
          expect(g, 5, "Constant.float_value");
          n.fval = read_float(s);
          n.cvalue = 2;
        } else if (g.number == 3) {
          expect(g, 0, "Constant.bool_value");
          n.ival = s.varint() != 0;
          n.cvalue = 3;
        } else if (g.number == 4) {
          expect(g, 2, "Constant.type");
          n.type = read_type(s.sub(), depth + 1);
        } else {
          s.skip(g.wire_type);
        }
      }
      result = add(std::move(n));
    } else if (f.number == 3) {  // CompareOp
      Node n;
      n.k = K::Compare;
      Layout L;
      L.op_field = 1;
      L.child[0] = 2;
      L.child[1] = 3;
      L.type_field = 4;
      read_with_layout(*this, s, depth, n, L);
      result = add(std::move(n));
    } else {
      result = other(f.number == 2 ? "scalar arithmetic" : "cast");
    }
  }
  return result;
}

int Ast::read_control(Wire w, int depth) {
  int result = other("empty control-flow node");
  while (!w.done()) {
    const Field f = next_field(w);
    if (f.number < 1 || f.number > 4) {
      w.skip(f.wire_type);
      continue;
    }
    expect(f, 2, "ControlFlowNode");
    Wire s = w.sub();
    if (f.number == 1) {  // IfOp
      Node n;
      n.k = K::If;
      Layout L;
      L.child[0] = 1;
      L.child[1] = 2;
      L.child[2] = 3;
      L.type_field = 4;
      read_with_layout(*this, s, depth, n, L);
      result = add(std::move(n));
    } else {
      result = other("for loop");
    }
  }
  return result;
}

int Ast::read_function(Wire w, int depth) {
  int result = other("empty function node");
  while (!w.done()) {
    const Field f = next_field(w);
    if (f.number < 1 || f.number > 2) {
      w.skip(f.wire_type);
      continue;
    }
    expect(f, 2, "FunctionNode");
    Wire s = w.sub();
    if (f.number == 1) {  // Parameter
      Node n;
      n.k = K::Parameter;
      while (!s.done()) {
        const Field g = next_field(s);
        if (g.number == 1) {
          expect(g, 2, "Parameter.name");
          n.text = read_string(s);
        } else if (g.number == 2) {
          expect(g, 2, "Parameter.type");
          n.type = read_type(s.sub(), depth + 1);
        } else {
          s.skip(g.wire_type);
        }
      }
      result = add(std::move(n));
    } else {
      result = other("function call");
    }
  }
  return result;
}

int Ast::read_binding(Wire w, int depth) {
  int result = other("empty binding node");
  while (!w.done()) {
    const Field f = next_field(w);
    if (f.number < 1 || f.number > 2) {
      w.skip(f.wire_type);
      continue;
    }
    expect(f, 2, "BindingNode");
    Wire s = w.sub();
    Node n;
    n.k = f.number == 1 ? K::Let : K::Ref;
    Layout L;
    L.id_field = 1;
    if (f.number == 1) L.child[0] = 2;
    read_with_layout(*this, s, depth, n, L);
    if (n.k == K::Let) {
      if (n.a < 0) fail(kErrProgram, "FunctionDef: LetBinding %lld has no value", (long long)n.id);
      lets[n.id] = n.a;
    }
    result = add(std::move(n));
  }
  return result;
}

int Ast::read_linalg(Wire w, int depth) {
  int result = other("empty linalg node");
  while (!w.done()) {
    const Field f = next_field(w);
    if (f.number < 1 || f.number > 9) {
      w.skip(f.wire_type);
      continue;
    }
    expect(f, 2, "LinalgNode");
    Wire s = w.sub();
    Node n;
    Layout L;
    switch (f.number) {
      case 2:  // LinalgMatmul
        n.k = K::Matmul;
        L.child[0] = 1;
        L.child[1] = 2;
        L.type_field = 3;
        break;
      case 3:  // LinalgMap
        n.k = K::Map;
        L.child[0] = 1;
        L.child[1] = 2;
        L.id_field = 3;
        L.type_field = 4;
        break;
      case 4:  // LinalgMapElement
        n.k = K::MapElement;
        L.id_field = 1;
        break;
      case 8:  // LinalgBinaryOp
        n.k = K::BinaryOp;
        L.child[0] = 1;
        L.child[1] = 2;
        L.op_field = 3;
        L.bcast_field = 4;
        L.type_field = 5;
        break;
      case 9:  // LinalgActivation
        n.k = K::Activation;
        L.child[0] = 1;
        L.op_field = 2;
        L.float_field = 3;
        L.type_field = 4;
        break;
      default:
        result = other(f.number == 1 ? "linalg.dot" : f.number >= 5 && f.number <= 7 ? "linalg.reduce"
                                                                                     : "linalg op");
        continue;
    }
    read_with_layout(*this, s, depth, n, L);
    result = add(std::move(n));
  }
  return result;
}

// ============================================================= programs
struct Param {
  std::string name;
  TypeSpec type;
};

// One dense layer: H = epilogue(input @ W (+ b)). The input is a parameter
// for the first layer of a chain and the previous layer's output after it.
struct Layer {
  int x = -1;  // parameter index of the input; -1: the previous layer's output
  int w = -1, b = -1;
  int epi = EDSL_EPI_NONE;
  float alpha = 0.0f;
};

// A parameter bound to a device-resident snapshot (bind_parameter): calls
// that pass the same host address with the same layout read the snapshot in
// place instead of copying the operand in.
struct Binding {
  const void* host = nullptr;  // address the snapshot was taken from
  int64_t rows = 0, cols = 0;  // its layout: `rows` contiguous rows of `cols` (1-D: rows == 1)
  std::shared_ptr<ResidentCopy> copy;
};

struct Bindings {
  std::mutex mu;
  std::map<int, Binding> by_param;  // parameter index -> binding
  std::string last_plan;            // kernels of the function's last successful run
};

struct Program {
  std::string name;
  std::vector<Param> params;
  TypeSpec ret;
  int dtype = EDSL_DTYPE_F32;
  std::vector<Layer> layers;   // in execution order
  int slot = -1;               // trampoline slot
  int nargs = 0;               // flat scalar arguments of the memref calling convention
  std::string form;            // e.g. "relu(relu(X @ W1 + b1) @ W2 + b2)"
  std::shared_ptr<Bindings> bound = std::make_shared<Bindings>();
};

const char* kDenseForms =
    "matmul(A, B), relu(A @ B), X @ W + b, relu(X @ W + b), leaky_relu(X @ W + b, alpha), "
    "tensor_map(X @ W [+ b], lambda v: If(v > 0, v, 0)) over i32 or f32, and chains of these layers "
    "(h @ W2 + b2 with h a previous layer), with A, B, X, W, b parameters";

struct Matcher {
  const Ast& ast;
  Program& prog;

  [[noreturn]] void reject(const char* fmt, ...) __attribute__((format(printf, 2, 3))) {
    char buf[400];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    fail(kErrProgram, "function '%s' is not a dense-path program (%s); the HIP backend runs %s",
         prog.name.c_str(), buf, kDenseForms);
  }

  // Follows LetBinding / ValueReference to the bound expression.
  const Node& res(int i) const {
    for (int hops = 0; hops < kMaxDepth; ++hops) {
      if (i < 0 || i >= (int)ast.nodes.size()) fail(kErrProgram, "FunctionDef: missing expression");
      const Node& n = ast.nodes[i];
      if (n.k == K::Let) {
        i = n.a;
      } else if (n.k == K::Ref) {
        auto it = ast.lets.find(n.id);
        if (it == ast.lets.end())
          fail(kErrProgram, "FunctionDef: ValueReference to unbound node id %lld", (long long)n.id);
        i = it->second;
      } else {
        return n;
      }
    }
    fail(kErrProgram, "FunctionDef: binding chain too long");
  }

  const char* kind_name(const Node& n) const {
    switch (n.k) {
      case K::Empty: return "empty node";
      case K::Other: return n.text.c_str();
      case K::Parameter: return "parameter";
      case K::Constant: return "constant";
      case K::Compare: return "comparison";
      case K::If: return "If";
      case K::Matmul: return "matmul";
      case K::BinaryOp: return "element-wise binary op";
      case K::Activation: return "activation";
      case K::Map: return "tensor_map";
      case K::MapElement: return "tensor_map element";
      default: return "binding";
    }
  }

  int param_index(const Node& n, const char* role) {
    if (n.k != K::Parameter) reject("the %s operand is not a function parameter (found: %s)", role, kind_name(n));
    for (size_t i = 0; i < prog.params.size(); ++i)
      if (prog.params[i].name == n.text) return (int)i;
    fail(kErrProgram, "FunctionDef: parameter '%s' is not declared by function '%s'", n.text.c_str(),
         prog.name.c_str());
  }

  // The lhs of a matmul is a parameter or, in a chain, a whole earlier
  // layer, which is appended to prog.layers before the layer that reads it.
  void matmul(const Node& n, Layer& L, int depth) {
    if (n.k != K::Matmul) reject("expected a matmul, found: %s", kind_name(n));
    const Node& lhs = res(n.a);
    if (lhs.k == K::Parameter) {
      L.x = param_index(lhs, "matmul lhs");
    } else if (lhs.k == K::Activation || lhs.k == K::Map || lhs.k == K::BinaryOp || lhs.k == K::Matmul) {
      layer(lhs, depth + 1);
      L.x = -1;
    } else {
      reject("the matmul lhs operand is not a function parameter or a dense layer (found: %s)",
             kind_name(lhs));
    }
    L.w = param_index(res(n.b), "matmul rhs");
  }

  // matmul, or matmul + bias (bias on either side: addf / addi commute bit for bit)
  void affine(const Node& n, Layer& L, int depth) {
    if (n.k == K::Matmul) {
      matmul(n, L, depth);
      return;
    }
    if (n.k != K::BinaryOp) reject("expected matmul or matmul + bias, found: %s", kind_name(n));
    if (n.op != kOpAdd) reject("element-wise op %d: only the bias add is fused", n.op);
    if (n.bcast == kBiasRight) {
      matmul(res(n.a), L, depth);
      L.b = param_index(res(n.b), "bias");
    } else if (n.bcast == kBiasLeft) {
      L.b = param_index(res(n.a), "bias");
      matmul(res(n.b), L, depth);
    } else {
      reject("element-wise add with broadcast mode %d: only the [M,N] + [N] bias is fused", n.bcast);
    }
    L.epi |= EDSL_EPI_BIAS;
  }

  bool is_elem(const Node& n, int64_t id) const { return n.k == K::MapElement && n.id == id; }
  bool is_zero(const Node& n) const {
    return n.k == K::Constant &&
           ((n.cvalue == 1 && n.ival == 0) || (n.cvalue == 2 && n.fval == 0.0f) || n.cvalue == 0);
  }
  bool is_negative_zero(const Node& n) const { return n.k == K::Constant && n.cvalue == 2 && std::signbit(n.fval); }

  // The activation a tensor_map body If(cmp, t, e) computes, as its epilogue
  // bits: EDSL_EPI_RELU (on i32 every spelling of max(v, 0); on f32 the one
  // with arith.maximumf's semantics), EDSL_EPI_IF_RELU (f32 v > 0 ? v : +0),
  // or a rejection.
  int map_activation(const Node& body, int64_t id, bool f32) {
    const char* not_relu = "tensor_map body is not If(v > 0, v, 0) (or an equivalent ReLU)";
    if (body.k != K::If) reject("%s", not_relu);
    const Node& c = res(body.a);
    const Node& t = res(body.b);
    const Node& e = res(body.c);
    if (c.k != K::Compare) reject("%s", not_relu);
    const Node& l = res(c.a);
    const Node& r = res(c.b);
    // The comparison as "v OP 0": strict or weak, greater or less.
    enum { kStrictGt, kWeakGt, kStrictLt, kWeakLt };
    int dir;
    switch (c.op) {
      case kGT: case kSGT: case kOGT: dir = kStrictGt; break;
      case kGE: case kSGE: case kOGE: dir = kWeakGt; break;
      case kLT: case kSLT: case kOLT: dir = kStrictLt; break;
      case kLE: case kSLE: case kOLE: dir = kWeakLt; break;
      default: reject("%s", not_relu);
    }
    if (is_zero(l) && is_elem(r, id)) {
      dir = dir == kStrictGt ? kStrictLt : dir == kWeakGt ? kWeakLt : dir == kStrictLt ? kStrictGt : kWeakGt;  // 0 < v is v > 0
    } else if (!(is_elem(l, id) && is_zero(r))) {
      reject("%s", not_relu);
    }
    // "v is positive" selects v, the other branch selects the zero.
    const bool then_is_v = dir == kStrictGt || dir == kWeakGt;
    const Node& v_branch = then_is_v ? t : e;
    const Node& zero_branch = then_is_v ? e : t;
    if (!is_elem(v_branch, id) || !is_zero(zero_branch)) reject("%s", not_relu);
    if (!f32) return EDSL_EPI_RELU;
    // f32: the reference builds arith.cmpf with ordered predicates only
    // (ArithBuilder.cpp:122-138), false whenever v is NaN; and -0 compares
    // equal to 0. Of the four spellings, v > 0 ? v : 0 maps NaN and -0 to +0,
    // and v <= 0 ? 0 : v is arith.maximumf exactly (NaN propagates, -0 -> +0).
    if (c.op != kOGT && c.op != kOGE && c.op != kOLT && c.op != kOLE)
      reject("float comparison predicate %d is not one the reference lowers", c.op);
    if (is_negative_zero(zero_branch))
      reject("tensor_map body selects -0.0, which no fused epilogue writes; select 0.0");
    if (dir == kStrictGt) return EDSL_EPI_IF_RELU;
    if (dir == kWeakLt) return EDSL_EPI_RELU;
    reject("tensor_map body If(v >= 0, v, 0) / If(v < 0, 0, v) over f32 keeps -0 (and the latter NaN), which no "
           "fused epilogue computes; write If(v > 0.0, v, 0.0) or relu()");
  }

  // One layer rooted at n (activation / tensor_map ReLU / affine); its
  // input layers are appended first, then the layer itself.
  void layer(const Node& n, int depth) {
    if (depth > 64) reject("more than 64 chained layers");
    Layer L;
    if (n.k == K::Activation) {
      if (n.op == kActRelu) {
        L.epi |= EDSL_EPI_RELU;
        if (prog.dtype == EDSL_DTYPE_I32)
          fail(kErrProgram,
               "function '%s': relu() emits arith.maximumf, which is float-only; write the integer ReLU "
               "as tensor_map(y, lambda v: If(v > 0, v, 0))",
               prog.name.c_str());
      } else if (n.op == kActLeaky) {
        L.epi |= EDSL_EPI_LEAKY;
        L.alpha = n.fval;
      } else {
        reject("activation type %d", n.op);
      }
      affine(res(n.a), L, depth);
    } else if (n.k == K::Map) {
      L.epi |= map_activation(res(n.b), n.id, prog.dtype == EDSL_DTYPE_F32);
      affine(res(n.a), L, depth);
    } else {
      affine(n, L, depth);
    }
    prog.layers.push_back(L);
  }
};

void check_types(Program& p) {
  auto tensor = [&](int idx, size_t rank, const char* role) -> const TypeSpec& {
    const TypeSpec& t = p.params[idx].type;
    if (t.kind != 3 || t.shape.size() != rank)
      fail(kErrProgram, "function '%s': %s '%s' must be a %zu-D tensor, got %s", p.name.c_str(), role,
           p.params[idx].name.c_str(), rank, type_str(t).c_str());
    for (int64_t d : t.shape)
      if (d < 0) fail(kErrProgram, "Dynamic tensor dimensions not supported");
    return t;
  };
  const TypeSpec& X = tensor(p.layers[0].x, 2, "matmul lhs");
  if (X.elem == kF32)
    p.dtype = EDSL_DTYPE_F32;
  else if (X.elem == kI32)
    p.dtype = EDSL_DTYPE_I32;
  else
    fail(kErrProgram, "function '%s': element type %s is not f32 or i32", p.name.c_str(), scalar_name(X.elem));
  const int64_t M = X.shape[0];
  int64_t K = X.shape[1];
  std::string lhs = type_str(X);
  for (const Layer& L : p.layers) {
    const TypeSpec& W = tensor(L.w, 2, "matmul rhs");
    if (W.elem != X.elem)
      fail(kErrProgram, "function '%s': matmul operand element types must match, got %s and %s",
           p.name.c_str(), lhs.c_str(), type_str(W).c_str());
    if (W.shape[0] != K)
      fail(kErrProgram, "function '%s': matmul inner dimensions must match, got lhs shape %s and rhs shape %s",
           p.name.c_str(), lhs.c_str(), type_str(W).c_str());
    const int64_t N = W.shape[1];
    if (L.b >= 0) {
      const TypeSpec& B = tensor(L.b, 1, "bias");
      if (B.elem != X.elem || B.shape[0] != N)
        fail(kErrProgram, "function '%s': bias %s does not broadcast over [%lld, %lld]", p.name.c_str(),
             type_str(B).c_str(), (long long)M, (long long)N);
    }
    if ((L.epi >> 1) == 2 && p.dtype != EDSL_DTYPE_F32)
      fail(kErrProgram, "function '%s': leaky_relu is float-only", p.name.c_str());
    K = N;
    lhs = "tensor<" + std::to_string(M) + "x" + std::to_string(N) + "x" + scalar_name(X.elem) + ">";
  }
  if (p.ret.kind != 3 || p.ret.shape.size() != 2 || p.ret.shape[0] != M || p.ret.shape[1] != K ||
      p.ret.elem != X.elem)
    fail(kErrProgram, "function '%s': return type %s does not match the result tensor<%lldx%lldx%s>",
         p.name.c_str(), type_str(p.ret).c_str(), (long long)M, (long long)K, scalar_name(X.elem));
}

std::string form_of(const Program& p) {
  std::string h;
  for (const Layer& L : p.layers) {
    const std::string in = L.x >= 0 ? p.params[L.x].name : h;
    std::string aff = in + " @ " + p.params[L.w].name;
    if (L.b >= 0) aff += " + " + p.params[L.b].name;
    switch (L.epi >> 1) {
      case 1: h = "relu(" + aff + ")"; break;
      case 3: h = "tensor_map(" + aff + ", lambda v: If(v > 0.0, v, 0.0))"; break;
      case 2: {
        char a[32];
        snprintf(a, sizeof(a), "%g", (double)L.alpha);
        h = "leaky_relu(" + aff + ", " + a + ")";
        break;
      }
      default: h = L.x >= 0 || p.layers.size() == 1 ? aff : "(" + aff + ")"; break;
    }
  }
  return h;
}

Program decode_function_def(const void* bytes, size_t len) {
  if (!bytes && len) fail(kErrArgument, "null FunctionDef bytes");
  Wire w{static_cast<const uint8_t*>(bytes), static_cast<const uint8_t*>(bytes) + len};
  Program p;
  Ast ast;
  int body = -1;
  while (!w.done()) {
    const Field f = next_field(w);
    if (f.number == 1) {
      expect(f, 2, "FunctionDef.name");
      p.name = read_string(w);
    } else if (f.number == 2) {
      expect(f, 2, "FunctionDef.params");
      Wire s = w.sub();
      Param prm;
      while (!s.done()) {
        const Field g = next_field(s);
        if (g.number == 1) {
          expect(g, 2, "FunctionParameter.name");
          prm.name = read_string(s);
        } else if (g.number == 2) {
          expect(g, 2, "FunctionParameter.type");
          prm.type = read_type(s.sub(), 1);
        } else {
          s.skip(g.wire_type);
        }
      }
      if (prm.type.kind == 0) fail(kErrProgram, "Parameter '%s': unsupported type", prm.name.c_str());
      p.params.push_back(std::move(prm));
    } else if (f.number == 3) {
      expect(f, 2, "FunctionDef.return_type");
      p.ret = read_type(w.sub(), 1);
    } else if (f.number == 4) {
      expect(f, 2, "FunctionDef.body");
      body = ast.read_node(w.sub(), 1);
    } else {
      w.skip(f.wire_type);
    }
  }
  if (p.name.empty()) fail(kErrProgram, "FunctionDef has no name");
  if (p.ret.kind == 0) fail(kErrProgram, "Unsupported return type");
  if (body < 0) fail(kErrProgram, "function '%s' has no body", p.name.c_str());
  for (size_t i = 0; i < p.params.size(); ++i)
    for (size_t j = 0; j < i; ++j)
      if (p.params[i].name == p.params[j].name)
        fail(kErrProgram, "function '%s': parameter '%s' declared twice", p.name.c_str(), p.params[i].name.c_str());
  Matcher m{ast, p};
  // Element type first (from the result): the integer ReLU forms depend on it.
  p.dtype = (p.ret.kind == 3 && p.ret.elem == kI32) ? EDSL_DTYPE_I32 : EDSL_DTYPE_F32;
  m.layer(m.res(body), 0);
  check_types(p);
  p.nargs = 7;  // out-param memref
  for (const Param& prm : p.params) p.nargs += 3 + 2 * (int)prm.type.shape.size();
  p.form = form_of(p);
  return p;
}

// ============================================================ trampolines
// Flat argument counts served by function pointers: X (7) + out (7) plus, per
// layer, W (7) and an optional bias (5), for 1 to 4 layers with all parameters
// distinct; a parameter used twice (A @ A) lowers the count, giving 14 and 19.
// Programs of any other count run through execute_gpu_function.
constexpr int kNumArities = 16;
constexpr int kArities[kNumArities] = {14, 19, 21, 26, 28, 33, 35, 38, 40, 42, 45, 47, 50, 52, 57, 62};
constexpr int kSlots = 64;  // function pointers per arity
std::mutex g_slot_mu;
std::shared_ptr<const Program> g_slot[kNumArities][kSlots];

int arity_index(int nargs) {
  for (int a = 0; a < kNumArities; ++a)
    if (kArities[a] == nargs) return a;
  return -1;
}

// The layer operations of p over its call operands (mats / vecs indexed by
// parameter), run with the chain executor. A parameter with a device-resident
// binding on the current device is read from its snapshot when the call
// passes the address and layout the snapshot was taken from; any other
// operand is copied in as usual. The snapshots are held until the
// (synchronous) run has finished, so an unbind or rebind on another thread
// cannot free one in use.
void run_program(const Program& p, std::vector<Mat> mats, std::vector<Vec> vecs, const Mat& Y) {
  std::vector<std::shared_ptr<ResidentCopy>> hold;
  std::string resident;
  {
    std::lock_guard<std::mutex> lock(p.bound->mu);
    if (!p.bound->by_param.empty()) {
      const int dev = current_device();
      for (auto& kv : p.bound->by_param) {
        const int i = kv.first;
        const Binding& b = kv.second;
        if (b.copy->device != dev) continue;
        bool hit = false;
        if (p.params[i].type.shape.size() == 2) {
          Mat& m = mats[i];
          if (m.base == b.host && m.rows == b.rows && m.cols == b.cols && (m.rows <= 1 || m.ld == b.cols)) {
            m.base = static_cast<char*>(b.copy->dev);
            m.ld = b.copy->dev_ld;
            hit = true;
          }
        } else {
          Vec& v = vecs[i];
          if (v.base == b.host && v.n == b.cols) {
            v.base = static_cast<char*>(b.copy->dev);
            hit = true;
          }
        }
        if (hit) {
          hold.push_back(b.copy);
          resident += (resident.empty() ? "" : ",") + p.params[i].name;
        }
      }
    }
  }
  std::vector<LayerOp> ops;
  ops.reserve(p.layers.size());
  for (const Layer& L : p.layers)
    ops.push_back(LayerOp{L.x >= 0 ? &mats[L.x] : nullptr, &mats[L.w], L.b >= 0 ? &vecs[L.b] : nullptr, L.epi,
                          L.alpha});
  sync_dense_chain(p.dtype, ops.data(), (int)ops.size(), Y);
  if (!resident.empty()) t_plan += " [resident: " + resident + "]";
  std::lock_guard<std::mutex> lock(p.bound->mu);
  p.bound->last_plan = t_plan;
}

void run_slot(int a, int s, const int64_t* v, int n) {
  std::shared_ptr<const Program> p;
  {
    std::lock_guard<std::mutex> lock(g_slot_mu);
    p = g_slot[a][s];
  }
  const int rc = guarded([&] {
    if (!p) fail(kErrUnknown, "function pointer slot %d is no longer bound (the module was cleared)", s);
    if (p->nargs != n) fail(kErrInternal, "function '%s' called with %d arguments, expected %d", p->name.c_str(), n, p->nargs);
    const size_t np = p->params.size();
    std::vector<Mat> mats(np + 1);
    std::vector<Vec> vecs(np);
    int pos = 0;
    auto ptr = [](int64_t x) { return reinterpret_cast<void*>((intptr_t)x); };
    for (size_t i = 0; i <= np; ++i) {
      const bool out = i == np;
      const TypeSpec& t = out ? p->ret : p->params[i].type;
      const int r = (int)t.shape.size();
      const int64_t* d = v + pos;  // allocated, aligned, offset, sizes[r], strides[r]
      pos += 3 + 2 * r;
      const char* nm = out ? "result" : p->params[i].name.c_str();
      for (int k = 0; k < r; ++k)
        if (d[3 + k] != t.shape[k])
          fail(kErrShape, "%s: descriptor size[%d] = %lld, the function was compiled for %lld", nm, k,
               (long long)d[3 + k], (long long)t.shape[k]);
      if (r == 2)
        mats[i] = mat_from_desc(ptr(d[1]), d[2], d[3], d[4], d[5], d[6], 4, nm);
      else if (r == 1)
        vecs[i] = vec_from_desc(ptr(d[1]), d[2], d[3], d[4], 4, nm);
    }
    run_program(*p, mats, vecs, mats[np]);
  });
  if (rc != 0)  // the memref calling convention has no error channel
    fprintf(stderr, "[edsl_hip] %s: %s\n", p ? p->name.c_str() : "?", t_err_msg.c_str());
}

template <int A, int S, typename Seq>
struct Tramp;
template <int A, int S, size_t... I>
struct Tramp<A, S, std::index_sequence<I...>> {
  static void fn(decltype((void)I, int64_t{})... a) {
    const int64_t v[] = {a...};
    run_slot(A, S, v, (int)sizeof...(I));
  }
};

template <int A, size_t... S>
std::array<void*, kSlots> arity_table(std::index_sequence<S...>) {
  return {reinterpret_cast<void*>(&Tramp<A, (int)S, std::make_index_sequence<kArities[A]>>::fn)...};
}

template <size_t... A>
std::array<std::array<void*, kSlots>, kNumArities> all_tables(std::index_sequence<A...>) {
  return {arity_table<(int)A>(std::make_index_sequence<kSlots>{})...};
}

void* trampoline(int a, int slot) {
  static const std::array<std::array<void*, kSlots>, kNumArities> tables =
      all_tables(std::make_index_sequence<kNumArities>{});
  return tables[a][slot];
}

// Binds p to a free slot of its arity; returns the slot, or -1 when the arity
// has no trampolines or all its slots are taken.
int acquire_slot(const std::shared_ptr<const Program>& p) {
  const int a = arity_index(p->nargs);
  if (a < 0) return -1;
  std::lock_guard<std::mutex> lock(g_slot_mu);
  for (int s = 0; s < kSlots; ++s)
    if (!g_slot[a][s]) {
      g_slot[a][s] = p;
      return s;
    }
  return -1;
}

void release_slot(const Program& p) {
  const int a = arity_index(p.nargs);
  if (a < 0 || p.slot < 0) return;
  std::lock_guard<std::mutex> lock(g_slot_mu);
  g_slot[a][p.slot].reset();
}

}  // namespace
}  // namespace rt
}  // namespace edsl

using namespace edsl::rt;

struct edsl_hip_module {
  std::mutex mu;
  std::map<std::string, std::shared_ptr<Program>> fns;  // sorted, like the reference's std::set
  std::string failure;                                 // last compile failure message
};

namespace {

void release_all(edsl_hip_module* m) {
  for (auto& kv : m->fns) release_slot(*kv.second);
  m->fns.clear();
}

std::shared_ptr<Program> lookup(edsl_hip_module* m, const char* name) {
  if (!m) fail(kErrArgument, "null module");
  if (!name) fail(kErrArgument, "null function name");
  auto it = m->fns.find(name);
  if (it == m->fns.end()) fail(kErrUnknown, "Function not compiled: %s", name);
  return it->second;
}

}  // namespace

extern "C" {

edsl_hip_module* edsl_hip_module_create(void) { return new (std::nothrow) edsl_hip_module(); }

void edsl_hip_module_destroy(edsl_hip_module* m) {
  if (!m) return;
  {
    std::lock_guard<std::mutex> lock(m->mu);
    release_all(m);
  }
  delete m;
}

int edsl_hip_module_compile_function(edsl_hip_module* m, const void* bytes, size_t len) {
  const int rc = guarded([&] {
    if (!m) fail(kErrArgument, "null module");
    auto p = std::make_shared<Program>(decode_function_def(bytes, len));
    std::lock_guard<std::mutex> lock(m->mu);
    if (m->fns.count(p->name)) fail(kErrArgument, "function '%s' is already compiled", p->name.c_str());
    p->slot = acquire_slot(p);
    m->fns[p->name] = p;
  });
  if (m) {
    std::lock_guard<std::mutex> lock(m->mu);
    m->failure = rc ? t_err_msg : std::string();
  }
  return rc;
}

int edsl_hip_module_has_function(edsl_hip_module* m, const char* name) {
  if (!m || !name) return 0;
  std::lock_guard<std::mutex> lock(m->mu);
  return m->fns.count(name) ? 1 : 0;
}

int edsl_hip_module_list_functions(edsl_hip_module* m, char* buf, size_t len) {
  std::string s;
  if (m) {
    std::lock_guard<std::mutex> lock(m->mu);
    for (auto& kv : m->fns) {
      if (!s.empty()) s += '\n';
      s += kv.first;
    }
  }
  return copy_out(s, buf, len);
}

void edsl_hip_module_clear(edsl_hip_module* m) {
  if (!m) return;
  std::lock_guard<std::mutex> lock(m->mu);
  release_all(m);
  m->failure.clear();
}

void* edsl_hip_module_get_function_pointer(edsl_hip_module* m, const char* name) {
  void* fp = nullptr;
  guarded([&] {
    std::shared_ptr<Program> p;
    if (!m) fail(kErrArgument, "null module");
    {
      std::lock_guard<std::mutex> lock(m->mu);
      p = lookup(m, name);
    }
    const int a = arity_index(p->nargs);
    if (a < 0)
      fail(kErrProgram,
           "function '%s' takes %d flat memref arguments; function pointers serve the dense forms with 1 to "
           "4 layers and every parameter used (use execute_gpu_function)",
           p->name.c_str(), p->nargs);
    if (p->slot < 0)
      fail(kErrLimit, "function '%s': all %d function-pointer slots of its form are in use; clear() the module",
           p->name.c_str(), kSlots);
    fp = trampoline(a, p->slot);
  });
  return fp;
}

int edsl_hip_module_describe(edsl_hip_module* m, char* buf, size_t len) {
  std::string s = "// libedsl_hip dense-path module (gfx950)\n";
  if (m) {
    std::lock_guard<std::mutex> lock(m->mu);
    for (auto& kv : m->fns) {
      const Program& p = *kv.second;
      s += "func @" + p.name + "(";
      for (size_t i = 0; i < p.params.size(); ++i) {
        if (i) s += ", ";
        s += "%" + p.params[i].name + ": " + type_str(p.params[i].type);
      }
      s += ") -> " + type_str(p.ret) + "\n";
      s += "  // form: " + p.form + " (" + (p.dtype == EDSL_DTYPE_F32 ? "f32" : "i32") + ", " +
           std::to_string(p.layers.size()) + (p.layers.size() == 1 ? " layer" : " layers") + ")\n";
      std::string h;
      for (size_t li = 0; li < p.layers.size(); ++li) {
        const Layer& L = p.layers[li];
        static const char* kAct[4] = {"", "relu", "leaky_relu", "tensor_map If(v > 0.0, v, 0.0)"};
        char line[256];
        snprintf(line, sizeof(line), "  // layer %zu: %s @ %s%s%s%s -> one fused launch (epilogue %d%s)\n", li,
                 L.x >= 0 ? p.params[L.x].name.c_str() : h.c_str(), p.params[L.w].name.c_str(),
                 L.b >= 0 ? " + " : "", L.b >= 0 ? p.params[L.b].name.c_str() : "",
                 (L.epi >> 1) ? (std::string(", then ") + kAct[L.epi >> 1]).c_str() : "", L.epi,
                 (L.epi >> 1) == 2 ? (", alpha " + std::to_string(L.alpha)).c_str() : "");
        s += line;
        h = "h" + std::to_string(li);
      }
      std::lock_guard<std::mutex> block(p.bound->mu);
      for (auto& b : p.bound->by_param)
        s += "  // resident: %" + p.params[b.first].name + " on device " + std::to_string(b.second.copy->device) +
             " (" + std::to_string(b.second.copy->bytes) + " bytes)\n";
      if (!p.bound->last_plan.empty()) s += "  // last run: " + p.bound->last_plan + "\n";
    }
  }
  return copy_out(s, buf, len);
}

int edsl_hip_module_param_index(edsl_hip_module* m, const char* name, const char* param, int* index) {
  return guarded([&] {
    std::shared_ptr<Program> p;
    {
      if (!m) fail(kErrArgument, "null module");
      std::lock_guard<std::mutex> lock(m->mu);
      p = lookup(m, name);
    }
    if (!param) fail(kErrArgument, "null parameter name");
    for (size_t i = 0; i < p->params.size(); ++i)
      if (p->params[i].name == param) {
        if (index) *index = (int)i;
        return;
      }
    fail(kErrArgument, "function '%s' has no parameter '%s'", p->name.c_str(), param);
  });
}

int edsl_hip_module_bind_parameter(edsl_hip_module* m, const char* name, int index, const void* data,
                                   const int64_t* shape, int rank) {
  return guarded([&] {
    std::shared_ptr<Program> p;
    {
      if (!m) fail(kErrArgument, "null module");
      std::lock_guard<std::mutex> lock(m->mu);
      p = lookup(m, name);
    }
    if (index < 0 || index >= (int)p->params.size())
      fail(kErrArgument, "function '%s' has %zu parameters, no parameter %d", p->name.c_str(), p->params.size(),
           index);
    const TypeSpec& t = p->params[index].type;
    const char* nm = p->params[index].name.c_str();
    if (t.kind != 3 || (t.shape.size() != 1 && t.shape.size() != 2))
      fail(kErrArgument, "%s: only 1-D and 2-D tensor parameters can be bound, got %s", nm, type_str(t).c_str());
    if (!shape && rank > 0) fail(kErrArgument, "null shape");
    if (rank != (int)t.shape.size())
      fail(kErrShape, "%s: rank %d, the function was compiled for rank %zu", nm, rank, t.shape.size());
    for (int k = 0; k < rank; ++k)
      if (shape[k] != t.shape[k])
        fail(kErrShape, "%s: shape[%d] = %lld, the function was compiled for %lld", nm, k, (long long)shape[k],
             (long long)t.shape[k]);
    const int64_t rows = rank == 2 ? shape[0] : 1, cols = shape[rank - 1];
    Binding b;
    b.host = data;
    b.rows = rows;
    b.cols = cols;
    b.copy = make_resident_copy(data, rows, cols, 4);
    std::lock_guard<std::mutex> lock(p->bound->mu);
    p->bound->by_param[index] = std::move(b);  // a replaced snapshot is freed once no call holds it
  });
}

int edsl_hip_module_unbind_parameter(edsl_hip_module* m, const char* name, int index) {
  return guarded([&] {
    std::shared_ptr<Program> p;
    {
      if (!m) fail(kErrArgument, "null module");
      std::lock_guard<std::mutex> lock(m->mu);
      p = lookup(m, name);
    }
    if (index < -1 || index >= (int)p->params.size())
      fail(kErrArgument, "function '%s' has %zu parameters, no parameter %d", p->name.c_str(), p->params.size(),
           index);
    std::lock_guard<std::mutex> lock(p->bound->mu);
    if (index < 0)
      p->bound->by_param.clear();
    else
      p->bound->by_param.erase(index);
  });
}

int edsl_hip_module_last_failure(edsl_hip_module* m, char* buf, size_t len) {
  std::string s;
  if (m) {
    std::lock_guard<std::mutex> lock(m->mu);
    s = m->failure;
  }
  return copy_out(s, buf, len);
}

int edsl_hip_module_function_form(edsl_hip_module* m, const char* name, int* dtype, int* num_layers, char* form,
                                  size_t form_len) {
  return guarded([&] {
    std::shared_ptr<Program> p;
    {
      if (!m) fail(kErrArgument, "null module");
      std::lock_guard<std::mutex> lock(m->mu);
      p = lookup(m, name);
    }
    if (dtype) *dtype = p->dtype;
    if (num_layers) *num_layers = (int)p->layers.size();
    copy_out(p->form, form, form_len);
  });
}

int edsl_hip_module_function_layer(edsl_hip_module* m, const char* name, int layer, int* x_param, int* w_param,
                                   int* b_param, int* epilogue, float* alpha) {
  return guarded([&] {
    std::shared_ptr<Program> p;
    {
      if (!m) fail(kErrArgument, "null module");
      std::lock_guard<std::mutex> lock(m->mu);
      p = lookup(m, name);
    }
    if (layer < 0 || layer >= (int)p->layers.size())
      fail(kErrArgument, "function '%s' has %zu layers, no layer %d", p->name.c_str(), p->layers.size(), layer);
    const Layer& L = p->layers[layer];
    if (x_param) *x_param = L.x;
    if (w_param) *w_param = L.w;
    if (b_param) *b_param = L.b;
    if (epilogue) *epilogue = L.epi;
    if (alpha) *alpha = L.alpha;
  });
}

int edsl_hip_module_execute_gpu_function(edsl_hip_module* m, const char* name, int num_inputs,
                                         const void* const* input_ptrs, const int64_t* const* input_shapes,
                                         const int* input_ranks, void* output, const int64_t* output_shape,
                                         int output_rank, size_t element_size) {
  return guarded([&] {
    std::shared_ptr<Program> p;
    {
      if (!m) fail(kErrArgument, "null module");
      std::lock_guard<std::mutex> lock(m->mu);
      p = lookup(m, name);
    }
    if (element_size != 4) fail(kErrDtype, "element_size %zu unsupported (f32 and i32 are 4 bytes)", element_size);
    if (num_inputs != (int)p->params.size())
      fail(kErrArgument, "function '%s' takes %zu inputs, got %d", p->name.c_str(), p->params.size(), num_inputs);
    if (!input_ptrs || !input_shapes || !input_ranks || !output_shape) fail(kErrArgument, "null argument array");
    std::vector<Mat> mats(num_inputs);
    std::vector<Vec> vecs(num_inputs);
    for (int i = 0; i < num_inputs; ++i) {
      const TypeSpec& t = p->params[i].type;
      const int r = input_ranks[i];
      const char* nm = p->params[i].name.c_str();
      if (r != (int)t.shape.size()) fail(kErrShape, "%s: rank %d, the function was compiled for rank %zu", nm, r, t.shape.size());
      for (int k = 0; k < r; ++k)
        if (input_shapes[i][k] != t.shape[k])
          fail(kErrShape, "%s: shape[%d] = %lld, the function was compiled for %lld", nm, k,
               (long long)input_shapes[i][k], (long long)t.shape[k]);
      void* ptr = const_cast<void*>(input_ptrs[i]);
      if (r == 2)
        mats[i] = mat_from_desc(ptr, 0, t.shape[0], t.shape[1], t.shape[1], 1, 4, nm);
      else if (r == 1)
        vecs[i] = vec_from_desc(ptr, 0, t.shape[0], 1, 4, nm);
    }
    if (output_rank != 2 || output_shape[0] != p->ret.shape[0] || output_shape[1] != p->ret.shape[1])
      fail(kErrShape, "output shape does not match %s", type_str(p->ret).c_str());
    const Mat Y = mat_from_desc(output, 0, p->ret.shape[0], p->ret.shape[1], p->ret.shape[1], 1, 4, "output");
    run_program(*p, mats, vecs, Y);
  });
}

}  // extern "C"
