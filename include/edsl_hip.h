/*
 * edsl_hip.h -- C ABI of the MI355X (gfx950) dense-path runtime.
 *
 * Drop-in boundary for ml-edsl's dense hot path: linalg.matmul and the dense
 * layer Y = ReLU(X.W + b) (plus the bias-only and leaky-ReLU epilogues), in
 * f32 and in i32.
 *
 * Calling convention: each function has exactly the signature of the function
 * the reference JIT produces for the same DSL program. MLIR's func-to-llvm
 * lowering expands every memref argument into the scalar run
 *     (T* allocated, T* aligned, int64 offset, int64 size[r], int64 stride[r])
 * and the tensor result becomes a trailing out-param memref with a void
 * return (reference mlir_edsl/backend.py:37-102 packs exactly these
 * descriptors; cpp/src/MLIRLowering.cpp:327-328 adds the out-param). A caller
 * that today does
 *     ctypes.CFUNCTYPE(None, *flat_types)(compiler.get_function_pointer(name))(*flat_args)
 * (reference mlir_edsl/backend.py:182-191) can call these symbols with the
 * same flat argument list.
 *
 * Semantics shared by every entry point below:
 *  - The element address is aligned + offset; strides are in elements. The
 *    innermost stride must be 1 (the reference passes C-contiguous arrays,
 *    mlir_edsl/backend.py:88-91); the row stride may be larger than the row.
 *  - Pointers may be host memory (copied in and out, like the reference GPU
 *    path, cpp/src/MLIRCompiler.cpp:367-454) or device memory (used in place).
 *  - Synchronous: on return the whole output has been written and is visible
 *    to the host (the reference synchronises after every launch,
 *    cpp/src/MLIRExecutor.cpp:211-214). Device-pointer work is ordered on the
 *    HIP null stream.
 *  - The output is written in full and never read; inputs are never written.
 *  - Errors: the reference's JIT'd function has no error channel, so these
 *    keep the void return and record the failure for edsl_hip_last_error()
 *    (thread-local), which the host facade turns into RuntimeError just as
 *    the reference turns std::runtime_error into RuntimeError
 *    (cpp/src/python_bindings.cpp:17-19, cpp/src/MLIRExecutor.cpp:160-167).
 *  - f32 arithmetic: fp32 products accumulated in fp32; results agree with
 *    the reference CPU JIT within relative Frobenius error 1e-5 and
 *    max|delta| <= 1e-4*sqrt(K). Bias is arith.addf; ReLU is arith.maximumf
 *    (NaN propagates, -0 -> +0); leaky is maximumf(x,0) + alpha*minimumf(x,0).
 *  - i32 arithmetic: arith.muli / arith.addi (two's complement, wrapping);
 *    results are bit-identical to the reference for every input. ReLU on i32
 *    is v > 0 ? v : 0, the reference's tensor_map(If(v > 0, v, 0)).
 *  - The f32 ReLU written tensor_map(v -> If(v > 0.0, v, 0.0)) is cmpf ogt
 *    then a select of v or +0.0: NaN and -0 give +0 (unlike maximumf).
 */
#ifndef EDSL_HIP_H
#define EDSL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EDSL_MEMREF2(T, p)                                                         \
  T *p##_allocated, T *p##_aligned, int64_t p##_offset, int64_t p##_size0,          \
      int64_t p##_size1, int64_t p##_stride0, int64_t p##_stride1
#define EDSL_MEMREF1(T, p) \
  T *p##_allocated, T *p##_aligned, int64_t p##_offset, int64_t p##_size0, int64_t p##_stride0

/* C = A x B.  f(A: Tensor[f32, M, K], B: Tensor[f32, K, N]) -> Tensor[f32, M, N]
 * with body `matmul(A, B)` or `A @ B`. 21 arguments. Replaces the GPU
 * execution of fill + linalg.matmul (reference cpp/src/builders/LinalgBuilder.cpp:106-139,
 * launched by cpp/src/MLIRCompiler.cpp:352-461) and is call-compatible with the
 * CPU JIT symbol bound at mlir_edsl/backend.py:182-191. */
void edsl_hip_matmul_f32(EDSL_MEMREF2(float, A), EDSL_MEMREF2(float, B), EDSL_MEMREF2(float, C));

/* i32 version of edsl_hip_matmul_f32 (reference tests/linalg/test_matmul_execution.py:93-103). */
void edsl_hip_matmul_i32(EDSL_MEMREF2(int32_t, A), EDSL_MEMREF2(int32_t, B),
                         EDSL_MEMREF2(int32_t, C));

/* Y = X @ W + b.  f(X: [M,K], W: [K,N], b: [N]) -> [M,N]. 26 arguments.
 * Replaces fill + matmul + the `bias_add` generic (reference
 * cpp/src/builders/LinalgBuilder.cpp:301-339; tests/gpu/test_gpu_execution.py:195-210). */
void edsl_hip_matmul_bias_f32(EDSL_MEMREF2(float, X), EDSL_MEMREF2(float, W),
                              EDSL_MEMREF1(float, b), EDSL_MEMREF2(float, Y));
void edsl_hip_matmul_bias_i32(EDSL_MEMREF2(int32_t, X), EDSL_MEMREF2(int32_t, W),
                              EDSL_MEMREF1(int32_t, b), EDSL_MEMREF2(int32_t, Y));

/* Y = relu(X @ W + b), one fused kernel.  26 arguments. Replaces the
 * reference's fill, matmul and merged bias+ReLU generic kernels (reference
 * cpp/src/builders/LinalgBuilder.cpp:180-239; three launches per call,
 * tests/gpu/test_gpu_execution.py:149-154). The i32 form is the integer dense
 * layer written tensor_map(X @ W + b, lambda v: If(v > 0, v, 0)). */
void edsl_hip_dense_relu_f32(EDSL_MEMREF2(float, X), EDSL_MEMREF2(float, W),
                             EDSL_MEMREF1(float, b), EDSL_MEMREF2(float, Y));
void edsl_hip_dense_relu_i32(EDSL_MEMREF2(int32_t, X), EDSL_MEMREF2(int32_t, W),
                             EDSL_MEMREF1(int32_t, b), EDSL_MEMREF2(int32_t, Y));

/* Y = leaky_relu(X @ W + b, alpha).  The reference bakes alpha into the IR
 * as a constant (cpp/src/builders/LinalgBuilder.cpp:216-225), so its JIT
 * symbol has only the 26 memref arguments; here alpha is a trailing argument
 * that the host facade binds per compiled function. */
void edsl_hip_dense_leaky_relu_f32(EDSL_MEMREF2(float, X), EDSL_MEMREF2(float, W),
                                   EDSL_MEMREF1(float, b), EDSL_MEMREF2(float, Y), float alpha);

/* Y = relu(A @ B): the activation applied straight to the matmul, no bias
 * (reference fill + matmul + `relu` generic, LinalgBuilder.cpp:106-139, 180-239). */
void edsl_hip_matmul_relu_f32(EDSL_MEMREF2(float, A), EDSL_MEMREF2(float, B), EDSL_MEMREF2(float, C));
void edsl_hip_matmul_relu_i32(EDSL_MEMREF2(int32_t, A), EDSL_MEMREF2(int32_t, B),
                              EDSL_MEMREF2(int32_t, C));

/* Y = tensor_map(X @ W + b, lambda v: If(v > 0.0, v, 0.0)) over f32, one
 * fused kernel. 26 arguments. Replaces fill + matmul + the bias generic + the
 * linalg.map whose body is the If (reference cpp/src/builders/LinalgBuilder.cpp:141-178;
 * the map form of tests/linalg/test_map_execution.py:40-52). */
void edsl_hip_dense_if_relu_f32(EDSL_MEMREF2(float, X), EDSL_MEMREF2(float, W),
                                EDSL_MEMREF1(float, b), EDSL_MEMREF2(float, Y));
/* Y = tensor_map(A @ B, lambda v: If(v > 0.0, v, 0.0)) over f32. 21 arguments. */
void edsl_hip_matmul_if_relu_f32(EDSL_MEMREF2(float, A), EDSL_MEMREF2(float, B), EDSL_MEMREF2(float, C));

/* Host-buffer entry in the shape of MLIRCompiler::executeGPUFunction
 * (reference cpp/src/MLIRCompiler.cpp:352-461, bound to Python as
 * execute_gpu_function at cpp/src/python_bindings.cpp:69-97): contiguous
 * row-major host inputs given as (pointer, shape) pairs, one contiguous host
 * output. `pattern` is an EDSL_PATTERN_* code (the function name -> pattern
 * binding is made by the host facade when the function is compiled).
 * Inputs: {A, B} for the matmul patterns, {X, W, b} otherwise.
 * element_size must be 4. Returns 0 on success, else an error code with the
 * message available from edsl_hip_last_error(). */
#define EDSL_PATTERN_MATMUL 0      /* matmul(A, B)                  */
#define EDSL_PATTERN_MATMUL_BIAS 1 /* X @ W + b                     */
#define EDSL_PATTERN_DENSE_RELU 2  /* relu(X @ W + b)               */
#define EDSL_PATTERN_DENSE_LEAKY 3 /* leaky_relu(X @ W + b, alpha)  */
#define EDSL_PATTERN_MATMUL_RELU 4 /* relu(A @ B)                   */
#define EDSL_PATTERN_DENSE_IF_RELU 5  /* tensor_map(X @ W + b, v -> If(v > 0, v, 0)) */
#define EDSL_PATTERN_MATMUL_IF_RELU 6 /* tensor_map(A @ B, v -> If(v > 0, v, 0))     */
#define EDSL_DTYPE_F32 0
#define EDSL_DTYPE_I32 1
int edsl_hip_execute_gpu_function(int pattern, int dtype, int num_inputs,
                                  const void *const *input_ptrs,
                                  const int64_t *const *input_shapes, const int *input_ranks,
                                  void *output, const int64_t *output_shape, int output_rank,
                                  size_t element_size, float alpha);

/* Last error recorded on the calling thread: returns its code (0 = none) and
 * copies the NUL-terminated message into buf (truncated to len). The
 * reference's counterpart is the std::runtime_error text surfaced as Python
 * RuntimeError (cpp/src/MLIRExecutor.cpp:160-167). */
int edsl_hip_last_error(char *buf, size_t len);
void edsl_hip_clear_error(void);

#undef EDSL_MEMREF1
#undef EDSL_MEMREF2

#ifdef __cplusplus
}
#endif

#endif /* EDSL_HIP_H */
