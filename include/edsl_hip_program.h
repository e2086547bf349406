/*
 * edsl_hip_program.h -- compile the reference front end's serialized
 * FunctionDef and run it on the gfx950 dense-path kernels.
 *
 * These entry points are what the reference's pybind module `_mlir_backend`
 * (reference cpp/src/python_bindings.cpp:8-98) binds on its MLIRCompiler
 * (reference cpp/include/mlir_edsl/MLIRCompiler.h, cpp/src/MLIRCompiler.cpp),
 * restated as a C ABI over an opaque module handle, for the dense-path
 * programs only:
 *
 *   matmul(A, B) / A @ B, relu(A @ B), X @ W + b, relu(X @ W + b),
 *   leaky_relu(X @ W + b, alpha), tensor_map(X @ W [+ b],
 *   lambda v: If(v > 0, v, 0)) over i32, and chains of such layers whose
 *   input is the previous layer (h = relu(X @ W1 + b1); relu(h @ W2 + b2)),
 *   run with the intermediates in device memory -- X, W, b being parameters
 *   with static tensor types.
 *
 * Any other program is rejected at compile time with an error that names
 * what was found. Errors: functions returning int return 0 on success or an
 * error code (the message is in edsl_hip_last_error(), include/edsl_hip.h),
 * as the reference raises std::runtime_error from the same calls.
 */
#ifndef EDSL_HIP_PROGRAM_H
#define EDSL_HIP_PROGRAM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A set of compiled functions (the reference's MLIRCompiler instance). */
typedef struct edsl_hip_module edsl_hip_module;

/* MLIRCompiler() / ~MLIRCompiler(). create returns NULL on allocation failure. */
edsl_hip_module *edsl_hip_module_create(void);
void edsl_hip_module_destroy(edsl_hip_module *m);

/* MLIRCompiler::compileFunction (reference cpp/src/MLIRCompiler.cpp:184-216),
 * bound as compile_function(bytes) (cpp/src/python_bindings.cpp:13-23):
 * `bytes` is a serialized mlir_edsl.FunctionDef (cpp/schemas/ast.proto:473-478).
 * Dynamic (-1) dimensions are rejected like the reference's convertTensorType
 * (cpp/src/MLIRBuilder.cpp:478-486). Compiling a name twice is an error. */
int edsl_hip_module_compile_function(edsl_hip_module *m, const void *bytes, size_t len);

/* MLIRCompiler::hasFunction / listFunctions (cpp/src/MLIRCompiler.cpp:314-320).
 * list writes the names in sorted order, '\n'-separated, NUL-terminated
 * (truncated to len) and returns the full length. */
int edsl_hip_module_has_function(edsl_hip_module *m, const char *name);
int edsl_hip_module_list_functions(edsl_hip_module *m, char *buf, size_t len);

/* MLIRCompiler::clear: forget every function. Function pointers handed out
 * before stop being bound (calling one records an error). */
void edsl_hip_module_clear(edsl_hip_module *m);

/* MLIRCompiler::getFunctionPointer (cpp/src/MLIRCompiler.cpp:277-280): an
 * entry point with the calling convention of the reference's JIT'd symbol
 * for this function -- each parameter's expanded memref descriptor in the
 * FunctionDef's parameter order, then the out-param descriptor, void return
 * (reference mlir_edsl/backend.py:162-198). NULL (with an error recorded) for
 * an unknown name ("Function not compiled: <name>", as
 * cpp/src/MLIRExecutor.cpp:109-115). The pointer records errors for
 * edsl_hip_last_error() and prints them to stderr, the JIT'd symbol having no
 * error channel. Pointers exist for the 14-, 19-, 21- and 26-argument forms
 * (every dense program whose parameters are all used); at most 256 functions
 * hold one at a time per process. */
void *edsl_hip_module_get_function_pointer(edsl_hip_module *m, const char *name);

/* MLIRCompiler::executeGPUFunction (cpp/src/MLIRCompiler.cpp:352-461), bound
 * as execute_gpu_function(name, inputs, output_shape, element_size)
 * (cpp/src/python_bindings.cpp:69-97): contiguous row-major inputs given as
 * (pointer, shape) pairs in parameter order, one contiguous output; host or
 * device memory; synchronous on return. */
int edsl_hip_module_execute_gpu_function(edsl_hip_module *m, const char *name, int num_inputs,
                                         const void *const *input_ptrs,
                                         const int64_t *const *input_shapes, const int *input_ranks,
                                         void *output, const int64_t *output_shape, int output_rank,
                                         size_t element_size);

/* Device-resident parameters. Replaces, for the operands a caller marks as
 * constant across calls (weights, biases), the per-call device allocation and
 * host-to-device copy of every operand in the reference's GPU path
 * (cpp/src/MLIRCompiler.cpp:367-376 allocates and copies each input,
 * :451-454 frees them), which the reference's JIT path has no way to avoid.
 *
 * bind_parameter copies `data` (contiguous row-major, host or device memory,
 * `shape`/`rank` equal to the parameter's compiled type) into device memory
 * on the current device and returns once the copy has landed. From then on a
 * call of the function -- through its function pointer or
 * execute_gpu_function -- that passes that same address (aligned + offset)
 * with the same shape and contiguous rows, with that device current, reads
 * the device copy in place: the operand is not copied in. The copy is a
 * SNAPSHOT of the array at bind time: later writes to the array are not seen
 * until it is bound again. Any other address runs as before (copied in).
 * Binding again replaces the snapshot; unbind (index -1: every parameter of
 * the function), clear() and destroy release it. index is the parameter's
 * position in the FunctionDef (param_index maps a name to it).
 * The caller must keep the memory at `data` allocated (and not reuse it for
 * other values) for as long as the parameter stays bound: calls are matched
 * by address, so memory freed and handed to a new array of the same shape
 * would be read from the stale snapshot. The Python facade holds the bound
 * object until unbind, rebind or clear for this reason. */
int edsl_hip_module_bind_parameter(edsl_hip_module *m, const char *name, int index, const void *data,
                                   const int64_t *shape, int rank);
int edsl_hip_module_unbind_parameter(edsl_hip_module *m, const char *name, int index);
int edsl_hip_module_param_index(edsl_hip_module *m, const char *name, const char *param, int *index);

/* MLIRCompiler::getModuleIR counterpart: a text listing of the compiled
 * functions -- signature, the dense form each was matched to, its layers and
 * epilogues, resident parameters, and the kernels of its last run. */
int edsl_hip_module_describe(edsl_hip_module *m, char *buf, size_t len);

/* MLIRCompiler::getFailureIR counterpart: the message of the last failed
 * compile_function on this module, empty after a success or clear(). */
int edsl_hip_module_last_failure(edsl_hip_module *m, char *buf, size_t len);

/* How a compiled function was matched (no reference counterpart: for tests
 * and tools). function_form gives the element type (EDSL_DTYPE_*), the number
 * of dense layers and the whole program as text ("relu(relu(X @ W1 + b1) @ W2
 * + b2)"); function_layer gives layer i (execution order): the parameter
 * indices of its input (-1: the previous layer's output), weight and bias
 * (-1: none), its EDSL_EPI_* epilogue and leaky alpha. Output pointers may be
 * NULL. */
int edsl_hip_module_function_form(edsl_hip_module *m, const char *name, int *dtype, int *num_layers,
                                  char *form, size_t form_len);
int edsl_hip_module_function_layer(edsl_hip_module *m, const char *name, int layer, int *x_param,
                                   int *w_param, int *b_param, int *epilogue, float *alpha);

#ifdef __cplusplus
}
#endif

#endif /* EDSL_HIP_PROGRAM_H */
