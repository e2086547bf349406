// Internal interface between the C-ABI runtime (runtime.cpp) and the
// FunctionDef front end (program.cpp). Not installed; not part of the ABI.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <exception>
#include <memory>
#include <string>

namespace edsl {
namespace rt {

// Error codes returned by the C ABI (edsl_hip_last_error). HIP errors are
// reported with their positive hipError_t value.
enum ErrorCode : int {
  kErrShape = -1,     // sizes inconsistent with the op
  kErrStride = -2,    // unsupported stride / layout
  kErrDtype = -3,     // element type / size
  kErrArgument = -4,  // null pointer, bad pattern, bad epilogue
  kErrLimit = -5,     // size beyond what the kernels index
  kErrInternal = -6,
  kErrProgram = -7,   // FunctionDef that is malformed or not a dense-path program
  kErrUnknown = -8,   // function name not compiled in the module
};

struct Failure {
  int code;
  std::string msg;
};

extern thread_local int t_err_code;
extern thread_local std::string t_err_msg;
extern thread_local std::string t_plan;  // edsl_hip_last_plan() of the calling thread

[[noreturn]] void fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Runs f, turning a thrown Failure (or any exception) into the thread's last
// error; returns 0 or the error code.
template <typename F>
int guarded(F&& f) {
  t_err_code = 0;
  t_err_msg.clear();
  try {
    f();
    return 0;
  } catch (const Failure& e) {
    t_err_code = e.code;
    t_err_msg = e.msg;
  } catch (const std::exception& e) {
    t_err_code = kErrInternal;
    t_err_msg = e.what();
  } catch (...) {
    t_err_code = kErrInternal;
    t_err_msg = "unknown error";
  }
  return t_err_code;
}

int copy_out(const std::string& s, char* buf, size_t len);

// A 2-D operand: element (r, c) at base + (r*ld + c) * element size.
struct Mat {
  char* base = nullptr;  // aligned + offset
  int64_t rows = 0, cols = 0, ld = 0;
};

struct Vec {
  char* base = nullptr;
  int64_t n = 0;
};

Mat mat_from_desc(void* aligned, int64_t offset, int64_t d0, int64_t d1, int64_t s0, int64_t s1,
                  size_t esize, const char* name);
Vec vec_from_desc(void* aligned, int64_t offset, int64_t d0, int64_t s0, size_t esize, const char* name);

// Y = epilogue(X @ W (+ b)) on the current device, host or device operands,
// synchronous on return. dtype is EDSL_DTYPE_*, epi an EDSL_EPI_* code.
void sync_dense(int dtype, int epi, float alpha, const Mat& X, const Mat& W, const Vec* b, const Mat& Y);

// One layer of a chain: H_i = epilogue(H_{i-1} @ W (+ b)). Only the first
// layer has an input X; later layers read the previous layer's output.
struct LayerOp {
  const Mat* X;  // first layer only, else nullptr
  const Mat* W;
  const Vec* b;  // when epi adds a bias
  int epi;
  float alpha;
};

// Runs the layers in order with the intermediates in device memory (host
// operands staged, only the last layer's output copied back), synchronous on
// return.
void sync_dense_chain(int dtype, const LayerOp* layers, int n, const Mat& Y);

// A snapshot of a 2-D (or 1-D: rows == 1) operand held in device memory on
// the device that was current when it was made, with rows padded to a
// multiple of 4 elements and 16-byte alignment, so every kernel can read it in
// place. The memory is freed when the last reference goes away.
struct ResidentCopy {
  int device = -1;
  void* dev = nullptr;
  int64_t rows = 0, cols = 0, dev_ld = 0;
  size_t bytes = 0;
  ResidentCopy() = default;
  ResidentCopy(const ResidentCopy&) = delete;
  ResidentCopy& operator=(const ResidentCopy&) = delete;
  ~ResidentCopy();
};

// Copies rows x cols contiguous elements of esize bytes (host or device
// memory) into a new ResidentCopy on the current device; returns once the
// copy has landed. Throws Failure.
std::shared_ptr<ResidentCopy> make_resident_copy(const void* src, int64_t rows, int64_t cols, size_t esize);

// The current HIP device. Throws Failure.
int current_device();

// Device memory for the small-M kernel's split-K partials that the caller
// fixes, in place of the library's grow-only per-device
// workspaces: nothing is allocated, and no cross-stream ordering is added.
struct FixedScratch {
  char* base;    // device address, 256-byte aligned
  size_t bytes;  // capacity; a plan that needs more is rejected (kErrLimit)
};

// Body of edsl_hip_dense_f32_launch (argument checks, plan, launch); with
// `fixed` non-null every scratch buffer comes from it. `plan_bias`, when not
// null, is a bias the epilogue does not add whose alignment the kernel
// choice still honours (see DenseLaunch::plan_bias). Throws Failure.
void dense_f32_launch(const float* X, int64_t ldx, const float* W, int64_t ldw, const float* bias, float* Y,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue, float alpha, void* stream,
                      const FixedScratch* fixed, const float* plan_bias = nullptr);

}  // namespace rt
}  // namespace edsl
