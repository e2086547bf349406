// Host-only stand-ins for the runtime functions program.cpp calls, so the
// FunctionDef decoder can be built with g++ and the address / undefined-
// behaviour sanitizers (no HIP, no device). Test infrastructure only.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../ml-edsl_amd/csrc/runtime_internal.hpp"

namespace edsl {
namespace rt {

thread_local int t_err_code = 0;
thread_local std::string t_err_msg;
thread_local std::string t_plan;

int current_device() { return 0; }

// Host memory stands in for the device copy (the decoder only passes it on).
ResidentCopy::~ResidentCopy() { delete[] static_cast<char*>(dev); }

std::shared_ptr<ResidentCopy> make_resident_copy(const void* src, int64_t rows, int64_t cols, size_t esize) {
  if (rows < 0 || cols < 0) fail(kErrShape, "negative size");
  auto c = std::make_shared<ResidentCopy>();
  c->device = 0;
  c->rows = rows;
  c->cols = cols;
  c->dev_ld = (cols + 3) & ~int64_t(3);
  c->bytes = (size_t)rows * (size_t)c->dev_ld * esize + 256;
  c->dev = new char[c->bytes]();
  for (int64_t r = 0; r < rows; ++r)
    memcpy(static_cast<char*>(c->dev) + r * c->dev_ld * esize, static_cast<const char*>(src) + r * cols * esize,
           (size_t)cols * esize);
  return c;
}

void fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  throw Failure{code, buf};
}

int copy_out(const std::string& s, char* buf, size_t len) {
  if (buf && len > 0) {
    const size_t n = std::min(len - 1, s.size());
    memcpy(buf, s.data(), n);
    buf[n] = '\0';
  }
  return (int)s.size();
}

Mat mat_from_desc(void* aligned, int64_t offset, int64_t d0, int64_t d1, int64_t s0, int64_t, size_t esize,
                  const char*) {
  Mat m;
  m.base = static_cast<char*>(aligned) + offset * (int64_t)esize;
  m.rows = d0;
  m.cols = d1;
  m.ld = s0;
  return m;
}

Vec vec_from_desc(void* aligned, int64_t offset, int64_t d0, int64_t, size_t esize, const char*) {
  Vec v;
  v.base = static_cast<char*>(aligned) + offset * (int64_t)esize;
  v.n = d0;
  return v;
}

// Checks the operands the decoder bound, touches nothing.
void sync_dense_chain(int, const LayerOp* layers, int n, const Mat& Y) {
  if (n < 1 || !layers[0].X || !Y.base) fail(kErrArgument, "bad chain");
  for (int i = 0; i < n; ++i)
    if (!layers[i].W || (i > 0 && layers[i].X)) fail(kErrArgument, "bad layer %d", i);
}

void sync_dense(int dtype, int epi, float alpha, const Mat& X, const Mat& W, const Vec* b, const Mat& Y) {
  const LayerOp op{&X, &W, b, epi, alpha};
  sync_dense_chain(dtype, &op, 1, Y);
}

}  // namespace rt
}  // namespace edsl
