// edsl_hip_dense_f32_launch_noalloc: the f32 device launch with its scratch in
// a fixed, statically sized device array instead of library allocations.
//
// The small-M (weight-streaming) plan needs scratch beyond the caller's
// operands: the split-K partial tiles that the reduce kernel sums. The
// ordinary entry point takes them from a grow-only per-device buffer that it
// allocates with hipMalloc on first use. This entry point takes them from
// `scratch` below, so it never allocates: callers that cannot call hipMalloc
// (code under HIP graph capture, serving loops, harnesses that forbid it) can
// use it.
//
// `scratch` is a file-scope __device__ array: every GPU the library runs on
// holds its own copy, for the life of the process. In host code its name is
// only a stand-in for the symbol, never a device address, so the address is
// looked up once per device with hipGetSymbolAddress (with that device
// current) and kept; kernels and copies only ever see that address.
//
// All calls on one GPU share that GPU's array and it keeps the last call's
// contents. Nothing in it needs to start at zero: every partial a reduce reads
// was written by the same call.
// Calls that overlap on one GPU (two streams, two threads) race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/edsl_hip_device.h"
#include "runtime_internal.hpp"

namespace {

constexpr size_t kStaticScratchBytes = EDSL_NOALLOC_SCRATCH_BYTES;
static_assert(kStaticScratchBytes % 256 == 0, "scratch size keeps 256-byte alignment");

static __device__ __align__(256) char scratch[kStaticScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_addr[kMaxScratchDevices] = {};

// Device address of the current device's copy of `scratch`, looked up on the
// first call made with that device current.
char* scratch_address() {
  using edsl::rt::fail;
  int dev = -1;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess) fail((int)ge, "hipGetDevice failed: %s", hipGetErrorString(ge));
  if (dev < 0 || dev >= kMaxScratchDevices)
    fail(edsl::rt::kErrLimit, "device index %d out of range for the static scratch", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      fail(e != hipSuccess ? (int)e : edsl::rt::kErrInternal, "hipGetSymbolAddress(scratch) failed on device %d: %s",
           dev, hipGetErrorString(e));
    g_scratch_addr[dev] = static_cast<char*>(p);
  }
  return g_scratch_addr[dev];
}

}  // namespace

extern "C" int edsl_hip_dense_f32_launch_noalloc(const float* X, int64_t ldx, const float* W, int64_t ldw,
                                                 const float* bias, float* Y, int64_t ldy, int64_t M, int64_t N,
                                                 int64_t K, int epilogue, float alpha, void* stream) {
  return edsl::rt::guarded([&] {
    const edsl::rt::FixedScratch fixed{scratch_address(), kStaticScratchBytes};
    edsl::rt::dense_f32_launch(X, ldx, W, ldw, bias, Y, ldy, M, N, K, epilogue, alpha, stream, &fixed);
  });
}
