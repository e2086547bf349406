// HIP runtime module for ml-edsl's dense hot path: the C ABI of
// include/edsl_hip.h and include/edsl_hip_device.h.
//
// It replaces the reference's NVVM/CUDA execution path -- MLIRGPUExecutor
// (reference cpp/src/MLIRExecutor.cpp:158-247) and
// MLIRCompiler::executeGPUFunction (cpp/src/MLIRCompiler.cpp:352-461), which
// allocate, copy in, launch fill / matmul / bias+ReLU as three synchronous
// kernels, copy out and free on every call -- with:
//  * descriptor validation of MLIR's expanded memref arguments,
//  * host or device operands (host operands staged through grow-only device
//    buffers that persist across calls instead of per-call alloc/free),
//  * one fused kernel per dense layer (two for the int8 path: narrow + GEMM),
//  * kernel selection by shape: small-M weight streaming or tiled MFMA, each
//    with variants for operands of any alignment, row stride and size.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/edsl_hip.h"
#include "../../include/edsl_hip_device.h"
#include "common.hpp"
#include "kernels.hpp"
#include "host_stage.hpp"
#include "runtime_internal.hpp"

namespace edsl {
namespace rt {

// ------------------------------------------------------------------ errors
thread_local int t_err_code = 0;
thread_local std::string t_err_msg;
thread_local std::string t_plan;

[[noreturn]] void fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  throw Failure{code, buf};
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) fail((int)e, "%s failed: %s", what, hipGetErrorString(e));
}

void set_plan(const char* fmt, ...) {
  char buf[256];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  t_plan = buf;
}

int copy_out(const std::string& s, char* buf, size_t len) {
  if (buf && len > 0) {
    const size_t n = std::min(len - 1, s.size());
    memcpy(buf, s.data(), n);
    buf[n] = '\0';
  }
  return (int)s.size();
}

// ------------------------------------------------------------ device state
struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
  // Workspaces of the device entry points may be baked into HIP graphs that
  // callers capture, so an outgrown one is kept (retired) rather than freed:
  // a replay still finds the buffer it was captured with. Growth is then at
  // least twofold, which bounds the retired total by the final capacity.
  bool keep_old = false;
  std::vector<void*> retired;

  DevBuf() = default;
  explicit DevBuf(bool keep) : keep_old(keep) {}

  // Grow-only. A buffer that is released may still be in use by queued work,
  // so the device is drained first.
  void* ensure(size_t bytes, bool zero_fill) {
    if (bytes <= cap && p) return p;
    size_t grow = 0;
    if (p && keep_old) {
      retired.push_back(p);
      grow = 2 * cap;
      p = nullptr;
      cap = 0;
    } else if (p) {
      check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
      check_hip(hipFree(p), "hipFree");
      p = nullptr;
      cap = 0;
    }
    const size_t want = std::max<size_t>({(bytes + 255) & ~size_t(255), size_t(256), grow});
    check_hip(hipMalloc(&p, want), "hipMalloc");
    if (zero_fill) {
      // Finished before any stream (blocking or not) can use the buffer.
      check_hip(hipMemset(p, 0, want), "hipMemset");
      check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
    }
    cap = want;
    return p;
  }
};

constexpr int kPipeBlocks = 4;  // row blocks of a pipelined host-buffer layer

struct DeviceState {
  bool ready = false;
  int cus = 256;
  DevBuf stage[4];  // host-operand staging: X/A, W/B, bias, Y/C
  DevBuf chain[2];  // intermediate activations of multi-layer programs (ping-pong)
  DevBuf gemv_partials{true};
  DevBuf i8_x{true}, i8_w{true}, i8_flags{true};
  // Ordering of the launches that use the library scratch above (split-K
  // partials, packed int8 operands and flag) across streams.
  hipStream_t ws_stream = nullptr;  // stream of the last such launch
  bool ws_seen = false;             // any such launch yet
  bool ws_multi = false;            // a second stream has used the scratch: ws_ev orders every use
  hipEvent_t ws_ev = nullptr;
  // Pipelined host-buffer layers: uploads, kernels and downloads on three
  // non-blocking streams (default priority), ordered by events.
  bool pipe_ready = false;
  hipStream_t pipe_up = nullptr, pipe_run = nullptr, pipe_down = nullptr;
  hipEvent_t ev_w = nullptr, ev_x[kPipeBlocks] = {}, ev_g[kPipeBlocks] = {};
};

constexpr int kMaxDevices = 64;
// Two locks, always taken in this order when both are held:
//  g_host_mu: the host-buffer path -- staging buffers, ping-pong buffers,
//    the pipeline's streams, the pinned ring and its copy threads -- held
//    for a whole synchronous host-buffer call;
//  g_mu: device state, tuning overrides and the launch workspaces (split-K
//    partials, packed int8 operands, their cross-stream ordering), held only
//    while a launch is planned and enqueued.
// A device launch from one thread therefore never waits for another thread's
// host-to-device or device-to-host copies.
std::mutex g_host_mu;
std::mutex g_mu;
DeviceState g_dev[kMaxDevices];
int g_force_cfg = -1;
int g_force_ksplit = 0;
int g_force_cols = 0;
int g_force_small_m = 0;  // 1: the small-M kernel whenever it can plan the layer
int g_force_i8 = -1;
bool g_no_pipeline = false;  // EDSL_HIP_HOST_PIPELINE=0: plain staged sequence for host buffers

void read_env_overrides() {
  static bool done = false;
  if (done) return;
  done = true;
  if (const char* s = getenv("EDSL_HIP_F32_CONFIG")) g_force_cfg = atoi(s);
  if (const char* s = getenv("EDSL_HIP_GEMV_KSPLIT")) g_force_ksplit = atoi(s);
  if (const char* s = getenv("EDSL_HIP_GEMV_COLS")) g_force_cols = atoi(s);
  if (const char* s = getenv("EDSL_HIP_SMALL_M")) g_force_small_m = atoi(s);
  if (const char* s = getenv("EDSL_HIP_I8_VARIANT")) g_force_i8 = atoi(s);
  if (const char* s = getenv("EDSL_HIP_HOST_PIPELINE")) g_no_pipeline = atoi(s) == 0;
}

DeviceState& device_state(int* dev_out) {
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) fail(kErrLimit, "device index %d out of range", dev);
  DeviceState& s = g_dev[dev];
  if (!s.ready) {
    hipDeviceProp_t prop;
    check_hip(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
    s.cus = std::max(1, prop.multiProcessorCount);
    s.ready = true;
  }
  if (dev_out) *dev_out = dev;
  return s;
}

// ------------------------------------------------ scratch stream ordering
// Launches on one stream run in order, so while a single stream uses the
// library scratch nothing is added. The first launch from a second stream
// waits for the whole device once (the earlier stream may since have been
// destroyed, so no event can be recorded on it after the fact); from then on
// every scratch launch records ws_ev after its kernels, and a launch from a
// stream other than the last one waits for that event first. Overlapping
// calls on different streams are thereby serialised on the device.
// While `stream` is being captured into a graph nothing is added: a captured
// launch cannot wait for work outside the capture, and replays are ordered
// by the stream the graph is launched on.
bool capturing(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &st) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return st != hipStreamCaptureStatusNone;
}

void scratch_begin(DeviceState& ds, hipStream_t stream) {
  if (capturing(stream)) return;
  if (!ds.ws_multi) {
    if (!ds.ws_seen || stream == ds.ws_stream) return;
    check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
    if (!ds.ws_ev) check_hip(hipEventCreateWithFlags(&ds.ws_ev, hipEventDisableTiming), "hipEventCreate");
    ds.ws_multi = true;
    return;
  }
  if (stream != ds.ws_stream) check_hip(hipStreamWaitEvent(stream, ds.ws_ev, 0), "hipStreamWaitEvent");
}

void scratch_end(DeviceState& ds, hipStream_t stream) {
  if (capturing(stream)) return;
  ds.ws_seen = true;
  ds.ws_stream = stream;
  if (ds.ws_multi) check_hip(hipEventRecord(ds.ws_ev, stream), "hipEventRecord");
}

// ---------------------------------------------------------- operand views
Mat mat_from_desc(void* aligned, int64_t offset, int64_t d0, int64_t d1, int64_t s0, int64_t s1,
                  size_t esize, const char* name) {
  if (d0 < 0 || d1 < 0) fail(kErrShape, "%s: negative size (%lld, %lld)", name, (long long)d0, (long long)d1);
  Mat m;
  m.rows = d0;
  m.cols = d1;
  m.ld = d1;
  if (d0 == 0 || d1 == 0) return m;
  if (!aligned) fail(kErrArgument, "%s: null data pointer", name);
  if (offset < 0) fail(kErrArgument, "%s: negative offset %lld", name, (long long)offset);
  if (d1 > 1 && s1 != 1)
    fail(kErrStride, "%s: innermost stride %lld unsupported (must be 1)", name, (long long)s1);
  if (d0 > 1) {
    if (s0 < d1) fail(kErrStride, "%s: row stride %lld < row length %lld", name, (long long)s0, (long long)d1);
    m.ld = s0;
  }
  m.base = static_cast<char*>(aligned) + offset * (int64_t)esize;
  return m;
}

Vec vec_from_desc(void* aligned, int64_t offset, int64_t d0, int64_t s0, size_t esize, const char* name) {
  if (d0 < 0) fail(kErrShape, "%s: negative size %lld", name, (long long)d0);
  Vec v;
  v.n = d0;
  if (d0 == 0) return v;
  if (!aligned) fail(kErrArgument, "%s: null data pointer", name);
  if (offset < 0) fail(kErrArgument, "%s: negative offset %lld", name, (long long)offset);
  if (d0 > 1 && s0 != 1) fail(kErrStride, "%s: stride %lld unsupported (must be 1)", name, (long long)s0);
  v.base = static_cast<char*>(aligned) + offset * (int64_t)esize;
  return v;
}

bool is_device_pointer(const void* p, int dev) {
  hipPointerAttribute_t a;
  const hipError_t e = hipPointerGetAttributes(&a, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  if (a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged) {
    if (a.type == hipMemoryTypeDevice && a.device != dev)
      fail(kErrArgument, "operand lives on device %d but the current device is %d", a.device, dev);
    return true;
  }
  return false;
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// ------------------------------------------------------- kernel selection
struct DenseLaunch {
  int dtype;  // EDSL_DTYPE_*
  int epi;
  float alpha;
  const void* x;
  int64_t ldx;
  const void* w;
  int64_t ldw;
  const void* bias;
  void* y;
  int64_t ldy;
  int64_t M, N, K;
  // A bias whose alignment the kernel choice takes into account although
  // this launch does not add it (the GEMM of the unfused sequence, so that it
  // runs the kernel the fused launch with that bias runs); null: none.
  const void* plan_bias = nullptr;
};

void check_dims(int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K < 0) fail(kErrShape, "negative dimension");
  if (M > INT_MAX / 2 || N > INT_MAX / 2 || K > INT_MAX / 2)
    fail(kErrLimit, "dimension beyond 2^30 (M=%lld N=%lld K=%lld)", (long long)M, (long long)N,
         (long long)K);
}

// Small-M plan. Widths are tried in the order 128, 256, 64, 32 columns per
// workgroup; for each, the K split is the smallest power of two that gives at
// least one workgroup per CU (every wave keeping >= 2 steps of 16 rows). The
// first width that fills the chip is taken; when none does, the plan with the
// most workgroups. The order is measured (M=16, K=N=8192 on MI355X): 128
// columns x 4 splits beat 256 x 8 (more partial traffic), 64 x 2 (256-byte row
// runs) and 32 x 1 (8-byte loads: the per-CU request rate, not the byte
// count, limits a streaming workgroup). A forced split
// (edsl_hip_set_gemv_ksplit) limits the choice to the widths that can take it.
bool plan_gemv(const DeviceState& ds, int64_t M, int64_t N, int64_t K, bool realign, int* cols_out, int* ks_out) {
  static const int kCols[] = {128, 256, 64, 32};
  if (N < 1 || K % 16 != 0) return false;
  int best_cols = 0, best_ks = 0;
  int64_t best_wgs = 0;
  // K is walked in 16-row chunks spread evenly over the ks x wk wave slices;
  // the automatic plan gives every slice at least two, a forced split at
  // least one. Realigned rows leave the last row of W to the K tail, so K =
  // 2^n falls one chunk short of the next split: there all slices but one
  // get two.
  const int64_t chunks = K / 16 + (realign ? 1 : 0);
  // Returns true when the width fills the chip.
  auto consider = [&](int cols) {
    if (g_force_cols > 0 && cols != g_force_cols) return false;
    const int64_t wk = gemv_f32_waves_k(cols, (int)M);
    // The last column block may be partial (its lanes past N read the last
    // columns and store nothing).
    const int64_t groups = (N + cols - 1) / cols;
    int ks = 1;
    if (g_force_ksplit > 0) {
      // A forced split is taken only by widths that can honour it.
      if (g_force_ksplit > gemv_f32_max_ksplit() || K < 16 * wk * g_force_ksplit) return false;
      ks = g_force_ksplit;
    } else {
      if (chunks < 2 * wk) return false;
      while (groups * ks < ds.cus && ks * 2 <= gemv_f32_max_ksplit() && chunks >= 2 * wk * ks * 2) ks *= 2;
    }
    const int64_t wgs = groups * ks;
    if (wgs > best_wgs) {
      best_cols = cols;
      best_ks = ks;
      best_wgs = wgs;
    }
    return wgs >= ds.cus;
  };
  // Realigned rows (four columns per lane) stream at 1.5-2x the rate of the
  // 4-byte loads that 32-column blocks fall back to: those are taken only when
  // no wider block fits.
  for (int cols : kCols)
    if ((!realign || cols > 32) && consider(cols)) break;
  if (realign && best_cols == 0) consider(32);
  if (best_cols == 0) return false;
  *cols_out = best_cols;
  *ks_out = best_ks;
  return true;
}

void launch_f32(DeviceState& ds, const DenseLaunch& L, hipStream_t stream, const FixedScratch* fixed) {
  const bool has_bias = epi_has_bias(L.epi);
  // The bias whose alignment constrains the kernels: the one added, or the
  // plan's stand-in.
  const void* bias_al = has_bias ? L.bias : L.plan_bias;
  const bool aligned = al16(L.x) && al16(L.w) && al16(L.y) && (!bias_al || al16(bias_al)) &&
                       L.ldx % 4 == 0 && L.ldw % 4 == 0 && L.ldy % 4 == 0;
  const int M = (int)L.M, N = (int)L.N, K = (int)L.K;

  // Small M: the streaming kernel walks the first K16 = K - K % 16 rows; the
  // reduce kernel adds the rest. Operands need no alignment: X rows that are
  // not 16-byte aligned are read with 4-byte loads; W rows that are not (or N
  // not a multiple of 4) are realigned from 16-byte chunks or read per column,
  // with Y and the bias written and read per element.
  int gemv_cols = 0, gemv_ks = 0;
  const bool w_vec = al16(L.w) && al16(L.y) && (!bias_al || al16(bias_al)) && L.ldw % 4 == 0 &&
                     L.ldy % 4 == 0 && N % 4 == 0;
  // Realigned W rows (two aligned 16-byte chunks per lane and row) leave the
  // last row of W to the reduce kernel's K tail.
  const bool w_realign = !w_vec && N >= 4;
  const int K16 = w_realign ? ((K - 1) & ~15) : (K & ~15);
  // With W, Y or the bias not vector-aligned the small-M kernel streams W
  // realigned at ~3.3-4.4 TB/s with one row block (~2 TB/s with 4-byte loads:
  // N < 4 or 32-column blocks); the 32x32 any-shape tile reads W once per 32
  // rows of M at ~2.8 TB/s. Measured, small-M kernel vs tile: 16x8192x8191 61
  // vs 134 us, 16x4096x50257 249 vs 290, 17x4096x50257 259 vs 283,
  // 32x4096x50257 300 vs 292, 48x4096x50257 362 vs 495, 64x4096x50257 442 vs
  // 498, 64x2048x50257 254 vs 258, 64x8192x8191 115 vs 166, 33x2048x4097 32
  // vs 41; short K goes to the tile: 32x1024x32001 57 vs 49. So realigned
  // rows take the small-M kernel for K >= 2048 (K >= 1024 with one row
  // block), with at least 8 MiB of W: below that the layer is latency-bound
  // and the tile's single launch wins (4x512x511: 8.4 vs 13.9 us;
  // 16x1024x1023: even; 8x2048x2047 at 16 MiB: 15.6 vs 30.6). With 4-byte
  // loads: when the plan splits K and M <= 48 (measured up to three row
  // blocks). A forced split (edsl_hip_set_gemv_ksplit) or
  // edsl_hip_set_small_m(1) takes the small-M kernel.
  const bool gemv_planned =
      M >= 1 && M <= kGemvMaxM && K16 > 0 && plan_gemv(ds, M, N, K16, w_realign, &gemv_cols, &gemv_ks);
  const bool realigned_plan = w_realign && gemv_cols > 32;
  const int row_blocks = (M + 15) / 16;
  const bool w_large = (int64_t)K * N * (int64_t)sizeof(float) >= (8 << 20);
  // Vector-aligned W: the small-M kernel's parallelism comes from splitting
  // K, the tiles' from the M x N output, so short K favours the tiles (32x32
  // tiles read W once up to 32 rows, twice up to 64). Measured on one box,
  // small-M kernel vs 32x32 tile: one row block 16x512x512 5.7 vs 6.1 us,
  // 16x256x4096 5.7 vs 4.4, 1x256x256 5.0 vs 4.2; two 32x1024x1024 7.9 vs
  // 9.4, 32x512x512 7.5 vs 6.1; three 48x2048x2048 14.3 vs 16.9,
  // 48x1024x4096 14.3 vs 10.4; four 64x8192x8192 101 vs 115, 64x4096x8192
  // 52 vs 57, 64x2048x1024 11.2 vs 16.3, 64x2048x8192 32 vs 28, 64x2048x2048
  // 17.4 vs 16.4, 64x1024x1024 10.3 vs 9.5. With X rows not 16-byte aligned
  // the tiles are the any-shape ones and the small-M kernel is kept.
  const bool x_vec = al16(L.x) && L.ldx % 4 == 0;
  bool vec_small_m = true;
  if (x_vec) {
    if (row_blocks == 1)
      vec_small_m = K >= 512;
    else if (row_blocks == 2)
      vec_small_m = K >= 1024;
    else if (row_blocks == 3)
      vec_small_m = K >= 2048;
    else
      vec_small_m = K >= 4096 || (int64_t)K >= 2 * (int64_t)N;
  }
  if (gemv_planned &&
      ((w_vec && vec_small_m) || g_force_ksplit > 0 || g_force_small_m == 1 ||
       (realigned_plan && w_large && (K >= 2048 || (row_blocks == 1 && K >= 1024))) ||
       (!w_vec && !realigned_plan && gemv_ks > 1 && M <= 48))) {
    const bool x_ok = x_vec;
    const bool tail = K16 < K;
    if (tail && gemv_ks == 1) gemv_ks = 2;  // the reduce kernel adds the tail
    GemvF32Args a{};
    a.X = static_cast<const float*>(L.x);
    a.W = static_cast<const float*>(L.w);
    a.bias = static_cast<const float*>(L.bias);
    a.Y = static_cast<float*>(L.y);
    a.ldx = L.ldx;
    a.ldw = L.ldw;
    a.ldy = L.ldy;
    a.M = M;
    a.N = N;
    a.K = K16;
    a.k_end = K;
    a.x_tail = static_cast<const float*>(L.x);
    a.ldx_tail = L.ldx;
    a.alpha = L.alpha;
    a.ksplit = gemv_ks;
    a.ldp = ((int64_t)N + 3) & ~int64_t(3);
    const int mb = (M + 15) / 16;
    const bool scratch = a.ksplit > 1;
    const size_t part_bytes = scratch ? (size_t)a.ksplit * 16 * mb * a.ldp * sizeof(float) : 0;
    if (!has_bias) a.bias = nullptr;
    // Two columns per lane (32-column blocks) read unaligned rows per column.
    a.w_mode = w_vec ? kWVector : (realigned_plan ? kWRealign : kWScalar);
    // Vector rows only where the operands allow them; the other modes are
    // correct on any rows (a bias the epilogue does not add may still have
    // ruled vector rows out, see DenseLaunch::plan_bias).
    if (a.w_mode == kWVector && !gemv_f32_vector_rows(a)) fail(kErrInternal, "small-M W mode mismatch");
    if (fixed) {
      // Caller-fixed scratch: nothing is allocated and no cross-stream
      // ordering is added.
      if (part_bytes > fixed->bytes)
        fail(kErrLimit, "small-M plan (M=%d N=%d K=%d, %d splits) needs %zu bytes of scratch; the fixed scratch holds %zu",
             M, N, K, a.ksplit, part_bytes, fixed->bytes);
      if (part_bytes) a.partials = reinterpret_cast<float*>(fixed->base);
    } else if (scratch) {
      scratch_begin(ds, stream);
      a.partials = static_cast<float*>(ds.gemv_partials.ensure(part_bytes, false));
    }
    check_hip(launch_gemv_f32(L.epi, gemv_cols, a, stream), "gemv_f32 launch");
    if (scratch && !fixed) scratch_end(ds, stream);
    set_plan("gemv_f32 mb=%d ksplit=%d cols=%d grid=%d%s%s%s%s%s", mb, a.ksplit, gemv_cols,
             ((N + gemv_cols - 1) / gemv_cols) * a.ksplit, a.ksplit > 1 ? " +reduce" : "",
             x_ok ? "" : " +xunaligned",
             a.w_mode == kWVector ? "" : a.w_mode == kWRealign ? " +wrealigned" : " +wunaligned", tail ? " +ktail" : "",
             fixed && scratch ? " +fixed-scratch" : "");
    return;
  }

  static_assert(kF32SmallM == kGemvMaxM, "the tile planner's small-M rule covers the small-M kernel's rows");
  const int cfg = plan_f32_tile(F32TileQuery{M, N, K, L.ldx, L.ldw, aligned, ds.cus, g_force_cfg});
  const GemmF32Config& g = gemm_f32_config(cfg);
  GemmF32Args a{};
  a.A = static_cast<const float*>(L.x);
  a.B = static_cast<const float*>(L.w);
  a.bias = static_cast<const float*>(L.bias);
  a.C = static_cast<float*>(L.y);
  a.lda = L.ldx;
  a.ldb = L.ldw;
  a.ldc = L.ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.alpha = L.alpha;
  a.tiles_m = (M + g.bm - 1) / g.bm;
  a.tiles_n = (N + g.bn - 1) / g.bn;
  check_hip(launch_gemm_f32(cfg, L.epi, a, stream), "gemm_f32 launch");
  set_plan("gemm_f32 cfg=%s grid=%d", g.name, a.tiles_m * a.tiles_n);
}

void launch_i32(DeviceState& ds, const DenseLaunch& L, hipStream_t stream) {
  if (epi_act(L.epi) == ACT_LEAKY) fail(kErrDtype, "leaky_relu is float-only");
  // On integers If(v > 0, v, 0) is the ReLU: the select codes run as it.
  const int epi = epi_act(L.epi) == ACT_IF_RELU ? epi_code(epi_has_bias(L.epi), ACT_RELU) : L.epi;
  GemmI32Args a{};
  a.X = static_cast<const int32_t*>(L.x);
  a.W = static_cast<const int32_t*>(L.w);
  a.bias = static_cast<const int32_t*>(L.bias);
  a.C = static_cast<int32_t*>(L.y);
  a.ldx = L.ldx;
  a.ldw = L.ldw;
  a.ldc = L.ldy;
  a.M = (int)L.M;
  a.N = (int)L.N;
  a.K = (int)L.K;
  // The int8 path is exact for K < 2^17 (each product of int8 values has
  // magnitude <= 2^14, so no i32 partial sum can overflow). Its packed copies
  // are padded with zeros to multiples of the 128-wide tile, so any M, N and
  // K run on it; only the stores are limited to the real M x N.
  const bool tiled = a.M > 0 && a.N > 0 && a.K > 0 && a.K < (1 << 17);
  if (tiled) {
    auto pad = [](int v) { return (v + kI8Tile - 1) / kI8Tile * kI8Tile; };
    const int Mp = pad(a.M), Np = pad(a.N), Kp = pad(a.K);
    a.Kp = Kp;
    const size_t xs = (size_t)Mp * Kp, ws = (size_t)Np * Kp;
    int8_t* x8 = static_cast<int8_t*>(ds.i8_x.ensure(xs, false));
    int8_t* w8 = static_cast<int8_t*>(ds.i8_w.ensure(ws, false));
    // One range flag per 64x64 tile of the padded X and W (rewritten by every call).
    const size_t fx = (size_t)(Mp / 64) * (Kp / 64), fw = (size_t)(Np / 64) * (Kp / 64);
    uint8_t* flags = static_cast<uint8_t*>(ds.i8_flags.ensure(fx + fw, false));
    NarrowI8Args n{};
    n.X = a.X;
    n.W = a.W;
    n.X8p = x8;
    n.W8p = w8;
    n.ldx = a.ldx;
    n.ldw = a.ldw;
    n.M = a.M;
    n.N = a.N;
    n.K = a.K;
    n.Mp = Mp;
    n.Np = Np;
    n.Kp = Kp;
    n.flags_x = flags;
    n.flags_w = flags + fx;
    scratch_begin(ds, stream);
    check_hip(launch_narrow_i8(n, stream), "narrow_i8 launch");
    a.A8p = x8;
    a.B8p = w8;
    a.flags_x = flags;
    a.flags_w = flags + fx;
    const int variant = (g_force_i8 >= 0 && g_force_i8 < kI8Variants) ? g_force_i8 : kI8DefaultVariant;
    check_hip(launch_gemm_i8(epi, a, stream, variant), "gemm_i8 launch");
    scratch_end(ds, stream);
    set_plan("narrow_i8+gemm_i8 variant=%d waves=%s depth=%d grid=%d", variant, gemm_i8_layout(variant),
             gemm_i8_depth(variant, Kp),
             (Mp / kI8Tile) * (Np / kI8Tile));
  } else {
    check_hip(launch_gemm_i32_valu(epi, a, stream), "gemm_i32_valu launch");
    set_plan("gemm_i32_valu grid=%d", ((a.M + 127) / 128) * ((a.N + 127) / 128));
  }
}

void launch_dense(DeviceState& ds, const DenseLaunch& L, hipStream_t stream, const FixedScratch* fixed = nullptr) {
  check_dims(L.M, L.N, L.K);
  if (L.M == 0 || L.N == 0) {
    set_plan("empty");
    return;
  }
  if (L.epi < 0 || L.epi > 7) fail(kErrArgument, "bad epilogue code %d", L.epi);
  if (L.dtype == EDSL_DTYPE_F32)
    launch_f32(ds, L, stream, fixed);
  else if (L.dtype == EDSL_DTYPE_I32 && !fixed)
    launch_i32(ds, L, stream);
  else
    fail(kErrDtype, "bad dtype %d", L.dtype);
}

// ------------------------------------------------- synchronous host entry
// Shapes: X [M,K], W [K,N], bias [N] (when the epilogue adds one), Y [M,N].
// Copies a host matrix into a device buffer with rows padded to a multiple
// of 4 elements (and back), staged through the pinned ring.
void copy_h2d(void* d, int64_t dld, const Mat& m, size_t es, hipStream_t stream) {
  stage_h2d(d, dld, m.base, m.ld, m.rows, m.cols, es, stream);
}

void copy_d2h(const Mat& m, const void* d, int64_t dld, size_t es, hipStream_t stream) {
  stage_d2h(m.base, m.ld, d, dld, m.rows, m.cols, es, stream);
}

// One f32 layer with host X and Y, large enough to overlap PCIe copies with
// the kernels: W (and b) go up first; then X is uploaded in kPipeBlocks row
// blocks on one stream, each block's kernel runs on a second stream as soon
// as its rows have landed, and its Y rows come down on a third while the next
// block computes. Returns false when the call does not qualify (the caller
// then runs the plain staged sequence).
constexpr int64_t kPipeMinRows = 1024;
constexpr int64_t kPipeRowAlign = 256;

bool pipelined_host_layer(DeviceState& ds, int dev, int dtype, const LayerOp& op, const Mat& Y) {
  const Mat& X = *op.X;
  const Mat& W = *op.W;
  const int64_t M = X.rows, K = X.cols, N = W.cols;
  if (dtype != EDSL_DTYPE_F32 || M < kPipeMinRows || K == 0 || N == 0) return false;
  if (is_device_pointer(X.base, dev) || is_device_pointer(Y.base, dev)) return false;
  const size_t es = 4;
  if ((size_t)M * (size_t)(K + N) * es < (size_t)(16u << 20)) return false;
  if (!ds.pipe_ready) {
    check_hip(hipStreamCreateWithFlags(&ds.pipe_up, hipStreamNonBlocking), "hipStreamCreate");
    check_hip(hipStreamCreateWithFlags(&ds.pipe_run, hipStreamNonBlocking), "hipStreamCreate");
    check_hip(hipStreamCreateWithFlags(&ds.pipe_down, hipStreamNonBlocking), "hipStreamCreate");
    check_hip(hipEventCreateWithFlags(&ds.ev_w, hipEventDisableTiming), "hipEventCreate");
    for (int i = 0; i < kPipeBlocks; ++i) {
      check_hip(hipEventCreateWithFlags(&ds.ev_x[i], hipEventDisableTiming), "hipEventCreate");
      check_hip(hipEventCreateWithFlags(&ds.ev_g[i], hipEventDisableTiming), "hipEventCreate");
    }
    ds.pipe_ready = true;
  }
  // Every host-buffer call is synchronous, so no earlier work on these or the
  // legacy stream can still touch the staging buffers.
  const int64_t dldx = (K + 3) & ~int64_t(3), dldy = (N + 3) & ~int64_t(3);
  char* dx = static_cast<char*>(ds.stage[0].ensure((size_t)M * dldx * es, false));
  char* dy = static_cast<char*>(ds.stage[3].ensure((size_t)M * dldy * es, false));
  DenseLaunch L{};
  L.dtype = dtype;
  L.epi = op.epi;
  L.alpha = op.alpha;
  L.K = K;
  L.N = N;
  if (is_device_pointer(W.base, dev)) {
    L.w = W.base;
    L.ldw = W.ld;
  } else {
    const int64_t dldw = (N + 3) & ~int64_t(3);
    void* dw = ds.stage[1].ensure((size_t)K * dldw * es, false);
    stage_h2d(dw, dldw, W.base, W.ld, K, N, es, ds.pipe_up);
    L.w = dw;
    L.ldw = dldw;
  }
  if (epi_has_bias(op.epi)) {
    if (is_device_pointer(op.b->base, dev)) {
      L.bias = op.b->base;
    } else {
      void* d = ds.stage[2].ensure((size_t)N * es, false);
      check_hip(hipMemcpyAsync(d, op.b->base, (size_t)N * es, hipMemcpyHostToDevice, ds.pipe_up),
                "hipMemcpyAsync H2D");
      L.bias = d;
    }
  }
  check_hip(hipEventRecord(ds.ev_w, ds.pipe_up), "hipEventRecord");
  check_hip(hipStreamWaitEvent(ds.pipe_run, ds.ev_w, 0), "hipStreamWaitEvent");

  const int64_t mb = ((M + kPipeBlocks - 1) / kPipeBlocks + kPipeRowAlign - 1) / kPipeRowAlign * kPipeRowAlign;
  const int nb = (int)((M + mb - 1) / mb);
  std::string plan0;
  auto download = [&](int i) {
    const int64_t r0 = i * mb, rows = std::min(mb, M - r0);
    check_hip(hipStreamWaitEvent(ds.pipe_down, ds.ev_g[i], 0), "hipStreamWaitEvent");
    stage_d2h(Y.base + r0 * Y.ld * (int64_t)es, Y.ld, dy + r0 * dldy * (int64_t)es, dldy, rows, N, es,
              ds.pipe_down);
  };
  for (int i = 0; i < nb; ++i) {
    const int64_t r0 = i * mb, rows = std::min(mb, M - r0);
    stage_h2d(dx + r0 * dldx * (int64_t)es, dldx, X.base + r0 * X.ld * (int64_t)es, X.ld, rows, K, es,
              ds.pipe_up);
    check_hip(hipEventRecord(ds.ev_x[i], ds.pipe_up), "hipEventRecord");
    check_hip(hipStreamWaitEvent(ds.pipe_run, ds.ev_x[i], 0), "hipStreamWaitEvent");
    L.M = rows;
    L.x = dx + r0 * dldx * (int64_t)es;
    L.ldx = dldx;
    L.y = dy + r0 * dldy * (int64_t)es;
    L.ldy = dldy;
    {
      std::lock_guard<std::mutex> lock(g_mu);
      launch_dense(ds, L, ds.pipe_run);
    }
    if (i == 0) plan0 = t_plan;
    check_hip(hipEventRecord(ds.ev_g[i], ds.pipe_run), "hipEventRecord");
    if (i > 0) download(i - 1);  // overlaps block i's kernel
  }
  download(nb - 1);
  check_hip(hipStreamSynchronize(ds.pipe_up), "hipStreamSynchronize");
  check_hip(hipStreamSynchronize(ds.pipe_run), "hipStreamSynchronize");
  check_hip(hipStreamSynchronize(ds.pipe_down), "hipStreamSynchronize");
  check_hip(hipGetLastError(), "kernel execution");
  set_plan("host pipeline %d x %lld rows: %s", nb, (long long)mb, plan0.c_str());
  return true;
}

void sync_dense_chain(int dtype, const LayerOp* layers, int n, const Mat& Y) {
  if (n < 1 || !layers || !layers[0].X) fail(kErrArgument, "a chain needs at least one layer and an input");
  const int64_t M = layers[0].X->rows;
  int64_t K = layers[0].X->cols;
  for (int i = 0; i < n; ++i) {
    const LayerOp& L = layers[i];
    if (i > 0 && L.X) fail(kErrArgument, "layer %d: only the first layer reads a parameter as its input", i);
    if (!L.W) fail(kErrArgument, "layer %d: null weight", i);
    if (L.W->rows != K)
      fail(kErrShape, "matmul inner dimensions must match: lhs K=%lld, rhs K=%lld", (long long)K,
           (long long)L.W->rows);
    const int64_t N = L.W->cols;
    if (epi_has_bias(L.epi) && (!L.b || L.b->n != N))
      fail(kErrShape, "bias length %lld does not match N=%lld", (long long)(L.b ? L.b->n : -1), (long long)N);
    check_dims(M, N, K);
    K = N;
  }
  if (Y.rows != M || Y.cols != K)
    fail(kErrShape, "output shape [%lld,%lld] does not match [%lld,%lld]", (long long)Y.rows,
         (long long)Y.cols, (long long)M, (long long)K);
  if (M == 0 || K == 0) {
    set_plan("empty");
    return;
  }

  std::lock_guard<std::mutex> host_lock(g_host_mu);
  int dev = 0;
  DeviceState* dsp = nullptr;
  bool no_pipeline = false;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    read_env_overrides();
    dsp = &device_state(&dev);
    no_pipeline = g_no_pipeline;
  }
  DeviceState& ds = *dsp;
  if (n == 1 && !no_pipeline) {
    bool done = false;
    try {
      done = pipelined_host_layer(ds, dev, dtype, layers[0], Y);
    } catch (...) {
      // Drain the pipeline's streams before anything else touches the
      // staging buffers (the legacy stream does not order against them).
      if (ds.pipe_ready)
        for (hipStream_t st : {ds.pipe_up, ds.pipe_run, ds.pipe_down}) (void)hipStreamSynchronize(st);
      throw;
    }
    if (done) return;
  }
  hipStream_t stream = nullptr;
  const size_t es = 4;

  // Host operands are staged through persistent device buffers with 16-byte
  // aligned rows so the fast kernels stay eligible. The stream orders each
  // layer's staging copies after the previous layer's kernels, so one set of
  // staging buffers serves every layer.
  auto stage_in = [&](const Mat& m, DevBuf& buf, int64_t* ld) -> const void* {
    if (m.rows == 0 || m.cols == 0 || is_device_pointer(m.base, dev)) {
      *ld = m.ld;
      return m.base;
    }
    const int64_t dld = (m.cols + 3) & ~int64_t(3);
    void* d = buf.ensure((size_t)m.rows * dld * es, false);
    copy_h2d(d, dld, m, es, stream);
    *ld = dld;
    return d;
  };

  // Intermediate activations ping-pong between two device buffers sized up
  // front, so no buffer is reallocated while a kernel may still use it.
  int64_t inter = 0;
  for (int i = 0; i + 1 < n; ++i) inter = std::max(inter, M * ((layers[i].W->cols + 3) & ~int64_t(3)));
  void* hbuf[2] = {nullptr, nullptr};
  if (n > 1) {
    hbuf[0] = ds.chain[0].ensure((size_t)inter * es, false);
    if (n > 2) hbuf[1] = ds.chain[1].ensure((size_t)inter * es, false);
  }
  const bool y_dev = is_device_pointer(Y.base, dev);
  const int64_t N_last = Y.cols;
  void* ystage = nullptr;
  int64_t ystage_ld = (N_last + 3) & ~int64_t(3);
  if (!y_dev) ystage = ds.stage[3].ensure((size_t)M * ystage_ld * es, false);

  std::string plans;
  const void* prev = nullptr;
  int64_t prev_ld = 0;
  for (int i = 0; i < n; ++i) {
    const LayerOp& op = layers[i];
    DenseLaunch L{};
    L.dtype = dtype;
    L.epi = op.epi;
    L.alpha = op.alpha;
    L.M = M;
    L.K = op.W->rows;
    L.N = op.W->cols;
    if (i == 0) {
      L.x = stage_in(*op.X, ds.stage[0], &L.ldx);
    } else {
      L.x = prev;
      L.ldx = prev_ld;
    }
    L.w = stage_in(*op.W, ds.stage[1], &L.ldw);
    if (epi_has_bias(op.epi)) {
      if (is_device_pointer(op.b->base, dev)) {
        L.bias = op.b->base;
      } else {
        void* d = ds.stage[2].ensure((size_t)L.N * es, false);
        check_hip(hipMemcpyAsync(d, op.b->base, (size_t)L.N * es, hipMemcpyHostToDevice, stream),
                  "hipMemcpyAsync H2D");
        L.bias = d;
      }
    }
    if (i + 1 < n) {
      L.y = hbuf[i % 2];
      L.ldy = (L.N + 3) & ~int64_t(3);
    } else if (y_dev) {
      L.y = Y.base;
      L.ldy = Y.ld;
    } else {
      L.y = ystage;
      L.ldy = ystage_ld;
    }
    {
      std::lock_guard<std::mutex> lock(g_mu);
      launch_dense(ds, L, stream);
    }
    if (n > 1) plans += (i ? " | " : "") + t_plan;
    prev = L.y;
    prev_ld = L.ldy;
  }
  if (n > 1) t_plan = plans;
  if (!y_dev) copy_d2h(Y, ystage, ystage_ld, es, stream);
  check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
  check_hip(hipGetLastError(), "kernel execution");
}

// The row stride of a matrix with a single row is never used to reach a second
// row, so a caller may pass anything there (a (1,K) view of a column vector
// has stride 1, a broadcast view 0). Such strides are replaced by the row
// length, as mat_from_desc does for descriptors, so that the planner's
// alignment tests and the X-row staging copy (whose source pitch must cover a
// row) see a consistent layout.
void normalize_single_row_strides(int64_t M, int64_t N, int64_t K, int64_t* ldx, int64_t* ldw, int64_t* ldy) {
  if (M <= 1) {
    *ldx = K;
    *ldy = N;
  }
  if (K <= 1) *ldw = N;
}

void sync_dense(int dtype, int epi, float alpha, const Mat& X, const Mat& W, const Vec* b, const Mat& Y) {
  const LayerOp op{&X, &W, b, epi, alpha};
  sync_dense_chain(dtype, &op, 1, Y);
}

int current_device() {
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  return dev;
}

ResidentCopy::~ResidentCopy() {
  if (!dev) return;
  int cur = -1;
  const bool switch_dev = hipGetDevice(&cur) == hipSuccess && cur != device;
  if (switch_dev) (void)hipSetDevice(device);
  (void)hipFree(dev);  // the calls that read it were synchronous
  if (switch_dev) (void)hipSetDevice(cur);
  (void)hipGetLastError();
}

std::shared_ptr<ResidentCopy> make_resident_copy(const void* src, int64_t rows, int64_t cols, size_t esize) {
  if (rows < 0 || cols < 0) fail(kErrShape, "negative size (%lld, %lld)", (long long)rows, (long long)cols);
  if (!src && rows > 0 && cols > 0) fail(kErrArgument, "null data pointer");
  std::lock_guard<std::mutex> lock(g_host_mu);  // the pinned staging ring is shared
  auto c = std::make_shared<ResidentCopy>();
  c->device = current_device();
  c->rows = rows;
  c->cols = cols;
  c->dev_ld = (cols + 3) & ~int64_t(3);
  c->bytes = std::max<size_t>((size_t)rows * (size_t)c->dev_ld * esize, 256);
  check_hip(hipMalloc(&c->dev, c->bytes), "hipMalloc (resident parameter)");
  if (rows > 0 && cols > 0) {
    if (is_device_pointer(src, c->device)) {
      check_hip(hipMemcpy2DAsync(c->dev, (size_t)c->dev_ld * esize, src, (size_t)cols * esize, (size_t)cols * esize,
                                 rows, hipMemcpyDeviceToDevice, nullptr),
                "hipMemcpy2DAsync (resident parameter)");
    } else {
      stage_h2d(c->dev, c->dev_ld, static_cast<const char*>(src), cols, rows, cols, esize, nullptr);
    }
    check_hip(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
  }
  return c;
}

void dense_f32_launch(const float* X, int64_t ldx, const float* W, int64_t ldw, const float* bias, float* Y,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue, float alpha, void* stream,
                      const FixedScratch* fixed, const float* plan_bias) {
  if (epi_has_bias(epilogue) && !bias && N > 0) fail(kErrArgument, "epilogue adds a bias but bias is null");
  if (M > 0 && N > 0 && (!Y || (K > 0 && (!X || !W)))) fail(kErrArgument, "null operand");
  if (K > 0 && M > 1 && ldx < K) fail(kErrStride, "ldx < K");
  if (N > 0 && K > 1 && ldw < N) fail(kErrStride, "ldw < N");
  if (N > 0 && M > 1 && ldy < N) fail(kErrStride, "ldy < N");
  normalize_single_row_strides(M, N, K, &ldx, &ldw, &ldy);
  std::lock_guard<std::mutex> lock(g_mu);
  read_env_overrides();
  DeviceState& ds = device_state(nullptr);
  DenseLaunch L{EDSL_DTYPE_F32, epilogue, alpha, X, ldx, W, ldw, bias, Y, ldy, M, N, K};
  L.plan_bias = plan_bias;
  launch_dense(ds, L, static_cast<hipStream_t>(stream), fixed);
}

}  // namespace rt
}  // namespace edsl

using namespace edsl;
using namespace edsl::rt;

// ====================================================================== ABI
#define MEMREF2(T, p) \
  T *p##_allocated, T *p##_aligned, int64_t p##_offset, int64_t p##_size0, int64_t p##_size1, \
      int64_t p##_stride0, int64_t p##_stride1
#define MEMREF1(T, p) T *p##_allocated, T *p##_aligned, int64_t p##_offset, int64_t p##_size0, int64_t p##_stride0
#define MAT(p, name) \
  mat_from_desc((void*)p##_aligned, p##_offset, p##_size0, p##_size1, p##_stride0, p##_stride1, 4, name)
#define VEC(p, name) vec_from_desc((void*)p##_aligned, p##_offset, p##_size0, p##_stride0, 4, name)

extern "C" {

void edsl_hip_matmul_f32(MEMREF2(float, A), MEMREF2(float, B), MEMREF2(float, C)) {
  (void)A_allocated; (void)B_allocated; (void)C_allocated;
  guarded([&] { sync_dense(EDSL_DTYPE_F32, EDSL_EPI_NONE, 0.f, MAT(A, "A"), MAT(B, "B"), nullptr, MAT(C, "C")); });
}

void edsl_hip_matmul_i32(MEMREF2(int32_t, A), MEMREF2(int32_t, B), MEMREF2(int32_t, C)) {
  (void)A_allocated; (void)B_allocated; (void)C_allocated;
  guarded([&] { sync_dense(EDSL_DTYPE_I32, EDSL_EPI_NONE, 0.f, MAT(A, "A"), MAT(B, "B"), nullptr, MAT(C, "C")); });
}

void edsl_hip_matmul_relu_f32(MEMREF2(float, A), MEMREF2(float, B), MEMREF2(float, C)) {
  (void)A_allocated; (void)B_allocated; (void)C_allocated;
  guarded([&] { sync_dense(EDSL_DTYPE_F32, EDSL_EPI_RELU, 0.f, MAT(A, "A"), MAT(B, "B"), nullptr, MAT(C, "C")); });
}

void edsl_hip_matmul_relu_i32(MEMREF2(int32_t, A), MEMREF2(int32_t, B), MEMREF2(int32_t, C)) {
  (void)A_allocated; (void)B_allocated; (void)C_allocated;
  guarded([&] { sync_dense(EDSL_DTYPE_I32, EDSL_EPI_RELU, 0.f, MAT(A, "A"), MAT(B, "B"), nullptr, MAT(C, "C")); });
}

void edsl_hip_matmul_bias_f32(MEMREF2(float, X), MEMREF2(float, W), MEMREF1(float, b), MEMREF2(float, Y)) {
  (void)X_allocated; (void)W_allocated; (void)b_allocated; (void)Y_allocated;
  guarded([&] {
    const Vec bv = VEC(b, "b");
    sync_dense(EDSL_DTYPE_F32, EDSL_EPI_BIAS, 0.f, MAT(X, "X"), MAT(W, "W"), &bv, MAT(Y, "Y"));
  });
}

void edsl_hip_matmul_bias_i32(MEMREF2(int32_t, X), MEMREF2(int32_t, W), MEMREF1(int32_t, b),
                              MEMREF2(int32_t, Y)) {
  (void)X_allocated; (void)W_allocated; (void)b_allocated; (void)Y_allocated;
  guarded([&] {
    const Vec bv = VEC(b, "b");
    sync_dense(EDSL_DTYPE_I32, EDSL_EPI_BIAS, 0.f, MAT(X, "X"), MAT(W, "W"), &bv, MAT(Y, "Y"));
  });
}

void edsl_hip_dense_relu_f32(MEMREF2(float, X), MEMREF2(float, W), MEMREF1(float, b), MEMREF2(float, Y)) {
  (void)X_allocated; (void)W_allocated; (void)b_allocated; (void)Y_allocated;
  guarded([&] {
    const Vec bv = VEC(b, "b");
    sync_dense(EDSL_DTYPE_F32, EDSL_EPI_BIAS_RELU, 0.f, MAT(X, "X"), MAT(W, "W"), &bv, MAT(Y, "Y"));
  });
}

void edsl_hip_dense_relu_i32(MEMREF2(int32_t, X), MEMREF2(int32_t, W), MEMREF1(int32_t, b),
                             MEMREF2(int32_t, Y)) {
  (void)X_allocated; (void)W_allocated; (void)b_allocated; (void)Y_allocated;
  guarded([&] {
    const Vec bv = VEC(b, "b");
    sync_dense(EDSL_DTYPE_I32, EDSL_EPI_BIAS_RELU, 0.f, MAT(X, "X"), MAT(W, "W"), &bv, MAT(Y, "Y"));
  });
}

void edsl_hip_dense_leaky_relu_f32(MEMREF2(float, X), MEMREF2(float, W), MEMREF1(float, b), MEMREF2(float, Y),
                                   float alpha) {
  (void)X_allocated; (void)W_allocated; (void)b_allocated; (void)Y_allocated;
  guarded([&] {
    const Vec bv = VEC(b, "b");
    sync_dense(EDSL_DTYPE_F32, EDSL_EPI_BIAS_LEAKY, alpha, MAT(X, "X"), MAT(W, "W"), &bv, MAT(Y, "Y"));
  });
}

void edsl_hip_dense_if_relu_f32(MEMREF2(float, X), MEMREF2(float, W), MEMREF1(float, b), MEMREF2(float, Y)) {
  (void)X_allocated; (void)W_allocated; (void)b_allocated; (void)Y_allocated;
  guarded([&] {
    const Vec bv = VEC(b, "b");
    sync_dense(EDSL_DTYPE_F32, EDSL_EPI_BIAS_IF_RELU, 0.f, MAT(X, "X"), MAT(W, "W"), &bv, MAT(Y, "Y"));
  });
}

void edsl_hip_matmul_if_relu_f32(MEMREF2(float, A), MEMREF2(float, B), MEMREF2(float, C)) {
  (void)A_allocated; (void)B_allocated; (void)C_allocated;
  guarded([&] { sync_dense(EDSL_DTYPE_F32, EDSL_EPI_IF_RELU, 0.f, MAT(A, "A"), MAT(B, "B"), nullptr, MAT(C, "C")); });
}

int edsl_hip_execute_gpu_function(int pattern, int dtype, int num_inputs, const void* const* input_ptrs,
                                  const int64_t* const* input_shapes, const int* input_ranks, void* output,
                                  const int64_t* output_shape, int output_rank, size_t element_size,
                                  float alpha) {
  return guarded([&] {
    if (element_size != 4) fail(kErrDtype, "element_size %zu unsupported (f32 and i32 are 4 bytes)", element_size);
    if (dtype != EDSL_DTYPE_F32 && dtype != EDSL_DTYPE_I32) fail(kErrDtype, "bad dtype %d", dtype);
    int epi = 0;
    int want_inputs = 3;
    switch (pattern) {
      case EDSL_PATTERN_MATMUL: epi = EDSL_EPI_NONE; want_inputs = 2; break;
      case EDSL_PATTERN_MATMUL_RELU: epi = EDSL_EPI_RELU; want_inputs = 2; break;
      case EDSL_PATTERN_MATMUL_BIAS: epi = EDSL_EPI_BIAS; break;
      case EDSL_PATTERN_DENSE_RELU: epi = EDSL_EPI_BIAS_RELU; break;
      case EDSL_PATTERN_DENSE_LEAKY: epi = EDSL_EPI_BIAS_LEAKY; break;
      case EDSL_PATTERN_DENSE_IF_RELU: epi = EDSL_EPI_BIAS_IF_RELU; break;
      case EDSL_PATTERN_MATMUL_IF_RELU: epi = EDSL_EPI_IF_RELU; want_inputs = 2; break;
      default: fail(kErrArgument, "unknown pattern %d", pattern);
    }
    if (num_inputs != want_inputs)
      fail(kErrArgument, "pattern %d takes %d inputs, got %d", pattern, want_inputs, num_inputs);
    if (!input_ptrs || !input_shapes || !input_ranks || !output_shape)
      fail(kErrArgument, "null argument array");
    for (int i = 0; i < 2; ++i)
      if (input_ranks[i] != 2) fail(kErrShape, "input %d must be 2-D, got rank %d", i, input_ranks[i]);
    if (want_inputs == 3 && input_ranks[2] != 1) fail(kErrShape, "bias must be 1-D, got rank %d", input_ranks[2]);
    if (output_rank != 2) fail(kErrShape, "output must be 2-D, got rank %d", output_rank);
    auto contiguous = [&](const void* p, const int64_t* s, const char* name) {
      return mat_from_desc(const_cast<void*>(p), 0, s[0], s[1], s[1], 1, 4, name);
    };
    const Mat X = contiguous(input_ptrs[0], input_shapes[0], "lhs");
    const Mat W = contiguous(input_ptrs[1], input_shapes[1], "rhs");
    const Mat Y = contiguous(output, output_shape, "output");
    Vec b;
    if (want_inputs == 3) b = vec_from_desc(const_cast<void*>(input_ptrs[2]), 0, input_shapes[2][0], 1, 4, "bias");
    sync_dense(dtype, epi, alpha, X, W, want_inputs == 3 ? &b : nullptr, Y);
  });
}

int edsl_hip_last_error(char* buf, size_t len) {
  copy_out(t_err_msg, buf, len);
  return t_err_code;
}

void edsl_hip_clear_error(void) {
  t_err_code = 0;
  t_err_msg.clear();
}

int edsl_hip_dense_f32_launch(const float* X, int64_t ldx, const float* W, int64_t ldw, const float* bias,
                              float* Y, int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue,
                              float alpha, void* stream) {
  return guarded([&] { dense_f32_launch(X, ldx, W, ldw, bias, Y, ldy, M, N, K, epilogue, alpha, stream, nullptr); });
}

int edsl_hip_dense_f32_launch_unfused(const float* X, int64_t ldx, const float* W, int64_t ldw,
                                      const float* bias, float* Y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                                      int epilogue, float alpha, void* stream) {
  return guarded([&] {
    // The checks of dense_f32_launch, before the fill touches Y.
    if (epilogue < 0 || epilogue > 7) fail(kErrArgument, "bad epilogue code %d", epilogue);
    check_dims(M, N, K);
    if (epi_has_bias(epilogue) && !bias && N > 0) fail(kErrArgument, "epilogue adds a bias but bias is null");
    if (M > 0 && N > 0 && (!Y || (K > 0 && (!X || !W)))) fail(kErrArgument, "null operand");
    if (K > 0 && M > 1 && ldx < K) fail(kErrStride, "ldx < K");
    if (N > 0 && K > 1 && ldw < N) fail(kErrStride, "ldw < N");
    if (N > 0 && M > 1 && ldy < N) fail(kErrStride, "ldy < N");
    if (M <= 1) ldy = N;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (M > 0 && N > 0) check_hip(launch_fill_zero_f32(Y, ldy, (int)M, (int)N, s), "fill launch");
    // The GEMM plans as the fused launch with this bias would, so that both
    // run the same kernel (and give the same bits).
    dense_f32_launch(X, ldx, W, ldw, nullptr, Y, ldy, M, N, K, EDSL_EPI_NONE, 0.f, stream, nullptr,
                     epi_has_bias(epilogue) ? bias : nullptr);
    const std::string gemm_plan = t_plan;
    if (M > 0 && N > 0) check_hip(launch_bias_act_f32(Y, ldy, bias, (int)M, (int)N, epilogue, alpha, s), "bias_act launch");
    set_plan("unfused: fill | %s | bias_act epi=%d", gemm_plan.c_str(), epilogue);
  });
}

int edsl_hip_dense_i32_launch(const int32_t* X, int64_t ldx, const int32_t* W, int64_t ldw,
                              const int32_t* bias, int32_t* Y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                              int epilogue, void* stream) {
  return guarded([&] {
    if (epi_has_bias(epilogue) && !bias && N > 0) fail(kErrArgument, "epilogue adds a bias but bias is null");
    if (M > 0 && N > 0 && (!Y || (K > 0 && (!X || !W)))) fail(kErrArgument, "null operand");
    if (K > 0 && M > 1 && ldx < K) fail(kErrStride, "ldx < K");
    if (N > 0 && K > 1 && ldw < N) fail(kErrStride, "ldw < N");
    if (N > 0 && M > 1 && ldy < N) fail(kErrStride, "ldy < N");
    normalize_single_row_strides(M, N, K, &ldx, &ldw, &ldy);
    std::lock_guard<std::mutex> lock(g_mu);
    read_env_overrides();
    DeviceState& ds = device_state(nullptr);
    DenseLaunch L{EDSL_DTYPE_I32, epilogue, 0.f, X, ldx, W, ldw, bias, Y, ldy, M, N, K};
    launch_dense(ds, L, static_cast<hipStream_t>(stream));
  });
}

int edsl_hip_last_plan(char* buf, size_t len) { return copy_out(t_plan, buf, len); }

void edsl_hip_set_f32_config(int cfg) {
  std::lock_guard<std::mutex> lock(g_mu);
  read_env_overrides();
  g_force_cfg = cfg;
}

void edsl_hip_set_gemv_ksplit(int ksplit) {
  std::lock_guard<std::mutex> lock(g_mu);
  read_env_overrides();
  g_force_ksplit = ksplit;
}

void edsl_hip_set_small_m(int mode) {
  std::lock_guard<std::mutex> lock(g_mu);
  read_env_overrides();
  g_force_small_m = mode;
}

void edsl_hip_set_gemv_cols(int cols) {
  std::lock_guard<std::mutex> lock(g_mu);
  read_env_overrides();
  g_force_cols = cols;
}

void edsl_hip_set_i8_variant(int variant) {
  std::lock_guard<std::mutex> lock(g_mu);
  read_env_overrides();
  g_force_i8 = variant;
}

int edsl_hip_i8_variant_count(void) { return kI8Variants; }

int edsl_hip_f32_config_count(void) { return gemm_f32_num_configs(); }

int edsl_hip_f32_config_name(int cfg, char* buf, size_t len) {
  if (cfg < 0 || cfg >= gemm_f32_num_configs()) return -1;
  return copy_out(gemm_f32_config(cfg).name, buf, len);
}

}  // extern "C"
