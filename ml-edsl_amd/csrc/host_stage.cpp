// Host <-> device copies of the synchronous host-buffer entry points.
//
// The reference's GPU path copies every operand in and every result out on
// each call (reference cpp/src/MLIRCompiler.cpp:367-454); the host-buffer
// entries here keep that contract. A copy from pageable memory runs at the
// driver's internal staging rate; this file stages through the library's own
// pinned ring instead:
//
//   H2D: chunk i is copied (by a pool of host threads) into pinned slot
//        i % kSlots, then an async DMA moves it to the device while the host
//        fills the next slot; a slot is refilled only after the DMA that last
//        read it has completed (one event per slot).
//   D2H: DMAs into kSlots slots are queued ahead; as each completes the pool
//        copies it out and the slot's next DMA is queued.
//
// The device side uses row pitch `dld` (elements), the host side `hld`; chunks
// are whole rows, so padded and strided layouts go through the same path.
// Copies smaller than kMinStaged bytes, with rows longer than a slot, or on a
// host where pinned memory cannot be allocated use the plain async copy. Callers hold the runtime's global lock, so the ring and
// the pool serve one copy at a time.
#include "host_stage.hpp"

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include <unistd.h>

#include "runtime_internal.hpp"

namespace edsl {
namespace rt {
namespace {

constexpr int kSlots = 4;
constexpr size_t kSlotBytes = 8u << 20;
constexpr size_t kMinStaged = 2u << 20;
constexpr int kMaxStageDevices = 64;

// Persistent worker threads for the pageable <-> pinned copies. run(fn)
// calls fn(part, parts) for every part in [0, parts): the last part on the
// calling thread, the others on the workers; it returns when all are done.
class CopyPool {
 public:
  static CopyPool& get() {
    static CopyPool pool(worker_count());
    return pool;
  }
  int parts() const { return (int)threads_.size() + 1; }

  void run(const std::function<void(int, int)>& fn) {
    const int n = parts();
    if (n == 1 || getpid() != owner_) {
      // No workers (or a forked child, which has none of the parent's
      // threads): every part on the calling thread.
      for (int p = 0; p < n; ++p) fn(p, n);
      return;
    }
    {
      std::lock_guard<std::mutex> lk(mu_);
      fn_ = &fn;
      remaining_ = n - 1;
      ++gen_;
    }
    go_.notify_all();
    fn(n - 1, n);
    std::unique_lock<std::mutex> lk(mu_);
    done_.wait(lk, [&] { return remaining_ == 0; });
    fn_ = nullptr;
  }

  ~CopyPool() {
    if (getpid() != owner_) {
      // A forked child: the worker threads are the parent's.
      for (auto& t : threads_) t.detach();
      return;
    }
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
    }
    go_.notify_all();
    for (auto& t : threads_) t.join();
  }

 private:
  static int worker_count() {
    if (const char* s = getenv("EDSL_HIP_STAGE_THREADS")) return std::max(0, atoi(s) - 1);
    const unsigned hw = std::thread::hardware_concurrency();
    return (int)std::min(8u, std::max(2u, hw / 2)) - 1;
  }

  explicit CopyPool(int workers) : owner_(getpid()) {
    for (int i = 0; i < workers; ++i) threads_.emplace_back([this, i] { loop(i); });
  }

  void loop(int id) {
    uint64_t seen = 0;
    for (;;) {
      const std::function<void(int, int)>* fn;
      {
        std::unique_lock<std::mutex> lk(mu_);
        go_.wait(lk, [&] { return stop_ || gen_ != seen; });
        if (stop_) return;
        seen = gen_;
        fn = fn_;
      }
      (*fn)(id, parts());
      std::lock_guard<std::mutex> lk(mu_);
      if (--remaining_ == 0) done_.notify_one();
    }
  }

  const pid_t owner_;
  std::mutex mu_;
  std::condition_variable go_, done_;
  const std::function<void(int, int)>* fn_ = nullptr;
  uint64_t gen_ = 0;
  int remaining_ = 0;
  bool stop_ = false;
  std::vector<std::thread> threads_;
};

// Pinned slots and their completion events, one ring per device. Never freed:
// the pinned pages are released with the process.
struct Ring {
  char* slot[kSlots] = {};
  hipEvent_t ev[kSlots] = {};
  bool busy[kSlots] = {};
  bool ready = false;
  bool unavailable = false;  // pinned memory could not be allocated: direct copies
};
Ring g_ring[kMaxStageDevices];

// The current device's ring, or nullptr when pinned memory is unavailable.
Ring* ring_for_current_device() {
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= kMaxStageDevices) fail(kErrLimit, "device index %d out of range", dev);
  Ring& r = g_ring[dev];
  if (!r.ready && !r.unavailable) {
    for (int i = 0; i < kSlots && !r.unavailable; ++i) {
      if (hipHostMalloc(reinterpret_cast<void**>(&r.slot[i]), kSlotBytes, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();  // not an error of the call: fall back to direct copies
        for (int j = 0; j < i; ++j) {  // nothing has used these yet
          (void)hipHostFree(r.slot[j]);
          (void)hipEventDestroy(r.ev[j]);
          r.slot[j] = nullptr;
        }
        r.slot[i] = nullptr;
        r.unavailable = true;
        break;
      }
      check_hip(hipEventCreateWithFlags(&r.ev[i], hipEventDisableTiming), "hipEventCreate");
    }
    r.ready = !r.unavailable;
  }
  return r.ready ? &r : nullptr;
}

// Copies `rows` rows of `row_bytes` bytes from src (pitch src_pitch) to dst
// (pitch dst_pitch) on the pool; one flat range when both sides are dense.
void pool_copy_rows(char* dst, size_t dst_pitch, const char* src, size_t src_pitch, int64_t rows,
                    size_t row_bytes) {
  CopyPool& pool = CopyPool::get();
  if (dst_pitch == row_bytes && src_pitch == row_bytes) {
    const size_t total = (size_t)rows * row_bytes;
    pool.run([&](int part, int parts) {
      const size_t per = ((total + parts - 1) / parts + 63) & ~size_t(63);
      const size_t b = std::min(total, per * part), e = std::min(total, b + per);
      if (e > b) memcpy(dst + b, src + b, e - b);
    });
    return;
  }
  pool.run([&](int part, int parts) {
    const int64_t per = (rows + parts - 1) / parts;
    const int64_t b = std::min<int64_t>(rows, per * part), e = std::min<int64_t>(rows, b + per);
    for (int64_t r = b; r < e; ++r) memcpy(dst + r * dst_pitch, src + r * src_pitch, row_bytes);
  });
}

bool direct(int64_t rows, int64_t dld, size_t es) {
  const size_t row = (size_t)dld * es;
  return (size_t)rows * row < kMinStaged || row > kSlotBytes;
}

}  // namespace

void stage_h2d(void* dev, int64_t dld, const void* host, int64_t hld, int64_t rows, int64_t cols, size_t es,
               hipStream_t stream) {
  if (rows <= 0 || cols <= 0) return;
  Ring* rp = direct(rows, dld, es) ? nullptr : ring_for_current_device();
  if (!rp) {
    if (hld == cols && dld == cols)
      check_hip(hipMemcpyAsync(dev, host, (size_t)rows * cols * es, hipMemcpyHostToDevice, stream),
                "hipMemcpyAsync H2D");
    else
      check_hip(hipMemcpy2DAsync(dev, dld * es, host, hld * es, cols * es, rows, hipMemcpyHostToDevice, stream),
                "hipMemcpy2DAsync H2D");
    return;
  }
  Ring& r = *rp;
  const size_t dpitch = (size_t)dld * es, hpitch = (size_t)hld * es, row_bytes = (size_t)cols * es;
  const int64_t chunk_rows = std::max<int64_t>(1, (int64_t)(kSlotBytes / dpitch));
  int s = 0;
  for (int64_t r0 = 0; r0 < rows; r0 += chunk_rows, s = (s + 1) % kSlots) {
    const int64_t n = std::min(chunk_rows, rows - r0);
    if (r.busy[s]) check_hip(hipEventSynchronize(r.ev[s]), "hipEventSynchronize");
    pool_copy_rows(r.slot[s], dpitch, static_cast<const char*>(host) + r0 * hpitch, hpitch, n, row_bytes);
    // Rows land with the device pitch; one flat DMA per chunk (the padding
    // columns carry whatever the slot held and are never read as data).
    check_hip(hipMemcpyAsync(static_cast<char*>(dev) + r0 * dpitch, r.slot[s], (size_t)n * dpitch,
                             hipMemcpyHostToDevice, stream),
              "hipMemcpyAsync H2D");
    check_hip(hipEventRecord(r.ev[s], stream), "hipEventRecord");
    r.busy[s] = true;
  }
}

void stage_d2h(void* host, int64_t hld, const void* dev, int64_t dld, int64_t rows, int64_t cols, size_t es,
               hipStream_t stream) {
  if (rows <= 0 || cols <= 0) return;
  Ring* rp = direct(rows, dld, es) ? nullptr : ring_for_current_device();
  if (!rp) {
    if (hld == cols && dld == cols)
      check_hip(hipMemcpyAsync(host, dev, (size_t)rows * cols * es, hipMemcpyDeviceToHost, stream),
                "hipMemcpyAsync D2H");
    else
      check_hip(hipMemcpy2DAsync(host, hld * es, dev, dld * es, cols * es, rows, hipMemcpyDeviceToHost, stream),
                "hipMemcpy2DAsync D2H");
    return;
  }
  Ring& r = *rp;
  const size_t dpitch = (size_t)dld * es, hpitch = (size_t)hld * es, row_bytes = (size_t)cols * es;
  const int64_t chunk_rows = std::max<int64_t>(1, (int64_t)(kSlotBytes / dpitch));
  const int64_t chunks = (rows + chunk_rows - 1) / chunk_rows;
  auto issue = [&](int64_t c) {
    const int s = (int)(c % kSlots);
    const int64_t r0 = c * chunk_rows, n = std::min(chunk_rows, rows - r0);
    // A slot still being read by an upload (possibly on another stream) is
    // overwritten only after that DMA; one this call already copied out is free.
    if (r.busy[s]) check_hip(hipStreamWaitEvent(stream, r.ev[s], 0), "hipStreamWaitEvent");
    check_hip(hipMemcpyAsync(r.slot[s], static_cast<const char*>(dev) + r0 * dpitch, (size_t)n * dpitch,
                             hipMemcpyDeviceToHost, stream),
              "hipMemcpyAsync D2H");
    check_hip(hipEventRecord(r.ev[s], stream), "hipEventRecord");
    r.busy[s] = true;
  };
  for (int64_t c = 0; c < std::min<int64_t>(chunks, kSlots); ++c) issue(c);
  for (int64_t c = 0; c < chunks; ++c) {
    const int s = (int)(c % kSlots);
    const int64_t r0 = c * chunk_rows, n = std::min(chunk_rows, rows - r0);
    check_hip(hipEventSynchronize(r.ev[s]), "hipEventSynchronize");
    r.busy[s] = false;
    pool_copy_rows(static_cast<char*>(host) + r0 * hpitch, hpitch, r.slot[s], dpitch, n, row_bytes);
    if (c + kSlots < chunks) issue(c + kSlots);
  }
}

}  // namespace rt
}  // namespace edsl
