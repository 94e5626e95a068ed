// Host data path of a stream executor on MI355X: host<->device copies with
// pinned staging, stream dependencies and host callbacks - what the
// reference's StreamExecutor plugin callbacks do
// (musa_ext/mu/musa_se_plugin.cc: pinned-bounce H2D :127-211, memcpy
// callbacks :599-760, create_stream_dependency :365-432, host_callback
// :808-835; staging pool musa_ext/mu/device/pinned_memory_pool.{h,cc}).
//
// Design:
//  * Staging pool per device: fixed 4 MiB pinned blocks (hipHostMalloc).  A
//    block used by an asynchronous copy returns to the free list only after
//    an event recorded behind the copy has completed; completed blocks are
//    reclaimed when the next block is requested (no polling thread).  At
//    most kMaxBlocks blocks exist per device; when all are in flight the
//    request waits for the oldest one.
//  * Pageable H2D runs in chunks: the host copy of chunk i+1 into a staging
//    block overlaps the DMA of chunk i, and each chunk's host copy is split
//    over a few worker threads.  The call returns once every chunk is
//    staged, so the caller may reuse the source at once - also for the
//    asynchronous copy (the reference falls back to a blocking copy there).
//  * Pinned sources and destinations copy directly; a device source turns
//    into a device-to-device copy (as the reference does).
//  * Synchronous D2H into pageable memory also runs in chunks: the DMA of
//    chunk i+1 overlaps the host copy out of chunk i.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <condition_variable>
#include <cstdlib>
#include <deque>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "tfma.h"
#include "tfma_internal.h"

namespace tfma {
namespace {

constexpr size_t kBlockBytes = size_t(4) << 20;
constexpr size_t kMaxBlocks = 32;                  // 128 MiB of staging per device
constexpr size_t kParallelMin = size_t(1) << 20;   // smaller copies stay on the caller

// ---------------------------------------------------------------------------
// Worker threads for the host side of a staged copy.
// ---------------------------------------------------------------------------
class CopyWorkers {
 public:
  static CopyWorkers& get() {
    static CopyWorkers* w = new CopyWorkers();  // never destroyed: workers may outlive main
    return *w;
  }
  // memcpy split into up to (workers + 1) slices; returns when all are done.
  void copy(void* dst, const void* src, size_t n) {
    const size_t parts = std::min<size_t>(threads_.size() + 1, std::max<size_t>(1, n / kParallelMin));
    if (parts <= 1) {
      memcpy(dst, src, n);
      return;
    }
    const size_t step = (n / parts + 63) & ~size_t(63);
    std::unique_lock<std::mutex> lk(mu_);
    pending_ = 0;
    for (size_t i = 1; i < parts; ++i) {
      const size_t off = i * step;
      if (off >= n) break;
      const size_t len = std::min(step, n - off);
      tasks_.push_back([=] {
        memcpy(static_cast<char*>(dst) + off, static_cast<const char*>(src) + off, len);
      });
      ++pending_;
    }
    cv_.notify_all();
    lk.unlock();
    memcpy(dst, src, std::min(step, n));
    lk.lock();
    done_.wait(lk, [&] { return pending_ == 0; });
  }

 private:
  CopyWorkers() {
    unsigned t = std::thread::hardware_concurrency();
    if (const char* e = getenv("TFMA_COPY_THREADS")) t = static_cast<unsigned>(atoi(e)) + 1;
    t = std::min(8u, std::max(1u, t / 2));
    for (unsigned i = 1; i < t; ++i) threads_.emplace_back([this] { run(); });
    for (auto& th : threads_) th.detach();
  }
  void run() {
    std::unique_lock<std::mutex> lk(mu_);
    while (true) {
      cv_.wait(lk, [&] { return !tasks_.empty(); });
      auto task = std::move(tasks_.front());
      tasks_.pop_front();
      lk.unlock();
      task();
      lk.lock();
      if (--pending_ == 0) done_.notify_all();
    }
  }
  std::mutex mu_;
  std::condition_variable cv_, done_;
  std::deque<std::function<void()>> tasks_;
  size_t pending_ = 0;
  std::vector<std::thread> threads_;
  std::mutex copy_mu_;

 public:
  std::mutex& serial() { return copy_mu_; }  // one staged copy uses the workers at a time
};

// ---------------------------------------------------------------------------
// Staging pool and event pool (per device).
// ---------------------------------------------------------------------------
struct Pending {
  void* block;  // nullptr for a stream-dependency event
  hipEvent_t ev;
};

struct DeviceHost {
  std::mutex mu;
  std::vector<void*> free_blocks;
  std::deque<Pending> pending;
  std::vector<hipEvent_t> spare_events;
  size_t blocks = 0;
  uint64_t host_allocs = 0;
  uint64_t reuses = 0;

  // Moves completed entries to the free lists (caller holds mu).
  void reap() {
    for (auto it = pending.begin(); it != pending.end();) {
      if (hipEventQuery(it->ev) == hipSuccess) {
        if (it->block) free_blocks.push_back(it->block);
        spare_events.push_back(it->ev);
        it = pending.erase(it);
      } else {
        ++it;
      }
    }
  }
  hipError_t take_event(hipEvent_t* ev) {  // caller holds mu
    if (!spare_events.empty()) {
      *ev = spare_events.back();
      spare_events.pop_back();
      return hipSuccess;
    }
    return hipEventCreateWithFlags(ev, hipEventDisableTiming);
  }
  hipError_t acquire(void** out) {
    std::unique_lock<std::mutex> lk(mu);
    reap();
    if (!free_blocks.empty()) {
      *out = free_blocks.back();
      free_blocks.pop_back();
      ++reuses;
      return hipSuccess;
    }
    if (blocks < kMaxBlocks) {
      hipError_t e = hipHostMalloc(out, kBlockBytes, hipHostMallocDefault);
      if (e != hipSuccess) return e;
      ++blocks;
      ++host_allocs;
      return hipSuccess;
    }
    // Every block is in flight: wait for the oldest staging block.
    for (auto it = pending.begin(); it != pending.end(); ++it) {
      if (!it->block) continue;
      const Pending p = *it;
      pending.erase(it);
      lk.unlock();
      const hipError_t e = hipEventSynchronize(p.ev);
      lk.lock();
      spare_events.push_back(p.ev);
      *out = p.block;
      ++reuses;
      return e;
    }
    return hipErrorOutOfMemory;  // blocks are all held by callers (not reachable here)
  }
  // Returns `block` once the work enqueued on `stream` so far has run.
  hipError_t release_after(void* block, hipStream_t stream) {
    std::lock_guard<std::mutex> lk(mu);
    hipEvent_t ev = nullptr;
    hipError_t e = take_event(&ev);
    if (e == hipSuccess) e = hipEventRecord(ev, stream);
    if (e != hipSuccess) {
      if (ev) spare_events.push_back(ev);
      free_blocks.push_back(block);  // unreachable by the copy: caller syncs on error
      return e;
    }
    pending.push_back({block, ev});
    return hipSuccess;
  }
  void release_now(void* block) {
    std::lock_guard<std::mutex> lk(mu);
    free_blocks.push_back(block);
  }
};

DeviceHost* device_host() {
  static DeviceHost hosts[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  return &hosts[dev];
}

enum class Mem { kPageable, kPinned, kDevice };

Mem classify(const void* p) {
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();  // pageable memory reports an error; clear it
    return Mem::kPageable;
  }
  switch (attr.type) {
    case hipMemoryTypeHost: return Mem::kPinned;
    case hipMemoryTypeDevice:
    case hipMemoryTypeManaged:
    case hipMemoryTypeArray: return Mem::kDevice;
    default: return Mem::kPageable;
  }
}

// Pageable -> device, staged.  Returns once the source has been read.
hipError_t staged_htod(DeviceHost* dh, void* dst, const void* src, size_t size,
                       hipStream_t stream) {
  CopyWorkers& w = CopyWorkers::get();
  std::lock_guard<std::mutex> serial(w.serial());
  for (size_t off = 0; off < size; off += kBlockBytes) {
    const size_t len = std::min(kBlockBytes, size - off);
    void* blk = nullptr;
    hipError_t e = dh->acquire(&blk);
    if (e != hipSuccess) return e;
    w.copy(blk, static_cast<const char*>(src) + off, len);
    e = hipMemcpyAsync(static_cast<char*>(dst) + off, blk, len, hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) {
      dh->release_now(blk);
      return e;
    }
    e = dh->release_after(blk, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Device -> pageable, staged and synchronous: DMA of chunk i+1 overlaps the
// host copy out of chunk i.
hipError_t staged_dtoh_sync(DeviceHost* dh, void* dst, const void* src, size_t size,
                            hipStream_t stream) {
  CopyWorkers& w = CopyWorkers::get();
  std::lock_guard<std::mutex> serial(w.serial());
  struct InFlight {
    void* blk;
    size_t off, len;
    hipEvent_t ev;
  };
  std::deque<InFlight> q;
  hipError_t err = hipSuccess;
  size_t off = 0;
  auto drain_one = [&]() {
    InFlight f = q.front();
    q.pop_front();
    hipError_t e = hipEventSynchronize(f.ev);
    if (e == hipSuccess) w.copy(static_cast<char*>(dst) + f.off, f.blk, f.len);
    if (err == hipSuccess) err = e;
    {
      std::lock_guard<std::mutex> lk(dh->mu);
      dh->spare_events.push_back(f.ev);
    }
    dh->release_now(f.blk);
  };
  while (off < size && err == hipSuccess) {
    const size_t len = std::min(kBlockBytes, size - off);
    void* blk = nullptr;
    hipError_t e = dh->acquire(&blk);
    hipEvent_t ev = nullptr;
    if (e == hipSuccess) {
      std::lock_guard<std::mutex> lk(dh->mu);
      e = dh->take_event(&ev);
    }
    if (e == hipSuccess)
      e = hipMemcpyAsync(blk, static_cast<const char*>(src) + off, len, hipMemcpyDeviceToHost,
                         stream);
    if (e == hipSuccess) e = hipEventRecord(ev, stream);
    if (e != hipSuccess) {
      if (blk) dh->release_now(blk);
      if (ev) {
        std::lock_guard<std::mutex> lk(dh->mu);
        dh->spare_events.push_back(ev);
      }
      err = e;
      break;
    }
    q.push_back({blk, off, len, ev});
    off += len;
    if (q.size() >= 2) drain_one();  // keep one DMA in flight ahead of the host copy
  }
  while (!q.empty()) drain_one();
  return err;
}

int set(TFMA_Status* st, int code, const char* msg) {
  if (st) {
    st->code = code;
    snprintf(st->message, sizeof(st->message), "%s", msg);
  }
  return code;
}

int hip_fail(TFMA_Status* st, hipError_t e, const char* what) {
  if (st) {
    st->code = TFMA_INTERNAL;
    snprintf(st->message, sizeof(st->message), "%s: %s", what, hipGetErrorString(e));
  }
  return TFMA_INTERNAL;
}

}  // namespace
}  // namespace tfma

extern "C" {

int TFMA_MemcpyHtoD(void* stream, void* device_dst, const void* host_src, uint64_t size,
                    int32_t sync, TFMA_Status* status) {
  using namespace tfma;
  if (size == 0) return set(status, TFMA_OK, "");
  if (!device_dst) return set(status, TFMA_INVALID_ARGUMENT, "null device pointer for dst in memcpy_htod");
  if (!host_src) return set(status, TFMA_INVALID_ARGUMENT, "null host pointer for src in memcpy_htod");
  DeviceHost* dh = device_host();
  if (!dh) return set(status, TFMA_INTERNAL, "memcpy_htod: no current device");
  hipStream_t s = sync ? nullptr : static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (classify(host_src)) {
    case Mem::kDevice:
      e = hipMemcpyAsync(device_dst, host_src, size, hipMemcpyDeviceToDevice, s);
      break;
    case Mem::kPinned:
      e = hipMemcpyAsync(device_dst, host_src, size, hipMemcpyHostToDevice, s);
      break;
    default:
      e = staged_htod(dh, device_dst, host_src, size, s);
      break;
  }
  if (e == hipSuccess && sync) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(status, e, sync ? "sync_memcpy_htod" : "memcpy_htod");
  return set(status, TFMA_OK, "");
}

int TFMA_MemcpyDtoH(void* stream, void* host_dst, const void* device_src, uint64_t size,
                    int32_t sync, TFMA_Status* status) {
  using namespace tfma;
  if (size == 0) return set(status, TFMA_OK, "");
  if (!host_dst) return set(status, TFMA_INVALID_ARGUMENT, "null host pointer for dst in memcpy_dtoh");
  if (!device_src) return set(status, TFMA_INVALID_ARGUMENT, "null device pointer for src in memcpy_dtoh");
  DeviceHost* dh = device_host();
  if (!dh) return set(status, TFMA_INTERNAL, "memcpy_dtoh: no current device");
  hipStream_t s = sync ? nullptr : static_cast<hipStream_t>(stream);
  hipError_t e;
  if (sync && classify(host_dst) == Mem::kPageable) {
    e = staged_dtoh_sync(dh, host_dst, device_src, size, s);
  } else {
    e = hipMemcpyAsync(host_dst, device_src, size, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess && sync) e = hipStreamSynchronize(s);
  }
  if (e != hipSuccess) return hip_fail(status, e, sync ? "sync_memcpy_dtoh" : "memcpy_dtoh");
  return set(status, TFMA_OK, "");
}

int TFMA_CreateStreamDependency(void* dependent, void* other, TFMA_Status* status) {
  using namespace tfma;
  if (!dependent || !other)
    return set(status, TFMA_INVALID_ARGUMENT, "null stream in create_stream_dependency");
  DeviceHost* dh = device_host();
  if (!dh) return set(status, TFMA_INTERNAL, "create_stream_dependency: no current device");
  std::lock_guard<std::mutex> lk(dh->mu);
  dh->reap();
  hipEvent_t ev = nullptr;
  hipError_t e = dh->take_event(&ev);
  if (e == hipSuccess) e = hipEventRecord(ev, static_cast<hipStream_t>(other));
  if (e == hipSuccess) e = hipStreamWaitEvent(static_cast<hipStream_t>(dependent), ev, 0);
  if (e != hipSuccess) {
    if (ev) dh->spare_events.push_back(ev);
    return hip_fail(status, e, "create_stream_dependency");
  }
  dh->pending.push_back({nullptr, ev});  // reused once the recorded work has run
  return set(status, TFMA_OK, "");
}

int TFMA_HostCallback(void* stream, void (*fn)(void*), void* arg, TFMA_Status* status) {
  using namespace tfma;
  if (!stream || !fn) return set(status, TFMA_INVALID_ARGUMENT, "null stream or callback in host_callback");
  const hipError_t e = hipLaunchHostFunc(static_cast<hipStream_t>(stream), fn, arg);
  if (e != hipSuccess) return hip_fail(status, e, "host_callback");
  return set(status, TFMA_OK, "");
}

int TFMA_StagingPoolStats(uint64_t* blocks, uint64_t* host_allocs, uint64_t* reuses,
                          uint64_t* pending, TFMA_Status* status) {
  using namespace tfma;
  DeviceHost* dh = device_host();
  if (!dh) return set(status, TFMA_INTERNAL, "staging pool: no current device");
  std::lock_guard<std::mutex> lk(dh->mu);
  dh->reap();
  if (blocks) *blocks = dh->blocks;
  if (host_allocs) *host_allocs = dh->host_allocs;
  if (reuses) *reuses = dh->reuses;
  if (pending) *pending = dh->pending.size();
  return set(status, TFMA_OK, "");
}

}  // extern "C"
