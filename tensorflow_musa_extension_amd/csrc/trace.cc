// Kernel launch tracing: HIP events attached, as its start and end, to the
// dispatch of every launch whose kernel name contains a chosen substring
// (TFMA_LAUNCH and the fused BN launcher take them from TraceTake).  Used by
// the benchmark to time kernels inside a timed region on the stream they
// run on.
#include <hip/hip_runtime.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "tfma_internal.h"

namespace tfma {
namespace {

struct Pending {
  hipEvent_t start;
  hipEvent_t end;
};

struct TraceState {
  std::mutex mu;
  std::atomic<bool> enabled{false};  // read without the mutex on every launch
  std::string substr;
  std::vector<Pending> pending;
  std::vector<hipEvent_t> pool;
  double total_ms = 0.0;
  int64_t launches = 0;
};

TraceState& state() {
  static TraceState* s = new TraceState();
  return *s;
}

thread_local const char* t_last_kernel = "";

hipEvent_t take_event(TraceState& s) {
  if (!s.pool.empty()) {
    hipEvent_t e = s.pool.back();
    s.pool.pop_back();
    return e;
  }
  // Device-scope release: a default event would also write the caches back
  // for the host (system scope), which costs microseconds between kernels.
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventReleaseToDevice) != hipSuccess) return nullptr;
  return e;
}

// Folds completed pending pairs into the totals (caller holds the mutex).
void drain(TraceState& s) {
  for (auto& p : s.pending) {
    float ms = 0.f;
    if (hipEventSynchronize(p.end) == hipSuccess &&
        hipEventElapsedTime(&ms, p.start, p.end) == hipSuccess) {
      s.total_ms += ms;
      s.launches += 1;
    }
    s.pool.push_back(p.start);
    s.pool.push_back(p.end);
  }
  s.pending.clear();
}

}  // namespace

void SetLastKernel(const char* kernel_name) { t_last_kernel = kernel_name; }

TraceEvents TraceTake(const char* kernel_name) {
  TraceEvents ev;
  TraceState& s = state();
  if (!s.enabled.load(std::memory_order_relaxed)) return ev;
  std::lock_guard<std::mutex> lk(s.mu);
  if (!s.enabled || strstr(kernel_name, s.substr.c_str()) == nullptr) return ev;
  ev.start = take_event(s);
  ev.end = take_event(s);
  if (!ev.start || !ev.end) {
    if (ev.start) s.pool.push_back(ev.start);
    if (ev.end) s.pool.push_back(ev.end);
    ev = TraceEvents();
  }
  return ev;
}

void TraceCommit(const TraceEvents& ev) {
  if (!ev.start) return;
  TraceState& s = state();
  std::lock_guard<std::mutex> lk(s.mu);
  s.pending.push_back(Pending{ev.start, ev.end});
  if (s.pending.size() > 4096) drain(s);
}


}  // namespace tfma

extern "C" {

int TFMA_TraceEnable(const char* name_substr, TFMA_Status* status) {
  tfma::TraceState& s = tfma::state();
  std::lock_guard<std::mutex> lk(s.mu);
  tfma::drain(s);
  s.total_ms = 0.0;
  s.launches = 0;
  s.enabled = name_substr != nullptr;
  s.substr = name_substr ? name_substr : "";
  if (status) {
    status->code = TFMA_OK;
    status->message[0] = '\0';
  }
  return TFMA_OK;
}

int TFMA_TraceRead(double* total_ms, int64_t* launches, TFMA_Status* status) {
  tfma::TraceState& s = tfma::state();
  std::lock_guard<std::mutex> lk(s.mu);
  tfma::drain(s);
  if (total_ms) *total_ms = s.total_ms;
  if (launches) *launches = s.launches;
  if (status) {
    status->code = TFMA_OK;
    status->message[0] = '\0';
  }
  return TFMA_OK;
}

const char* TFMA_LastKernelName(void) { return tfma::t_last_kernel; }

}  // extern "C"
