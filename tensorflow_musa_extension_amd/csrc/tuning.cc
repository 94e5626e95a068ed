// Plan and cache-mode overrides for tests and measurements
// (TFMA_SetTuningOverride).  Each override is one relaxed atomic int, so the
// launch paths read it without a lock, a libc call or a race with setenv in
// another thread.  Its starting value comes from the environment variable of
// the same name (TFMA_ + the name in upper case), read once, at the first
// query of any override.
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "tfma_internal.h"

namespace tfma {
namespace {

struct Override {
  const char* name;
  const char* env;
};
constexpr Override kOverrides[kTuneCount] = {
    {"ew_nt", "TFMA_EW_NT"},
    {"bn_slice_tw", "TFMA_BN_SLICE_TW"},
    {"bn_sliced_overlap", "TFMA_BN_SLICED_OVERLAP"},
    {"bn_nchw_owned", "TFMA_BN_NCHW_OWNED"},
    {"bag_fused", "TFMA_BAG_FUSED"},
};

std::atomic<int> g_value[kTuneCount];
std::once_flag g_env_once;

void read_env() {
  for (int k = 0; k < kTuneCount; ++k) {
    const char* e = getenv(kOverrides[k].env);
    g_value[k].store(e && e[0] ? atoi(e) : -1, std::memory_order_relaxed);
  }
}

}  // namespace

int TuneValue(Tune k) {
  std::call_once(g_env_once, read_env);
  return g_value[k].load(std::memory_order_relaxed);
}

bool SetTune(const char* name, int value) {
  std::call_once(g_env_once, read_env);
  for (int k = 0; k < kTuneCount; ++k) {
    if (strcmp(kOverrides[k].name, name) == 0) {
      g_value[k].store(value, std::memory_order_relaxed);
      return true;
    }
  }
  return false;
}

}  // namespace tfma
