// Library-level entry points: error string, version, arch.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "qa_common.h"

namespace qa {

static thread_local std::string g_last_error;

static void vset(const char* fmt, va_list ap) {
  char buf[1024];
  vsnprintf(buf, sizeof(buf), fmt, ap);
  g_last_error = buf;
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vset(fmt, ap);
  va_end(ap);
}

int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vset(fmt, ap);
  va_end(ap);
  return 1;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail("%s: launch failed: %s", what, hipGetErrorString(err));
  return 0;
}

// ---- kernel timing -----------------------------------------------------------
namespace {
struct PendingTiming {
  hipEvent_t start;
  hipEvent_t stop;
  std::string label;
};
std::mutex g_timing_mu;
bool g_timing_on = false;
std::vector<PendingTiming> g_pending;
std::vector<hipEvent_t> g_free_events;
std::map<std::string, std::pair<double, int64_t>> g_totals;

hipEvent_t take_event() {
  if (!g_free_events.empty()) {
    hipEvent_t e = g_free_events.back();
    g_free_events.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Resolve every recorded pair (waits for them) into the per-label totals.
void drain_pending() {
  for (PendingTiming& t : g_pending) {
    float ms = 0.f;
    if (hipEventSynchronize(t.stop) == hipSuccess && hipEventElapsedTime(&ms, t.start, t.stop) == hipSuccess) {
      auto& tot = g_totals[t.label];
      tot.first += ms;
      tot.second += 1;
    }
    g_free_events.push_back(t.start);
    g_free_events.push_back(t.stop);
  }
  g_pending.clear();
}
}  // namespace

KernelTimer::KernelTimer(const char* label, hipStream_t stream) : label_(label), stream_(stream) {
  std::lock_guard<std::mutex> lock(g_timing_mu);
  if (!g_timing_on) return;
  start_ = take_event();
  if (start_ != nullptr && hipEventRecord(start_, stream_) != hipSuccess) {
    g_free_events.push_back(start_);
    start_ = nullptr;
  }
}

KernelTimer::~KernelTimer() {
  if (start_ == nullptr) return;
  std::lock_guard<std::mutex> lock(g_timing_mu);
  hipEvent_t stop = take_event();
  if (stop == nullptr || hipEventRecord(stop, stream_) != hipSuccess) {
    g_free_events.push_back(start_);
    if (stop != nullptr) g_free_events.push_back(stop);
    return;
  }
  g_pending.push_back({start_, stop, label_});
}

}  // namespace qa

extern "C" void qa_set_kernel_timing(int32_t enabled) {
  std::lock_guard<std::mutex> lock(qa::g_timing_mu);
  qa::drain_pending();
  qa::g_totals.clear();
  qa::g_timing_on = enabled != 0;
}

extern "C" int qa_read_kernel_timing(const char* label, double* total_ms, int64_t* launches) {
  std::lock_guard<std::mutex> lock(qa::g_timing_mu);
  qa::drain_pending();
  auto it = qa::g_totals.find(label != nullptr ? label : "");
  if (total_ms != nullptr) *total_ms = it == qa::g_totals.end() ? 0.0 : it->second.first;
  if (launches != nullptr) *launches = it == qa::g_totals.end() ? 0 : it->second.second;
  return 0;
}

extern "C" const char* qa_last_error(void) { return qa::g_last_error.c_str(); }

extern "C" int32_t qa_version(void) { return 1; }

extern "C" const char* qa_arch(void) { return "gfx950"; }
