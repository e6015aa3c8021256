// Per-kernel launch timing for measurement harnesses.
//
// When enabled (dil_timing_enable(1)), every kernel launch made by the entry
// points is bracketed by a pair of hipEvents recorded on the launch stream.
// dil_timing_read() waits for the recorded events and reports, per kernel
// name, the number of launches and the summed event-to-event time.  Disabled
// (the default), a LaunchTimer costs one relaxed atomic load.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "dil_internal.hpp"

namespace dil {

namespace {

struct Pending {
  const char* name;
  hipEvent_t start, stop;
};

struct Total {
  std::string name;
  double ms = 0.0;
  int64_t count = 0;
};

std::atomic<int> g_enabled{0};
std::mutex g_mu;
std::vector<Pending> g_pending;
std::vector<Total> g_totals;
std::vector<hipEvent_t> g_free;   // recycled events

hipEvent_t take_event() {
  if (!g_free.empty()) {
    hipEvent_t e = g_free.back();
    g_free.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Fold finished records into the totals.  Caller holds g_mu.
int drain_locked() {
  int status = 0;
  for (const Pending& p : g_pending) {
    float ms = 0.f;
    hipError_t e = hipEventSynchronize(p.stop);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, p.start, p.stop);
    if (e != hipSuccess) {
      status = static_cast<int>(e);
    } else {
      Total* t = nullptr;
      for (Total& x : g_totals)
        if (x.name == p.name) t = &x;
      if (t == nullptr) {
        g_totals.push_back(Total{p.name, 0.0, 0});
        t = &g_totals.back();
      }
      t->ms += ms;
      t->count += 1;
    }
    g_free.push_back(p.start);
    g_free.push_back(p.stop);
  }
  g_pending.clear();
  return status;
}

}  // namespace

LaunchTimer::LaunchTimer(const char* name, void* stream) : name_(name), stream_(stream) {
  if (g_enabled.load(std::memory_order_relaxed) == 0) return;
  std::lock_guard<std::mutex> lock(g_mu);
  start_ = take_event();
  stop_ = take_event();
  if (start_ == nullptr || stop_ == nullptr) return;
  if (hipEventRecord(static_cast<hipEvent_t>(start_), static_cast<hipStream_t>(stream_)) != hipSuccess)
    start_ = nullptr;
}

LaunchTimer::~LaunchTimer() {
  if (start_ == nullptr || stop_ == nullptr) return;
  std::lock_guard<std::mutex> lock(g_mu);
  if (hipEventRecord(static_cast<hipEvent_t>(stop_), static_cast<hipStream_t>(stream_)) != hipSuccess)
    return;
  g_pending.push_back(Pending{name_, static_cast<hipEvent_t>(start_), static_cast<hipEvent_t>(stop_)});
}

}  // namespace dil

extern "C" {

int dil_timing_enable(int on) {
  dil::g_enabled.store(on ? 1 : 0);
  return 0;
}

int dil_timing_reset(void) {
  std::lock_guard<std::mutex> lock(dil::g_mu);
  const int status = dil::drain_locked();
  dil::g_totals.clear();
  return status;
}

int dil_timing_count(void) {
  std::lock_guard<std::mutex> lock(dil::g_mu);
  dil::drain_locked();
  return static_cast<int>(dil::g_totals.size());
}

int dil_timing_read(int index, char* name, int name_capacity, double* total_ms, int64_t* launches) {
  std::lock_guard<std::mutex> lock(dil::g_mu);
  const int status = dil::drain_locked();
  if (status != 0) return status;
  if (index < 0 || index >= static_cast<int>(dil::g_totals.size())) return dil::kErrShape;
  const dil::Total& t = dil::g_totals[static_cast<size_t>(index)];
  if (name != nullptr && name_capacity > 0) {
    std::strncpy(name, t.name.c_str(), static_cast<size_t>(name_capacity) - 1);
    name[name_capacity - 1] = '\0';
  }
  if (total_ms != nullptr) *total_ms = t.ms;
  if (launches != nullptr) *launches = t.count;
  return 0;
}

}  // extern "C"
