// Optional per-kernel timing with HIP events.
//
// While enabled (tgx_profile_begin .. tgx_profile_end), every kernel launch
// wrapped in TGX_PROFILE records a start and a stop event on its own stream;
// tgx_profile_end synchronises those events and accumulates elapsed time per
// kernel name.  Disabled, a scope costs one relaxed atomic load.
#include <hip/hip_runtime.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "tgx.h"
#include "tgx_profile.h"

namespace tgx {
namespace {

struct Pending {
  const char* name;
  hipEvent_t start, stop;
};

struct Totals {
  int64_t launches = 0;
  double ms = 0.0;
};

constexpr size_t kEventReserve = 2048;   // start + stop of 1024 launches

std::atomic<bool> g_enabled{false};
std::mutex g_mu;
std::vector<Pending> g_pending;
std::vector<hipEvent_t> g_pool;
std::map<std::string, Totals> g_totals;

hipEvent_t take_event() {
  if (!g_pool.empty()) {
    hipEvent_t e = g_pool.back();
    g_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

}  // namespace

ProfScope::ProfScope(const char* name, hipStream_t s) : name_(name), stream_(s) {
  if (!g_enabled.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_mu);
  start_ = take_event();
  if (start_) hipEventRecord(start_, s);
}

ProfScope::~ProfScope() {
  if (!start_) return;
  std::lock_guard<std::mutex> lock(g_mu);
  hipEvent_t stop = take_event();
  if (!stop) return;
  hipEventRecord(stop, stream_);
  g_pending.push_back(Pending{name_, start_, stop});
}

}  // namespace tgx

using namespace tgx;

extern "C" int tgx_profile_begin(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  g_totals.clear();
  // Events are created here, not at the first launches of the profiled
  // region: hipEventCreate inside a timed loop would add its cost to every
  // launch it times.
  while (g_pool.size() < kEventReserve) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) break;
    g_pool.push_back(e);
  }
  g_enabled.store(true);
  return TGX_OK;
}

extern "C" int tgx_profile_end(void) {
  g_enabled.store(false);
  std::lock_guard<std::mutex> lock(g_mu);
  for (const Pending& p : g_pending) {
    float ms = 0.f;
    if (hipEventSynchronize(p.stop) == hipSuccess &&
        hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
      Totals& t = g_totals[p.name];
      t.launches += 1;
      t.ms += ms;
    }
    g_pool.push_back(p.start);
    g_pool.push_back(p.stop);
  }
  g_pending.clear();
  return TGX_OK;
}

extern "C" int tgx_profile_count(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  return static_cast<int>(g_totals.size());
}

extern "C" int tgx_profile_entry(int index, char* name, int name_capacity, int64_t* launches,
                                 double* total_ms) {
  std::lock_guard<std::mutex> lock(g_mu);
  if (index < 0 || index >= static_cast<int>(g_totals.size()) || !name || name_capacity <= 0 ||
      !launches || !total_ms)
    return TGX_INVALID_ARGUMENT;
  auto it = g_totals.begin();
  std::advance(it, index);
  snprintf(name, name_capacity, "%s", it->first.c_str());
  *launches = it->second.launches;
  *total_ms = it->second.ms;
  return TGX_OK;
}
