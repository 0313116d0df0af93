// Error state and version of the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "common.hpp"

namespace {
thread_local char g_error[512] = "";
}

void mko_set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
}

int mko_check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    mko_set_error("%s: launch failed: %s", what, hipGetErrorString(err));
    return MKO_ELAUNCH;
  }
  return MKO_OK;
}

extern "C" int mko_abi_version(void) { return MKO_ABI_VERSION; }

extern "C" const char* mko_last_error(void) { return g_error; }

extern "C" size_t mko_sizeof_selscan_params(void) { return sizeof(mko_selscan_params); }

extern "C" size_t mko_sizeof_state_update_params(void) { return sizeof(mko_state_update_params); }

extern "C" size_t mko_sizeof_ssd_params(void) { return sizeof(mko_ssd_params); }

// ---------------------------------------------------------------- kernel timing
//
// Opt-in per-kernel timing with HIP events recorded on the launch stream around
// each kernel.  Events come from a pool and are never destroyed while the
// process runs; enabling it costs two event records per launch.

namespace {

struct Pending {
  int slot;
  hipEvent_t start, stop;
};

struct Slot {
  std::string name;
  double total_ms = 0.0;
  int64_t count = 0;
};

std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<Slot> g_slots;
std::vector<Pending> g_pending;
std::vector<hipEvent_t> g_event_pool;

hipEvent_t take_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

int slot_of(const char* name) {
  for (size_t i = 0; i < g_slots.size(); ++i)
    if (g_slots[i].name == name) return static_cast<int>(i);
  g_slots.push_back(Slot{name});
  return static_cast<int>(g_slots.size() - 1);
}

void resolve_locked() {
  for (const Pending& p : g_pending) {
    float ms = 0.0f;
    if (hipEventSynchronize(p.stop) == hipSuccess && hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
      g_slots[p.slot].total_ms += ms;
      g_slots[p.slot].count += 1;
    }
    g_event_pool.push_back(p.start);
    g_event_pool.push_back(p.stop);
  }
  g_pending.clear();
}

}  // namespace

mko::ProfScope::ProfScope(const char* name, hipStream_t stream) : stream_(stream) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  if (!g_prof_on) return;
  start_ = take_event();
  stop_ = take_event();
  if (!start_ || !stop_) return;
  slot_ = slot_of(name);
  hipEventRecord(start_, stream_);
}

mko::ProfScope::~ProfScope() {
  if (slot_ < 0) return;
  std::lock_guard<std::mutex> lock(g_prof_mu);
  hipEventRecord(stop_, stream_);
  g_pending.push_back(Pending{slot_, start_, stop_});
}

extern "C" int mko_profile_enable(int on) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  const int was = g_prof_on ? 1 : 0;
  g_prof_on = on != 0;
  return was;
}

extern "C" void mko_profile_reset(void) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  resolve_locked();
  g_slots.clear();
}

extern "C" int mko_profile_count(void) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  resolve_locked();
  return static_cast<int>(g_slots.size());
}

extern "C" int mko_profile_entry(int index, char* name, size_t name_len, double* total_ms, int64_t* launches) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  resolve_locked();
  if (index < 0 || index >= static_cast<int>(g_slots.size())) return MKO_EINVAL;
  const Slot& s = g_slots[index];
  if (name && name_len) {
    strncpy(name, s.name.c_str(), name_len - 1);
    name[name_len - 1] = '\0';
  }
  if (total_ms) *total_ms = s.total_ms;
  if (launches) *launches = s.count;
  return MKO_OK;
}
