// Optional per-kernel device timing with HIP events.
//
// When enabled (ts_timing_enable(1)), every kernel launch of the library is
// bracketed by a pair of events recorded on the launch stream; ts_timing_read
// sums the elapsed time of the recorded pairs per kernel name.  Disabled (the
// default), a launch costs one relaxed atomic load.
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"
#include "timing.h"
#include "../../include/thundersync_hip.h"

namespace ts {
namespace {

struct Pair {
  std::string name;
  hipEvent_t start, stop;
};

std::atomic<int> g_enabled{0};
std::mutex g_mu;
std::vector<Pair> g_pairs;
std::vector<hipEvent_t> g_free;

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

}  // namespace

TimedLaunch::TimedLaunch(const char* name, hipStream_t stream) : index_(-1), stream_(stream) {
  if (!g_enabled.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_mu);
  hipEvent_t a = take_event(), b = take_event();
  if (!a || !b) return;
  g_pairs.push_back(Pair{name, a, b});
  index_ = (int)g_pairs.size() - 1;
  (void)hipEventRecord(a, stream_);
}

TimedLaunch::~TimedLaunch() {
  if (index_ < 0) return;
  std::lock_guard<std::mutex> lock(g_mu);
  if (index_ < (int)g_pairs.size()) (void)hipEventRecord(g_pairs[index_].stop, stream_);
}

}  // namespace ts

extern "C" {

int ts_timing_enable(int enable) {
  ts::g_enabled.store(enable ? 1 : 0);
  return TS_OK;
}

int ts_timing_reset(void) {
  std::lock_guard<std::mutex> lock(ts::g_mu);
  for (auto& p : ts::g_pairs) {
    (void)hipEventSynchronize(p.stop);
    ts::g_free.push_back(p.start);
    ts::g_free.push_back(p.stop);
  }
  ts::g_pairs.clear();
  return TS_OK;
}

int ts_timing_read(const char* kernel, double* total_ms, int64_t* launches) {
  TS_CHECK_ARG(kernel && total_ms && launches, "ts_timing_read: null pointer");
  std::lock_guard<std::mutex> lock(ts::g_mu);
  double total = 0.0;
  int64_t n = 0;
  for (auto& p : ts::g_pairs) {
    if (p.name != kernel) continue;
    if (hipEventSynchronize(p.stop) != hipSuccess) {
      ts::set_error("ts_timing_read: event synchronize failed");
      return TS_ERR_LAUNCH;
    }
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
      total += ms;
      ++n;
    }
  }
  *total_ms = total;
  *launches = n;
  return TS_OK;
}

}  // extern "C"
