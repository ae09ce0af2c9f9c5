// RAII bracket of one kernel launch for the optional per-kernel timing.
#pragma once
#include <hip/hip_runtime.h>

namespace ts {

class TimedLaunch {
 public:
  TimedLaunch(const char* name, hipStream_t stream);
  ~TimedLaunch();
  TimedLaunch(const TimedLaunch&) = delete;
  TimedLaunch& operator=(const TimedLaunch&) = delete;

 private:
  int index_;
  hipStream_t stream_;
};

}  // namespace ts
