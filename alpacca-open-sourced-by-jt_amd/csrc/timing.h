// HIP-event bracket around a kernel launch (active only while timing is on).
#pragma once
#include <hip/hip_runtime.h>

namespace alpx {

class TimedRegion {
 public:
  TimedRegion(int kernel, hipStream_t stream);
  ~TimedRegion();
  void finish();  // record the stop event now (before later launches)

 private:
  int kernel_;
  hipStream_t stream_;
  hipEvent_t start_, stop_;
};

}  // namespace alpx
