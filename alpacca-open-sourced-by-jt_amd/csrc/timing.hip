// Kernel timing for measurement: while enabled, entry points bracket their
// kernels with HIP events recorded on the launch stream; totals are read
// back (after synchronising the recorded events) per kernel id.
#include <mutex>
#include <vector>

#include "alpx_common.h"
#include "timing.h"

namespace alpx {
namespace {

struct Pending {
  int kernel;
  hipEvent_t start, stop;
};

std::mutex g_mu;
bool g_enabled = false;
std::vector<Pending> g_pending;
std::vector<hipEvent_t> g_free;
double g_total_ms[ALPX_TIMING_KERNELS];
int64_t g_count[ALPX_TIMING_KERNELS];

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

void drain_locked() {
  for (const Pending& p : g_pending) {
    float ms = 0.f;
    if (hipEventSynchronize(p.stop) == hipSuccess &&
        hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
      g_total_ms[p.kernel] += ms;
      g_count[p.kernel] += 1;
    }
    g_free.push_back(p.start);
    g_free.push_back(p.stop);
  }
  g_pending.clear();
}

}  // namespace

TimedRegion::TimedRegion(int kernel, hipStream_t stream)
    : kernel_(kernel), stream_(stream), start_(nullptr), stop_(nullptr) {
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_enabled || kernel < 0 || kernel >= ALPX_TIMING_KERNELS) return;
  start_ = take_event();
  stop_ = take_event();
  if (start_ && stop_) (void)hipEventRecord(start_, stream_);
}

TimedRegion::~TimedRegion() { finish(); }

void TimedRegion::finish() {
  if (!start_ || !stop_) return;
  (void)hipEventRecord(stop_, stream_);
  std::lock_guard<std::mutex> lock(g_mu);
  g_pending.push_back({kernel_, start_, stop_});
  start_ = stop_ = nullptr;
}

}  // namespace alpx

extern "C" int alpx_timing_enable(int enable) {
  using namespace alpx;
  std::lock_guard<std::mutex> lock(g_mu);
  drain_locked();
  for (int i = 0; i < ALPX_TIMING_KERNELS; ++i) {
    g_total_ms[i] = 0.0;
    g_count[i] = 0;
  }
  g_enabled = enable != 0;
  return ALPX_OK;
}

extern "C" int alpx_timing_read(int kernel, double* total_ms, int64_t* launches) {
  using namespace alpx;
  if (kernel < 0 || kernel >= ALPX_TIMING_KERNELS || !total_ms || !launches)
    return fail(ALPX_EINVAL, "alpx_timing_read: bad kernel id or null output");
  std::lock_guard<std::mutex> lock(g_mu);
  drain_locked();
  *total_ms = g_total_ms[kernel];
  *launches = g_count[kernel];
  return ALPX_OK;
}
