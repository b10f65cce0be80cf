// Kernel launch timer: cqgdn_timer_arm / cqgdn_timer_read (include/cqgdn.h).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <mutex>
#include <vector>

#include "cqgdn.h"
#include "gdn_timer.hpp"

namespace cqgdn {

const char* const kKernelNames[K_COUNT] = {"fwd_prep",  "fwd_scan", "fwd_out", "bwd_local",
                                           "bwd_scan",  "bwd_dkw",  "recurrent"};

namespace {

struct Timer {
  std::mutex mu;
  std::atomic<int> armed{-1};
  std::vector<hipEvent_t> events;  // [start, stop] per launch
  int capacity = 0;                // launches the events can hold
  int used = 0;                    // launches recorded
  bool open = false;               // a start was recorded without its stop
  hipError_t error = hipSuccess;   // first failure while recording
};

Timer& timer() {
  static Timer t;
  return t;
}

void release(Timer& t) {
  for (hipEvent_t e : t.events) (void)hipEventDestroy(e);
  t.events.clear();
  t.capacity = t.used = 0;
  t.open = false;
  t.error = hipSuccess;
}

}  // namespace

void timer_mark(int id, bool end, hipStream_t stream) {
  Timer& t = timer();
  if (t.armed.load(std::memory_order_relaxed) != id) return;
  std::lock_guard<std::mutex> lock(t.mu);
  if (t.armed.load(std::memory_order_relaxed) != id) return;
  if (!end) {
    if (t.used >= t.capacity) return;
    const hipError_t e = hipEventRecord(t.events[2 * t.used], stream);
    if (e != hipSuccess && t.error == hipSuccess) t.error = e;
    t.open = (e == hipSuccess);
  } else if (t.open) {
    const hipError_t e = hipEventRecord(t.events[2 * t.used + 1], stream);
    if (e != hipSuccess && t.error == hipSuccess) t.error = e;
    if (e == hipSuccess) ++t.used;
    t.open = false;
  }
}

}  // namespace cqgdn

using namespace cqgdn;

extern "C" {

int cqgdn_timer_arm(const char* kernel, int max_launches) {
  Timer& t = timer();
  std::lock_guard<std::mutex> lock(t.mu);
  t.armed.store(-1);
  release(t);
  if (!kernel) return ok();  // disarm
  int id = -1;
  for (int i = 0; i < K_COUNT; ++i)
    if (std::strcmp(kernel, kKernelNames[i]) == 0) id = i;
  if (id < 0) return fail(CQGDN_EINVAL, "cqgdn_timer_arm: unknown kernel '%.64s'", kernel);
  if (max_launches <= 0 || max_launches > (1 << 16))
    return fail(CQGDN_EINVAL, "cqgdn_timer_arm: max_launches %d not in 1..65536", max_launches);
  t.events.resize(2 * (size_t)max_launches);
  for (size_t i = 0; i < t.events.size(); ++i) {
    // timing events without the system-scope fence: they bracket one kernel on
    // one device, and the fence's cache write-back would lengthen the gap they
    // measure across (on a side stream, right at the kernel's launch)
    if (hipEventCreateWithFlags(&t.events[i], hipEventDisableSystemFence) != hipSuccess) {
      t.events.resize(i);
      release(t);
      return fail(CQGDN_EHIP, "cqgdn_timer_arm: hipEventCreateWithFlags failed");
    }
  }
  t.capacity = max_launches;
  t.armed.store(id);
  return ok();
}

int cqgdn_timer_read(float* launch_ms, int capacity, int* launches) {
  Timer& t = timer();
  std::lock_guard<std::mutex> lock(t.mu);
  t.armed.store(-1);
  int rc = (t.error == hipSuccess) ? CQGDN_OK : CQGDN_EHIP;
  const int n = t.used;
  for (int i = 0; i < n && rc == CQGDN_OK; ++i) {
    float ms = 0.f;
    if (hipEventSynchronize(t.events[2 * i + 1]) != hipSuccess ||
        hipEventElapsedTime(&ms, t.events[2 * i], t.events[2 * i + 1]) != hipSuccess) {
      rc = CQGDN_EHIP;
      break;
    }
    if (launch_ms && i < capacity) launch_ms[i] = ms;
  }
  if (launches) *launches = (rc == CQGDN_OK) ? n : 0;
  release(t);
  return rc == CQGDN_OK ? ok() : fail(rc, "cqgdn_timer_read: a timed launch or its events failed");
}

}  // extern "C"
