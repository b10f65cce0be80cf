// Per-kernel launch timing with hipEvents (instrumentation behind
// cqgdn_timer_arm / cqgdn_timer_read).  When one kernel is armed, every launch
// of it is bracketed by two hipEventRecord calls on the stream it is launched
// on, so the measured span is that kernel's own execution on that stream.
// Unarmed, a launch pays one relaxed atomic load.
#pragma once
#include <hip/hip_runtime.h>

namespace cqgdn {

enum KernelId {
  K_FWD_PREP,
  K_FWD_SCAN,
  K_FWD_OUT,
  K_BWD_LOCAL,
  K_BWD_SCAN,
  K_BWD_DKW,
  K_RECURRENT,
  K_COUNT
};

// the C ABI's error state (capi.hip): fail() records a message for
// cqgdn_last_error and returns code; ok() clears it and returns CQGDN_OK
int fail(int code, const char* fmt, ...);
int ok();

// names accepted by cqgdn_timer_arm, indexed by KernelId
extern const char* const kKernelNames[K_COUNT];

void timer_mark(int id, bool end, hipStream_t stream);

// RAII bracket around one launch
struct TimedLaunch {
  int id;
  hipStream_t stream;
  TimedLaunch(int id_, hipStream_t s) : id(id_), stream(s) { timer_mark(id, false, stream); }
  ~TimedLaunch() { timer_mark(id, true, stream); }
};

}  // namespace cqgdn
