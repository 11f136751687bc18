// Error plumbing and version of libccq_hip.
#include "ccq_common.h"

#include <string.h>

namespace ccq {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int arg_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return CCQ_EINVAL;
}

static thread_local LaunchTimer g_timer = {nullptr, nullptr};

LaunchTimer take_launch_timer() {
  const LaunchTimer t = g_timer;
  g_timer = LaunchTimer{nullptr, nullptr};
  return t;
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

}  // namespace ccq

extern "C" int ccq_version(void) { return 100; }

extern "C" const char* ccq_last_error(void) { return ccq::g_err; }

extern "C" int ccq_launch_timer(void* start_event, void* stop_event) {
  CCQ_REQUIRE((start_event == nullptr) == (stop_event == nullptr),
              "ccq_launch_timer: give both events or neither");
  ccq::g_timer = ccq::LaunchTimer{reinterpret_cast<hipEvent_t>(start_event), reinterpret_cast<hipEvent_t>(stop_event)};
  return 0;
}
