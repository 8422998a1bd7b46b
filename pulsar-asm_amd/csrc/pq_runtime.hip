// pq_runtime.hip -- error state and version of the C ABI.
#include <string.h>

#include "pq_host.h"

namespace pq {

static thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

TimedLaunch &timed_launch() {
  static thread_local TimedLaunch t;
  return t;
}

}  // namespace pq

extern "C" const char *pq_version(void) { return "pulsar-amd 0.1 gfx950"; }

extern "C" const char *pq_last_error(void) { return pq::g_err; }

extern "C" int pq_time_next_launch(void *start_event, void *stop_event) {
  PQ_REQUIRE((start_event == nullptr) == (stop_event == nullptr), PQ_ERR_ARG,
             "pq_time_next_launch: pass both events or neither");
  pq::TimedLaunch &t = pq::timed_launch();
  t.start = reinterpret_cast<hipEvent_t>(start_event);
  t.stop = reinterpret_cast<hipEvent_t>(stop_event);
  return PQ_OK;
}
