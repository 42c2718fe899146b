// Error reporting and launch accounting shared by every C-ABI entry point.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "grm_hip.h"
#include "grm_hip_common.h"

namespace grmhip {

namespace {
thread_local char g_last_error[512] = "";
std::atomic<uint64_t> g_launches{0};
}  // namespace

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void count_launch() { g_launches.fetch_add(1, std::memory_order_relaxed); }

// Called right after a kernel launch: records it and turns a launch error
// into a status code.  Does not synchronise.
int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return static_cast<int>(e);
  }
  count_launch();
  return GRM_HIP_OK;
}

}  // namespace grmhip

extern "C" int grm_hip_abi_version(void) { return 109; }

extern "C" const char* grm_hip_last_error(void) { return grmhip::g_last_error; }

extern "C" uint64_t grm_hip_launch_count(void) {
  return grmhip::g_launches.load(std::memory_order_relaxed);
}
