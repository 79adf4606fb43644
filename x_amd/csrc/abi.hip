// Error plumbing of the C-ABI: every entry point returns 0 on success or 1 with a message kept per host
// thread, returned by atl_last_error().
#include "common.h"
#include "../../include/atl_hip.h"

#include <cstdarg>
#include <cstring>

namespace atlhip {

namespace {
thread_local char g_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return 0;
  set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return 1;
}

}  // namespace atlhip

extern "C" {

const char* atl_last_error(void) { return atlhip::g_error; }

int atl_abi_version(void) { return ATL_HIP_ABI_VERSION; }

}  // extern "C"
