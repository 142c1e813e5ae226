// Error reporting and version query shared by the C entry points.
#include <stdarg.h>
#include <stdio.h>

#include "gs_common.h"

namespace gs {
namespace {
thread_local char g_err[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return GS_OK;
  set_error("%s: %s", what, hipGetErrorString(e));
  return GS_ERR_HIP;
}

int launch_check(const char* what) { return hip_check(hipGetLastError(), what); }

}  // namespace gs

extern "C" const char* gs_last_error(void) { return gs::g_err; }
extern "C" int gs_abi_version(void) { return 14; }
