// Host-side error state of libqattn: thread-local last-error string behind qattn_last_error().
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace qattn {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(QATTN_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return QATTN_OK;
}

}  // namespace qattn

extern "C" const char* qattn_last_error(void) { return qattn::g_last_error; }
extern "C" int qattn_version(void) { return 1; }
