// Error state and version query for libmoc.
#include <stdarg.h>
#include <stdio.h>

#include "moc_common.h"

namespace moc {

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
  if (e != hipSuccess) return set_error(MOC_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return MOC_OK;
}

}  // namespace moc

extern "C" {

const char* moc_last_error(void) { return moc::g_last_error; }

int moc_abi_version(void) { return MOC_ABI_VERSION; }

}  // extern "C"
