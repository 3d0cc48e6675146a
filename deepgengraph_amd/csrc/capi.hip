// Library-wide C ABI plumbing: ABI version, thread-local error message, launch-status check.
#include "common.h"

namespace dgg {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(DGG_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return DGG_OK;
}

}  // namespace dgg

extern "C" int dgg_abi_version(void) { return DGG_ABI_VERSION; }

extern "C" const char* dgg_last_error(void) { return dgg::g_err; }
