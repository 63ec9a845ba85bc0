// ABI plumbing: version, thread-local error message.
#include <stdarg.h>
#include <stdio.h>

#include "gdn_common.h"

namespace gdn {

static thread_local char g_err[512];

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return GDN_OK;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

}  // namespace gdn

extern "C" int gdn_abi_version(void) { return GDN_ABI_VERSION; }

extern "C" const char *gdn_last_error_string(void) { return gdn::g_err; }
