// Status plumbing of the C ABI: per-thread last-error message.
#include <cstdarg>
#include <cstdio>

#include "qs_common.h"

namespace qs {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

int hip_status(hipError_t e, const char* what) {
  set_error("%s: %s (hip error %d)", what, hipGetErrorString(e), (int)e);
  return QS_ERR_HIP;
}

}  // namespace qs

extern "C" const char* qs_last_error(void) { return qs::g_err; }
extern "C" int qs_abi_version(void) { return QS_ABI_VERSION; }
