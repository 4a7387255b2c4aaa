// Error reporting and version entry points of libgeoweave_hip.so.
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "gw_common.h"

namespace gw {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error.assign(buf);
  return code;
}

void clear_error() { g_last_error.clear(); }

int hip_error(hipError_t err, const char* what) {
  return set_error(GW_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(err), (int)err);
}

}  // namespace gw

extern "C" const char* gw_last_error(void) { return gw::g_last_error.c_str(); }

extern "C" int gw_abi_version(void) { return 105; }
