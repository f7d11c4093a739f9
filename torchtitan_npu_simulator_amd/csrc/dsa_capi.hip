// C-ABI plumbing shared by every entry point: thread-local error text, version.
#include <cstdarg>
#include <cstdio>
#include <string>

#include "dsa_common.h"

namespace dsa {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(DSA_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return DSA_OK;
}

}  // namespace dsa

extern "C" const char* dsa_last_error(void) { return dsa::g_last_error.c_str(); }

extern "C" int dsa_abi_version(void) { return 11; }
