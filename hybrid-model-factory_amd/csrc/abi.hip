// Library-wide C ABI plumbing: version, thread-local error message.
#include "common.hpp"

namespace hmx {

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
  if (e != hipSuccess)
    return set_error(HMX_EHIP, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
  return HMX_OK;
}

}  // namespace hmx

extern "C" int hmx_abi_version(void) { return HMX_ABI_VERSION; }

extern "C" const char* hmx_last_error(void) { return hmx::g_last_error; }
