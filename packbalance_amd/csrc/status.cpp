// Thread-local error reporting behind pb_last_error().
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "common.hpp"

namespace pb {

static thread_local char g_msg[512] = {0};

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
}

void clear_error() { g_msg[0] = 0; }

int launch_status(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return PB_EHIP;
  }
  return PB_OK;
}

}  // namespace pb

extern "C" const char *pb_last_error(void) { return pb::g_msg; }

extern "C" int pb_abi_version(void) { return 4; }
