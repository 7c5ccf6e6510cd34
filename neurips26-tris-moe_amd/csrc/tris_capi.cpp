// Error state and version entry points of the C ABI.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "tris_moe_hip.h"

namespace tris {

namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(err));
    return TRIS_ERR_HIP;
  }
  return TRIS_OK;
}

}  // namespace tris

extern "C" int tris_abi_version(void) { return TRIS_COMPACT3_KERNEL_ABI_VERSION; }

extern "C" const char* tris_last_error(void) { return tris::g_last_error; }
