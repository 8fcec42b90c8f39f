// Status / error-text plumbing shared by every C entry point.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/moe_amd.h"

namespace moe {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: HIP error %d (%s)", what, (int)err, hipGetErrorString(err));
    return MOE_ERR_HIP;
  }
  return MOE_OK;
}

}  // namespace moe

extern "C" int moe_amd_abi_version(void) { return 1; }

extern "C" const char* moe_amd_last_error(void) { return moe::g_last_error; }
