#include "status.hpp"

#include <cstdarg>
#include <cstdio>

namespace {
thread_local char g_last_error[512] = {0};
}  // namespace

namespace qlin {

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return code;
}

int ok() {
  g_last_error[0] = '\0';
  return INFER_HIP_OK;
}

int check_launch(const char* what) {
  const hipError_t status = hipGetLastError();
  if (status != hipSuccess) {
    return fail(INFER_HIP_LAUNCH_FAILED, "%s: kernel launch failed: %s", what,
                hipGetErrorString(status));
  }
  return ok();
}

}  // namespace qlin

extern "C" const char* infer_hip_last_error(void) { return g_last_error; }

extern "C" int infer_hip_abi_version(void) { return INFER_HIP_ABI_VERSION; }
