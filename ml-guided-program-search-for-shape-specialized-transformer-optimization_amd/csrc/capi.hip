// Library identity and the thread-local status message behind sah_last_error().
#include "sah_common.hpp"

namespace sah {

namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
}

int fail(int status, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return status;
}

int check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return SAH_OK;
  return fail(SAH_ERR_HIP, "%s failed: %s", what, hipGetErrorString(err));
}

}  // namespace sah

extern "C" int sah_abi_version(void) { return SAH_ABI_VERSION; }

extern "C" const char* sah_last_error(void) { return sah::g_last_error; }
