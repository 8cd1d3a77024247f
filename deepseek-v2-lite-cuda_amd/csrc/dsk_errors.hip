// Error state of the C ABI: a thread-local message behind dsk_last_error(),
// and the post-launch check every entry point runs.
#include "dsk_common.hpp"

namespace dsk {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return DSK_ERR_LAUNCH;
  }
  return DSK_OK;
}

}  // namespace dsk

extern "C" const char* dsk_last_error(void) { return dsk::g_last_error.c_str(); }

extern "C" int dsk_abi_version(void) { return 3; }
