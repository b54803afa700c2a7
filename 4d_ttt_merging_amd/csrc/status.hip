// Thread-local error reporting shared by every entry point.
#include "vgo_common.h"

namespace vgo {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(VGO_ELAUNCH, std::string(what) + ": " + hipGetErrorString(err));
  }
  return VGO_OK;
}

}  // namespace vgo

extern "C" const char* vgo_last_error(void) { return vgo::g_last_error.c_str(); }

extern "C" int vgo_abi_version(void) { return VGO_ABI_VERSION; }
