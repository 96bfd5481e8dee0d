// Status / message plumbing of the C-ABI.
#include <string>

#include "sph_common.h"

namespace sph {

static thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(static_cast<int>(e), std::string(what) + ": " +
                                              hipGetErrorString(e));
  }
  return SPH_OK;
}

}  // namespace sph

extern "C" const char* sph_last_error(void) { return sph::g_last_error.c_str(); }

extern "C" int sph_abi_version(void) { return SPH_ABI_VERSION; }
