// Host-side plumbing of the C ABI: per-thread last-error text, launch checks.
#include "rrl_common.hpp"

namespace rrl {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return RRL_ELAUNCH;
  }
  return RRL_OK;
}

}  // namespace rrl

extern "C" const char* rrl_last_error(void) { return rrl::g_last_error.c_str(); }
extern "C" int rrl_abi_version(void) { return RRL_ABI_VERSION; }
