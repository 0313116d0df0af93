// Error state and version of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace {
thread_local char g_error[512] = "";
}

void mko_set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
}

int mko_check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    mko_set_error("%s: launch failed: %s", what, hipGetErrorString(err));
    return MKO_ELAUNCH;
  }
  return MKO_OK;
}

extern "C" int mko_abi_version(void) { return MKO_ABI_VERSION; }

extern "C" const char* mko_last_error(void) { return g_error; }

extern "C" size_t mko_sizeof_selscan_params(void) { return sizeof(mko_selscan_params); }

extern "C" size_t mko_sizeof_state_update_params(void) { return sizeof(mko_state_update_params); }
