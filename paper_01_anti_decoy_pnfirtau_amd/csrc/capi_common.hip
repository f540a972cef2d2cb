// Error state and version entry points of libpnfx.so.
#include <stdarg.h>
#include <stdio.h>

#include "pnfx_common.h"

namespace pnfx {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return PNFX_ELAUNCH;
  }
  return PNFX_OK;
}

}  // namespace pnfx

extern "C" int pnfx_abi_version(void) { return PNFX_ABI_VERSION; }
extern "C" const char* pnfx_last_error(void) { return pnfx::g_err; }
