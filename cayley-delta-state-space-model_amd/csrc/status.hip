// Error reporting for the C-ABI: every entry point returns an int status and
// leaves a human-readable message retrievable with cdssm_last_error().
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace {
thread_local char g_err[512] = "";
}

namespace cdssm_host {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* op) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", op, hipGetErrorString(e));
    return CDSSM_EHIP;
  }
  return CDSSM_OK;
}

}  // namespace cdssm_host

extern "C" const char* cdssm_last_error(void) { return g_err; }

extern "C" int cdssm_abi_version(void) { return 1; }
