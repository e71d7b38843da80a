// Status strings, the thread-local last-error message and the ABI version.
#include "rp_common.h"

#include <stdarg.h>
#include <stdio.h>

namespace {
thread_local char g_last_error[512] = "";
}

extern "C" void rp_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

extern "C" const char* rp_last_error(void) { return g_last_error; }

extern "C" int rp_abi_version(void) { return 3; }

extern "C" const char* rp_status_string(int status) {
  switch (status) {
    case RP_OK: return "ok";
    case RP_ERR_INVALID_ARGUMENT: return "invalid argument";
    case RP_ERR_UNSUPPORTED: return "unsupported shape or layout";
    case RP_ERR_WORKSPACE: return "workspace missing or too small";
    case RP_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown status";
  }
}
