// Library-level entry points: version, status strings, per-thread error text.
#include <stdarg.h>
#include <stdio.h>

#include "tm_common.h"

namespace {
thread_local char g_last_error[512] = {0};
}

int tm_fail(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

void tm_clear_error() { g_last_error[0] = 0; }

extern "C" int tm_version(void) { return 100; }

extern "C" const char *tm_status_string(int status) {
  switch (status) {
    case TM_OK: return "TM_OK";
    case TM_EINVAL_SHAPE: return "TM_EINVAL_SHAPE";
    case TM_EINVAL_DTYPE: return "TM_EINVAL_DTYPE";
    case TM_EINVAL_ARG: return "TM_EINVAL_ARG";
    case TM_EHIP: return "TM_EHIP";
    case TM_EWORKSPACE: return "TM_EWORKSPACE";
    default: return "TM_UNKNOWN";
  }
}

extern "C" const char *tm_last_error(void) { return g_last_error; }
