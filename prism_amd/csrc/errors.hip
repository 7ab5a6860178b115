// Host-side error reporting for the prism_bsa C-ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

static thread_local char g_err[512] = "";

void prism_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

extern "C" {

// Message of the last failed call on this thread ("" if none).
const char* prism_last_error(void) { return g_err; }

// ABI version of this library; bumped on any signature change.
int prism_abi_version(void) { return 10; }

}  // extern "C"
