// The C ABI's error channel: a negative status from every entry point, and a message for the calling thread.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace sh {

static thread_local char g_message[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_message, sizeof g_message, fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(E_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return OK;
}

}  // namespace sh

extern "C" {

const char* sh_last_error(void) { return sh::g_message; }

int sh_version(void) { return 1; }

int sh_kind_block(int kind, int* weights_per_block, int* bytes_per_block) {
  if (kind < 0 || kind >= sh::N_KINDS) return sh::fail(sh::E_KIND, "unknown block kind %d", kind);
  if (weights_per_block) *weights_per_block = sh::wpb(kind);
  if (bytes_per_block) *bytes_per_block = sh::bpb(kind);
  return sh::OK;
}

size_t sh_tables_bytes(void) { return sh::TAB_BYTES; }

}  // extern "C"
