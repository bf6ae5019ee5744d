// Library-wide C-ABI entry points: version, error reporting.
#include <stdio.h>
#include <string.h>

#include "pjx_internal.h"

namespace pjx {

static thread_local char g_error[512];

void set_error(const char* msg) {
  strncpy(g_error, msg, sizeof(g_error) - 1);
  g_error[sizeof(g_error) - 1] = '\0';
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* where) {
  const hipError_t err = hipGetLastError();
  if (err == hipSuccess) return PJX_OK;
  char buf[512];
  snprintf(buf, sizeof(buf), "%s: kernel launch failed: %s", where, hipGetErrorString(err));
  set_error(buf);
  return PJX_ERR_LAUNCH;
}

}  // namespace pjx

extern "C" int pjx_version(void) { return 100; }

extern "C" const char* pjx_last_error(void) { return pjx::g_error; }
