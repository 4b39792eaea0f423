// Version and error reporting of the C ABI (include/forge_attn.h).
#include <stdio.h>
#include <string.h>

#include "forge_internal.h"

namespace forge {

static thread_local char g_last_error[512] = "";

int set_error(const char* msg) {
  snprintf(g_last_error, sizeof(g_last_error), "%s", msg);
  return -1;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch() {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return 0;
  snprintf(g_last_error, sizeof(g_last_error), "kernel launch failed: %s", hipGetErrorString(e));
  return (int)e;
}

}  // namespace forge

extern "C" int forge_abi_version(void) { return FORGE_ABI_VERSION; }

extern "C" const char* forge_last_error(void) { return forge::g_last_error; }
