// Error reporting shared by every C-ABI entry point of libuttt_hip.so.
#include <stdarg.h>

#include "common.h"

namespace {
thread_local char g_last_error[512] = {0};
}

namespace uttt {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

// Turns a failed launch into UTTT_ERR_HIP with the runtime's message.
int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(err));
    return UTTT_ERR_HIP;
  }
  return UTTT_OK;
}

}  // namespace uttt

extern "C" int uttt_abi_version(void) { return 1; }

extern "C" const char* uttt_last_error(void) { return g_last_error; }
