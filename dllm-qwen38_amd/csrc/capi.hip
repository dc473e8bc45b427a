// C ABI plumbing shared by every entry point: thread-local last-error text and library metadata.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace dllm {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace dllm

extern "C" const char* dllm_last_error(void) { return dllm::g_last_error; }

extern "C" int dllm_abi_version(void) { return 1; }
