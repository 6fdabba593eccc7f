// Error reporting and version entry points of the anna_mi C ABI.
#include <stdarg.h>

#include "common.hpp"

namespace anna {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail_hip(hipError_t e, const char* what) {
  set_error("%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
  return ANNA_MI_EHIP;
}

}  // namespace anna

extern "C" {

const char* anna_mi_last_error(void) { return anna::g_last_error; }

int anna_mi_abi_version(void) { return ANNA_MI_ABI_VERSION; }

#ifndef ANNA_MI_SOURCE_HASH
#define ANNA_MI_SOURCE_HASH "unstamped"
#endif
const char* anna_mi_source_hash(void) { return ANNA_MI_SOURCE_HASH; }

}  // extern "C"
