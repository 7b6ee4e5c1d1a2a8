// Thread-local error message and ABI version.
#include "tf_common.hpp"

namespace tf {

namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char *fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace tf

extern "C" const char *tf_last_error(void) { return tf::g_last_error; }

extern "C" int32_t tf_abi_version(void) { return 15; }
