// ABI version and per-thread error message of the motif C ABI.
#include "capi_internal.h"

namespace motif {

static thread_local std::string g_last_error;

int set_error(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

}  // namespace motif

extern "C" int motif_abi_version(void) { return 1; }

extern "C" const char *motif_last_error(void) { return motif::g_last_error.c_str(); }
