// ABI version and per-thread error message of the motif C ABI.
#include "capi_internal.h"

#include <algorithm>

namespace motif {

static thread_local std::string g_last_error;

int set_error(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

// Zero fill as a kernel (a memset node recorded into a captured graph is avoided:
// such nodes have given wrong results on replays).
__global__ void __launch_bounds__(256) zero_bytes_kernel(unsigned char *p, size_t n) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256)
    p[i] = 0;
}

int zero_async(void *p, size_t n, hipStream_t s) {
  if (n == 0) return MOTIF_OK;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 1024);
  zero_bytes_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(static_cast<unsigned char *>(p), n);
  return check_launch("zero_bytes_kernel");
}

}  // namespace motif

extern "C" int motif_abi_version(void) { return 2; }

extern "C" const char *motif_last_error(void) { return motif::g_last_error.c_str(); }
