// Error plumbing shared by the C-ABI launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "../../include/motif_hip.h"

namespace motif {

int set_error(int code, const std::string &msg);

// Zero n bytes at p on stream s with a kernel (safe inside a captured graph).
int zero_async(void *p, size_t n, hipStream_t s);

inline int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(MOTIF_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return MOTIF_OK;
}

}  // namespace motif
