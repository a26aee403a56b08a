// motif_chord_decode_noalloc: the device-cursor Chord decode step for callers that
// cannot allocate device memory (code under graph capture that must not call
// hipMalloc, tight serving loops, harnesses that forbid allocation).  Same kernels
// and arguments as motif_chord_decode, but the split partials (and the fp32 path's
// bias table) live in `scratch`, a file-scope device array of kScratchBytes that
// every GPU the library runs on holds until the process ends.
//
// Host code never passes the array's name to a kernel: on the host it is only a
// stand-in symbol.  The first call on a device (that device current) resolves the
// array's device address with hipGetSymbolAddress and keeps it per device; kernels
// receive that address as their workspace.
//
// All calls on one GPU share its scratch: calls that overlap in time on one GPU
// (different streams, or concurrent host threads) race on it.  Nothing in the
// scratch needs clearing between calls: every split writes all of its partial rows
// and the bias table is rewritten by each fp32 call.
#include <mutex>

#include "capi_internal.h"
#include "chord_internal.h"

namespace motif {
namespace {

constexpr size_t kScratchBytes = size_t(16) << 20;  // 16 MiB per device
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (resolved once per device).
int scratch_ptr(void **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(MOTIF_ERR_HIP, std::string("chord_decode_noalloc: hipGetDevice: ") +
                                                         hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(MOTIF_ERR_UNSUPPORTED, "chord_decode_noalloc: device index beyond the supported 64");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(MOTIF_ERR_HIP, std::string("chord_decode_noalloc: hipGetSymbolAddress: ") +
                                          hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOTIF_OK;
}

}  // namespace
}  // namespace motif

extern "C" size_t motif_chord_decode_noalloc_scratch_bytes(void) { return motif::kScratchBytes; }

extern "C" int motif_chord_decode_noalloc(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int *length_dev, int capacity,
    const float *alpha, const float *beta, const float *mu, const float *ssmax,
    const float *log_n, int64_t ln_sb, int64_t ln_st, const float *log_table, int log_table_len,
    void *out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int Hkv, int L, int D, float scale, float eps, int dtype, void *stream) {
  using namespace motif;
  const size_t need = motif_chord_decode_workspace_bytes(B, H, Hkv, L, capacity, D, dtype, nullptr);
  if (need > kScratchBytes)
    return set_error(MOTIF_ERR_INVALID, "chord_decode_noalloc: these sizes need " + std::to_string(need) +
                                            " bytes of scratch, more than the library's " +
                                            std::to_string(kScratchBytes) + "; use motif_chord_decode");
  // sizes the decode rejects (or has nothing to do for) never reach the scratch
  if (B <= 0 || L <= 0 || H <= 0 || Hkv <= 0)
    return chord_decode_run(q, q_sb, q_sh, q_st, k_cache, k_sb, k_sh, k_st, v_cache, v_sb, v_sh, v_st, length_dev,
                            capacity, alpha, beta, mu, ssmax, log_n, ln_sb, ln_st, log_table, log_table_len, out,
                            o_sb, o_sh, o_st, B, H, Hkv, L, D, scale, eps, nullptr, 0, dtype, stream);
  void *ws = nullptr;
  const int rc = scratch_ptr(&ws);
  if (rc) return rc;
  return chord_decode_run(q, q_sb, q_sh, q_st, k_cache, k_sb, k_sh, k_st, v_cache, v_sb, v_sh, v_st, length_dev,
                          capacity, alpha, beta, mu, ssmax, log_n, ln_sb, ln_st, log_table, log_table_len, out, o_sb,
                          o_sh, o_st, B, H, Hkv, L, D, scale, eps, ws, kScratchBytes, dtype, stream);
}
