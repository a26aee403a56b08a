// Short causal depthwise conv + SiLU (the GDN q/k/v front end) for gfx950.
//
// One thread owns one channel over a run of TCH timesteps and slides a K-1
// window in registers; a wave reads 64 consecutive channels of one timestep
// (coalesced).  The conv tail (last K-1 pre-activation inputs) is written by
// the thread that owns the sequence's final run.
#include "capi_internal.h"
#include "common.h"

namespace motif {

struct ConvArgs {
  const void *x; int64_t x_sb, x_st;
  const void *w;
  const void *tail_in;
  void *tail_out;
  void *y; int64_t y_sb, y_st;
  int B, L, D;
  const int32_t *cu;
  int tch;  // timesteps per thread
};

template <typename T, int K>
__global__ void __launch_bounds__(256) short_conv_silu_kernel(ConvArgs a) {
  const int d = blockIdx.x * 256 + threadIdx.x;
  const int sq = blockIdx.y;
  if (d >= a.D) return;
  int batch, t_begin, len;
  if (a.cu == nullptr) {
    batch = sq;
    t_begin = 0;
    len = a.L;
  } else {
    batch = 0;
    t_begin = a.cu[sq];
    len = a.cu[sq + 1] - t_begin;
  }
  const int t_lo = blockIdx.z * a.tch;
  // An empty sequence still owns its (all-tail) conv state: run z == 0 writes it.
  if (t_lo >= len && !(blockIdx.z == 0 && len == 0)) return;
  const int t_hi = min(len, t_lo + a.tch);

  const T *x = static_cast<const T *>(a.x) + batch * a.x_sb + int64_t(t_begin) * a.x_st + d;
  T *y = static_cast<T *>(a.y) + batch * a.y_sb + int64_t(t_begin) * a.y_st + d;
  const T *w = static_cast<const T *>(a.w) + d * K;
  // Padded batches continue from tail_in; packed sequences start from zeros.
  const T *tail = (a.cu == nullptr && a.tail_in)
                      ? static_cast<const T *>(a.tail_in) + (static_cast<size_t>(batch) * a.D + d) * (K - 1)
                      : nullptr;

  float wr[K];
#pragma unroll
  for (int r = 0; r < K; ++r) wr[r] = ld(w + r);

  // Window = inputs at sequence positions t_lo-K+1 .. t_lo-1 (negative -> tail).
  float win[K - 1];
#pragma unroll
  for (int r = 0; r < K - 1; ++r) {
    const int pos = t_lo - (K - 1) + r;
    win[r] = pos >= 0 ? ld(x + int64_t(pos) * a.x_st) : (tail ? ld(tail + pos + (K - 1)) : 0.f);
  }
  // Tail out needs the last K-1 entries of [tail || x]; capture the ones that
  // come from tail_in before anything is written (tail_out may alias tail_in).
  float tail_keep[K - 1];
  const bool last_run = t_hi == len;
  if (last_run) {
#pragma unroll
    for (int r = 0; r < K - 1; ++r) {
      const int pos = len - (K - 1) + r;
      tail_keep[r] = pos >= 0 ? 0.f : (tail ? ld(tail + pos + (K - 1)) : 0.f);
    }
  }

  for (int t = t_lo; t < t_hi; ++t) {
    const float xt = ld(x + int64_t(t) * a.x_st);
    float acc = wr[K - 1] * xt;
#pragma unroll
    for (int r = 0; r < K - 1; ++r) acc = fmaf(wr[r], win[r], acc);
    const float sig = 1.f / (1.f + exp_f(-acc));
    st(y + int64_t(t) * a.y_st, acc * sig);
#pragma unroll
    for (int r = 0; r < K - 2; ++r) win[r] = win[r + 1];
    win[K - 2] = xt;
  }

  if (last_run && a.tail_out) {
    T *to = static_cast<T *>(a.tail_out) + (static_cast<size_t>(sq) * a.D + d) * (K - 1);
#pragma unroll
    for (int r = 0; r < K - 1; ++r) {
      const int pos = len - (K - 1) + r;
      st(to + r, pos >= 0 ? ld(x + int64_t(pos) * a.x_st) : tail_keep[r]);
    }
  }
}

template <typename T>
static int launch_conv(const ConvArgs &a, int K, int nseq, int max_len, hipStream_t s) {
  dim3 grid((a.D + 255) / 256, nseq, max(1, (max_len + a.tch - 1) / a.tch)), block(256);
  switch (K) {
    case 2: short_conv_silu_kernel<T, 2><<<grid, block, 0, s>>>(a); break;
    case 3: short_conv_silu_kernel<T, 3><<<grid, block, 0, s>>>(a); break;
    case 4: short_conv_silu_kernel<T, 4><<<grid, block, 0, s>>>(a); break;
    case 5: short_conv_silu_kernel<T, 5><<<grid, block, 0, s>>>(a); break;
    default: return set_error(MOTIF_ERR_UNSUPPORTED, "short_conv_silu: K must be in {2, 3, 4, 5}");
  }
  return check_launch("short_conv_silu_kernel");
}

}  // namespace motif

using namespace motif;

extern "C" int motif_short_conv_silu(
    const void *x, int64_t x_sb, int64_t x_st,
    const void *weight, const void *tail_in, void *tail_out,
    void *y, int64_t y_sb, int64_t y_st,
    int B, int L, int D, int K,
    const int32_t *cu_seqlens, int nseq, int max_seqlen,
    int dtype, void *stream) {
  if (B < 0 || L < 0 || D <= 0 || K < 2 || nseq < 0 || max_seqlen < 0)
    return set_error(MOTIF_ERR_INVALID, "short_conv_silu: bad size");
  const bool packed = cu_seqlens != nullptr;
  if (packed && B != 1) return set_error(MOTIF_ERR_INVALID, "short_conv_silu: packed sequences need B == 1");
  if (!packed && (nseq != B || max_seqlen != L))
    return set_error(MOTIF_ERR_INVALID, "short_conv_silu: padded batches need nseq == B and max_seqlen == L");
  if (nseq == 0 || (!packed && L == 0)) {
    if (!packed && tail_out && tail_out != tail_in && B > 0) {
      const size_t n = static_cast<size_t>(B) * D * (K - 1) * (dtype == MOTIF_F32 ? 4 : 2);
      hipError_t e = tail_in ? hipMemcpyAsync(tail_out, tail_in, n, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream))
                             : hipMemsetAsync(tail_out, 0, n, static_cast<hipStream_t>(stream));
      if (e != hipSuccess) return set_error(MOTIF_ERR_HIP, hipGetErrorString(e));
    }
    return MOTIF_OK;
  }
  if (!x || !weight || !y) return set_error(MOTIF_ERR_INVALID, "short_conv_silu: NULL pointer");
  ConvArgs a;
  a.x = x; a.x_sb = x_sb; a.x_st = x_st;
  a.w = weight; a.tail_in = tail_in; a.tail_out = tail_out;
  a.y = y; a.y_sb = y_sb; a.y_st = y_st;
  a.B = B; a.L = L; a.D = D; a.cu = cu_seqlens;
  // A run that reads tail_in and a run that writes an aliased tail_out must be
  // the same thread, so in-place updates use a single run per sequence.
  const bool aliased = tail_out != nullptr && tail_out == tail_in;
  a.tch = aliased ? max(1, max_seqlen) : 64;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MOTIF_F32) return launch_conv<float>(a, K, nseq, max_seqlen, s);
  if (dtype == MOTIF_BF16) return launch_conv<bf16_t>(a, K, nseq, max_seqlen, s);
  return set_error(MOTIF_ERR_UNSUPPORTED, "short_conv_silu: unsupported dtype");
}
