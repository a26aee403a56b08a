// Short causal depthwise conv + SiLU (the GDN q/k/v front end) for gfx950,
// optionally followed by the per-head L2 normalisation and scale of q / k.
//
// One thread owns one channel over a run of timesteps and slides a K-1 window in
// registers; a wavefront covers 64 consecutive channels of one timestep (coalesced).
// Each run is processed 16 timesteps at a time with all 16 loads issued before the
// arithmetic.  With HD > 0 a head is HD consecutive lanes: the sum of squares is a
// butterfly over those lanes, y / max(||y||, 1e-12) * scale (F.normalize semantics).
// The conv tail (last K-1 pre-activation inputs) is written by the thread that owns
// the sequence's final run.
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
  float scale;
};

constexpr int kConvStep = 16;

template <typename T, int K, int HD>
__global__ void __launch_bounds__(256) short_conv_silu_kernel(ConvArgs a) {
  const int d = blockIdx.x * 256 + threadIdx.x;
  const bool active = d < a.D;  // inactive lanes stay for the head reductions
  const int sq = blockIdx.y;
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
  const int dc = active ? d : 0;

  const T *x = static_cast<const T *>(a.x) + batch * a.x_sb + int64_t(t_begin) * a.x_st + dc;
  T *y = static_cast<T *>(a.y) + batch * a.y_sb + int64_t(t_begin) * a.y_st + dc;
  const T *w = static_cast<const T *>(a.w) + dc * K;
  // Padded batches continue from tail_in; packed sequences start from zeros.
  const T *tail = (a.cu == nullptr && a.tail_in)
                      ? static_cast<const T *>(a.tail_in) + (static_cast<size_t>(batch) * a.D + dc) * (K - 1)
                      : nullptr;

  float wr[K];
#pragma unroll
  for (int r = 0; r < K; ++r) wr[r] = active ? ld(w + r) : 0.f;

  // Window = inputs at sequence positions t_lo-K+1 .. t_lo-1 (negative -> tail).
  float win[K - 1];
#pragma unroll
  for (int r = 0; r < K - 1; ++r) {
    const int pos = t_lo - (K - 1) + r;
    win[r] = !active ? 0.f : pos >= 0 ? ld(x + int64_t(pos) * a.x_st) : (tail ? ld(tail + pos + (K - 1)) : 0.f);
  }
  // Tail out needs the last K-1 entries of [tail || x]; capture the ones that
  // come from tail_in before anything is written (tail_out may alias tail_in).
  float tail_keep[K - 1];
  const bool last_run = t_hi == len;
  if (last_run) {
#pragma unroll
    for (int r = 0; r < K - 1; ++r) {
      const int pos = len - (K - 1) + r;
      tail_keep[r] = (pos >= 0 || !active) ? 0.f : (tail ? ld(tail + pos + (K - 1)) : 0.f);
    }
  }

  for (int t0 = t_lo; t0 < t_hi; t0 += kConvStep) {
    float xs[kConvStep];
#pragma unroll
    for (int i = 0; i < kConvStep; ++i) xs[i] = (active && t0 + i < t_hi) ? ld(x + int64_t(t0 + i) * a.x_st) : 0.f;
#pragma unroll
    for (int i = 0; i < kConvStep; ++i) {
      float acc = wr[K - 1] * xs[i];
#pragma unroll
      for (int r = 0; r < K - 1; ++r) acc = fmaf(wr[r], win[r], acc);
      float v = acc / (1.f + exp_fast(-acc));
      if (HD > 0) {
        float ss = v * v;
#pragma unroll
        for (int off = 1; off < HD; off <<= 1) ss += __shfl_xor(ss, off, 64);
        v *= a.scale / fmaxf(sqrtf(ss), 1e-12f);
      }
      if (active && t0 + i < t_hi) st(y + int64_t(t0 + i) * a.y_st, v);
#pragma unroll
      for (int r = 0; r < K - 2; ++r) win[r] = win[r + 1];
      win[K - 2] = xs[i];
    }
  }

  if (last_run && active && a.tail_out) {
    T *to = static_cast<T *>(a.tail_out) + (static_cast<size_t>(sq) * a.D + d) * (K - 1);
#pragma unroll
    for (int r = 0; r < K - 1; ++r) {
      const int pos = len - (K - 1) + r;
      st(to + r, pos >= 0 ? ld(x + int64_t(pos) * a.x_st) : tail_keep[r]);
    }
  }
}

template <typename T, int HD>
static int launch_conv_hd(const ConvArgs &a, int K, dim3 grid, hipStream_t s) {
  const dim3 block(256);
  switch (K) {
    case 2: short_conv_silu_kernel<T, 2, HD><<<grid, block, 0, s>>>(a); break;
    case 3: short_conv_silu_kernel<T, 3, HD><<<grid, block, 0, s>>>(a); break;
    case 4: short_conv_silu_kernel<T, 4, HD><<<grid, block, 0, s>>>(a); break;
    case 5: short_conv_silu_kernel<T, 5, HD><<<grid, block, 0, s>>>(a); break;
    default: return set_error(MOTIF_ERR_UNSUPPORTED, "short_conv_silu: K must be in {2, 3, 4, 5}");
  }
  return check_launch("short_conv_silu_kernel");
}

template <typename T>
static int launch_conv(const ConvArgs &a, int K, int nseq, int max_len, int head_dim, hipStream_t s) {
  const dim3 grid((a.D + 255) / 256, nseq, max(1, (max_len + a.tch - 1) / a.tch));
  switch (head_dim) {
    case 0: return launch_conv_hd<T, 0>(a, K, grid, s);
    case 16: return launch_conv_hd<T, 16>(a, K, grid, s);
    case 32: return launch_conv_hd<T, 32>(a, K, grid, s);
    case 64: return launch_conv_hd<T, 64>(a, K, grid, s);
    default: return set_error(MOTIF_ERR_UNSUPPORTED, "short_conv_silu: head_dim must be 0, 16, 32 or 64");
  }
}

}  // namespace motif

using namespace motif;

static int conv_entry(
    const void *x, int64_t x_sb, int64_t x_st,
    const void *weight, const void *tail_in, void *tail_out,
    void *y, int64_t y_sb, int64_t y_st,
    int B, int L, int D, int K,
    const int32_t *cu_seqlens, int nseq, int max_seqlen,
    int head_dim, float scale, int dtype, void *stream) {
  if (B < 0 || L < 0 || D <= 0 || K < 2 || nseq < 0 || max_seqlen < 0)
    return set_error(MOTIF_ERR_INVALID, "short_conv_silu: bad size");
  if (head_dim && D % head_dim) return set_error(MOTIF_ERR_INVALID, "short_conv_silu: D must be a multiple of head_dim");
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
  a.scale = scale;
  // A run that reads tail_in and a run that writes an aliased tail_out must be
  // the same thread, so in-place updates use a single run per sequence.
  const bool aliased = tail_out != nullptr && tail_out == tail_in;
  a.tch = aliased ? max(1, max_seqlen) : kConvStep;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MOTIF_F32) return launch_conv<float>(a, K, nseq, max_seqlen, head_dim, s);
  if (dtype == MOTIF_BF16) return launch_conv<bf16_t>(a, K, nseq, max_seqlen, head_dim, s);
  return set_error(MOTIF_ERR_UNSUPPORTED, "short_conv_silu: unsupported dtype");
}

extern "C" int motif_short_conv_silu(
    const void *x, int64_t x_sb, int64_t x_st,
    const void *weight, const void *tail_in, void *tail_out,
    void *y, int64_t y_sb, int64_t y_st,
    int B, int L, int D, int K,
    const int32_t *cu_seqlens, int nseq, int max_seqlen,
    int dtype, void *stream) {
  return conv_entry(x, x_sb, x_st, weight, tail_in, tail_out, y, y_sb, y_st, B, L, D, K, cu_seqlens, nseq,
                    max_seqlen, 0, 1.f, dtype, stream);
}

extern "C" int motif_short_conv_silu_l2norm(
    const void *x, int64_t x_sb, int64_t x_st,
    const void *weight, const void *tail_in, void *tail_out,
    void *y, int64_t y_sb, int64_t y_st,
    int B, int L, int D, int K,
    const int32_t *cu_seqlens, int nseq, int max_seqlen,
    int head_dim, float scale, int dtype, void *stream) {
  if (head_dim != 16 && head_dim != 32 && head_dim != 64)
    return set_error(MOTIF_ERR_UNSUPPORTED, "short_conv_silu_l2norm: head_dim must be 16, 32 or 64");
  return conv_entry(x, x_sb, x_st, weight, tail_in, tail_out, y, y_sb, y_st, B, L, D, K, cu_seqlens, nseq,
                    max_seqlen, head_dim, scale, dtype, stream);
}
