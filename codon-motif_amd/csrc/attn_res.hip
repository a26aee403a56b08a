// Intra-block attention-residual read, fused: for every token
//   r_n = 1 / sqrt(mean(x_n^2) + eps),  s_n = sum_d q_d w_d x_nd r_n,
//   alpha = softmax_n(s),               h = sum_n alpha_n x_n
// over the block's sources x_n [B, T, D] (fp32 arithmetic).  The same math as the
// reference's fused read (motif/ops/attn_res.py:22-55 `_ar_logit`, :94-186) and
// its eager form (motif/ops/attn_res.py:588-593).
//
// One wavefront per token; every source row is read once (16-byte loads) and kept
// in registers for the weighted sum, so the op moves (nsrc + 1) * D elements per
// token -- HBM-bound.
#include "capi_internal.h"
#include "common.h"

namespace motif {

namespace {

constexpr int kMaxSrc = 8;

struct AttnResArgs {
  const void *src[kMaxSrc];
  int64_t sb[kMaxSrc], st[kMaxSrc];
  const void *query, *weight;
  void *out;
  int64_t ob, ot;
  int nsrc, B, T, D;
  float eps;
};

// 16-byte piece <-> 8 (bf16) or 4 (fp32) floats
template <typename T> struct Piece;
template <> struct Piece<bf16_t> {
  static constexpr int N = 8;
  __device__ static void load(const bf16_t *p, float *x) {
    const uint4 u = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ static void store(bf16_t *p, const float *x) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(f32_to_bf16(x[2 * i])) | (static_cast<uint32_t>(f32_to_bf16(x[2 * i + 1])) << 16);
    *reinterpret_cast<uint4 *>(p) = uint4{w[0], w[1], w[2], w[3]};
  }
};
template <> struct Piece<float> {
  static constexpr int N = 4;
  __device__ static void load(const float *p, float *x) {
    const float4 u = *reinterpret_cast<const float4 *>(p);
    x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
  }
  __device__ static void store(float *p, const float *x) {
    *reinterpret_cast<float4 *>(p) = float4{x[0], x[1], x[2], x[3]};
  }
};

// PPL: 16-byte pieces per lane (D <= 64 * PPL * Piece::N).
template <typename T, int PPL>
__global__ void __launch_bounds__(256) attn_res_kernel(AttnResArgs a) {
  constexpr int E = Piece<T>::N;
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= a.B * a.T) return;
  const int b = tok / a.T, t = tok - b * a.T;
  const int np = a.D / E;

  float qw[PPL][E];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int p = lane + 64 * i;
    float qv[E], wv[E];
    if (p < np) {
      Piece<T>::load(static_cast<const T *>(a.query) + p * E, qv);
      Piece<T>::load(static_cast<const T *>(a.weight) + p * E, wv);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) qv[e] = wv[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) qw[i][e] = qv[e] * wv[e];
  }

  float x[kMaxSrc][PPL][E];
  float logit[kMaxSrc];
  float mx = -INFINITY;
#pragma unroll
  for (int n = 0; n < kMaxSrc; ++n) {
    logit[n] = -INFINITY;
    if (n < a.nsrc) {
      const T *row = static_cast<const T *>(a.src[n]) + b * a.sb[n] + int64_t(t) * a.st[n];
      float ss = 0.f, dot = 0.f;
#pragma unroll
      for (int i = 0; i < PPL; ++i) {
        const int p = lane + 64 * i;
        if (p < np) Piece<T>::load(row + p * E, x[n][i]);
        else {
#pragma unroll
          for (int e = 0; e < E; ++e) x[n][i][e] = 0.f;
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
          ss = fmaf(x[n][i][e], x[n][i][e], ss);
          dot = fmaf(x[n][i][e], qw[i][e], dot);
        }
      }
      ss = wave_sum(ss);
      dot = wave_sum(dot);
      logit[n] = dot * rsqrtf(ss / a.D + a.eps);
      mx = fmaxf(mx, logit[n]);
    }
  }
  float alpha[kMaxSrc], den = 0.f;
#pragma unroll
  for (int n = 0; n < kMaxSrc; ++n) {
    alpha[n] = n < a.nsrc ? exp_f(logit[n] - mx) : 0.f;
    den += alpha[n];
  }
  const float inv = 1.f / den;
  T *orow = static_cast<T *>(a.out) + b * a.ob + int64_t(t) * a.ot;
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int p = lane + 64 * i;
    if (p >= np) continue;
    float h[E];
#pragma unroll
    for (int e = 0; e < E; ++e) h[e] = 0.f;
#pragma unroll
    for (int n = 0; n < kMaxSrc; ++n)
      if (n < a.nsrc) {
#pragma unroll
        for (int e = 0; e < E; ++e) h[e] = fmaf(alpha[n] * inv, x[n][i][e], h[e]);
      }
    Piece<T>::store(orow + p * E, h);
  }
}

template <typename T>
int launch(const AttnResArgs &a, hipStream_t s) {
  constexpr int E = Piece<T>::N;
  const int np = a.D / E;
  const dim3 grid((a.B * a.T + 3) / 4), block(256);
  if (np <= 64) attn_res_kernel<T, 1><<<grid, block, 0, s>>>(a);
  else if (np <= 128) attn_res_kernel<T, 2><<<grid, block, 0, s>>>(a);
  else if (np <= 256) attn_res_kernel<T, 4><<<grid, block, 0, s>>>(a);
  else return set_error(MOTIF_ERR_UNSUPPORTED, "attn_res_read: D too large (at most 256 16-byte pieces)");
  return check_launch("attn_res_kernel");
}

}  // namespace

}  // namespace motif

extern "C" int motif_attn_res_read(const void *const *sources, const int64_t *src_sb, const int64_t *src_st,
                                   int nsrc, const void *query, const void *norm_weight, float eps, void *out,
                                   int64_t out_sb, int64_t out_st, int B, int T, int D, int dtype, void *stream) {
  using namespace motif;
  if (nsrc < 1 || nsrc > kMaxSrc)
    return set_error(MOTIF_ERR_UNSUPPORTED, "attn_res_read: 1 to 8 sources");
  if (B < 0 || T < 0 || D <= 0 || !sources || !src_sb || !src_st || !query || !norm_weight || !out)
    return set_error(MOTIF_ERR_INVALID, "attn_res_read: bad argument");
  if (dtype != MOTIF_F32 && dtype != MOTIF_BF16) return set_error(MOTIF_ERR_UNSUPPORTED, "attn_res_read: dtype");
  const int esz = dtype == MOTIF_BF16 ? 2 : 4, vec = 16 / esz;
  if (D % vec) return set_error(MOTIF_ERR_UNSUPPORTED, "attn_res_read: D must be a multiple of 16 bytes");
  AttnResArgs a{};
  uintptr_t align = reinterpret_cast<uintptr_t>(query) | reinterpret_cast<uintptr_t>(norm_weight) |
                    reinterpret_cast<uintptr_t>(out);
  int64_t strides = out_sb | out_st;
  for (int n = 0; n < nsrc; ++n) {
    if (!sources[n]) return set_error(MOTIF_ERR_INVALID, "attn_res_read: NULL source");
    a.src[n] = sources[n];
    a.sb[n] = src_sb[n];
    a.st[n] = src_st[n];
    align |= reinterpret_cast<uintptr_t>(sources[n]);
    strides |= src_sb[n] | src_st[n];
  }
  if ((align & 15) || (strides % vec))
    return set_error(MOTIF_ERR_UNSUPPORTED, "attn_res_read: rows must be 16-byte aligned");
  if (B == 0 || T == 0) return MOTIF_OK;
  a.query = query;
  a.weight = norm_weight;
  a.out = out;
  a.ob = out_sb;
  a.ot = out_st;
  a.nsrc = nsrc;
  a.B = B;
  a.T = T;
  a.D = D;
  a.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == MOTIF_BF16 ? launch<bf16_t>(a, s) : launch<float>(a, s);
}
