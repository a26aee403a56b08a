// Intra-block attention-residual read, fused: for every token
//   r_n = 1 / sqrt(mean(x_n^2) + eps),  s_n = sum_d q_d w_d x_nd r_n,
//   alpha = softmax_n(s),               h = sum_n alpha_n x_n
// over the block's sources x_n [B, T, D] (fp32 arithmetic).  The same math as the
// reference's fused read (motif/ops/attn_res.py:22-55 `_ar_logit`, :94-186) and
// its eager form (motif/ops/attn_res.py:588-593).
//
// 32 lanes per token (64 for rows of more than 128 16-byte pieces); every source row
// is read once (16-byte loads) and kept in registers for the weighted sum, so the op
// moves (nsrc + 1) * D elements per token -- HBM-bound.  Row sums use DPP and lane
// swaps, not LDS.
#include "capi_internal.h"
#include "common.h"

namespace motif {

namespace {

constexpr int kMaxSrc = 8;

struct AttnResArgs {
  const void *src[kMaxSrc];
  int64_t sb[kMaxSrc], st[kMaxSrc];
  const void *query, *weight;
  void *out;                 // h (may be NULL when the norms are requested)
  int64_t ob, ot;
  int nsrc, B, T, D;
  float eps;
  // optional RMSNorms of h (the decoder's attn_norm / mlp_norm): nout[i] =
  // RMSNorm(h; nw[i], neps) for i < nnorm
  int nnorm;
  const void *nw[2];
  void *nout[2];
  int64_t nb[2], nt[2];
  float neps;
};

// 16-byte piece <-> 8 (bf16) or 4 (fp32) floats
template <typename T> struct Piece;
template <> struct Piece<bf16_t> {
  static constexpr int N = 8;
  __device__ static void load(const bf16_t *p, float *x) { unpack(*reinterpret_cast<const uint4 *>(p), x); }
  __device__ static void unpack(const uint4 u, float *x) {
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
  __device__ static void load(const float *p, float *x) { unpack(*reinterpret_cast<const uint4 *>(p), x); }
  __device__ static void unpack(const uint4 u, float *x) {
    x[0] = __uint_as_float(u.x); x[1] = __uint_as_float(u.y);
    x[2] = __uint_as_float(u.z); x[3] = __uint_as_float(u.w);
  }
  __device__ static void store(float *p, const float *x) {
    *reinterpret_cast<float4 *>(p) = float4{x[0], x[1], x[2], x[3]};
  }
};

template <typename T> __device__ __forceinline__ float round_to(float v);
template <> __device__ __forceinline__ float round_to<float>(float v) { return v; }
template <> __device__ __forceinline__ float round_to<bf16_t>(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// Sum over the LPT-lane group of a lane (LPT = 32 or 64) with DPP and lane swaps: no
// LDS traffic, a few cycles per step.
template <int LPT>
__device__ __forceinline__ float group_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, false));  // row_half_mirror
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xF, 0xF, false));  // row_mirror
  const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
  if (LPT == 64) {
    const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
  }
  return x;
}

// LPT lanes per token (64 / LPT tokens per wave), PPL 16-byte pieces per lane
// (D <= LPT * PPL * Piece::N).  Every lane of a wave takes part in the group sums;
// lanes of tokens past the end compute on zeros and store nothing.
template <typename T, int LPT, int PPL, int NS>
__global__ void __launch_bounds__(256) attn_res_kernel(AttnResArgs a) {
  constexpr int E = Piece<T>::N;
  const int sub = threadIdx.x & (LPT - 1);
  const int tok_raw = blockIdx.x * (blockDim.x / LPT) + threadIdx.x / LPT;
  const bool tok_ok = tok_raw < a.B * a.T;
  const int tok = tok_ok ? tok_raw : 0;
  const int b = tok / a.T, t = tok - b * a.T;
  const int np = a.D / E;

  const uint32_t dbytes = static_cast<uint32_t>(a.D * sizeof(T));
  const buf_t qb = make_buf(a.query, dbytes), wb = make_buf(a.weight, dbytes);
  float qw[PPL][E];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    float qv[E], wv[E];
    Piece<T>::unpack(buf_ld16(qb, (sub + LPT * i) * 16), qv);
    Piece<T>::unpack(buf_ld16(wb, (sub + LPT * i) * 16), wv);
#pragma unroll
    for (int e = 0; e < E; ++e) qw[i][e] = qv[e] * wv[e];
  }

  // the norm weights of the outputs, requested first (read after the reductions they
  // would add a memory round trip at the end); only the norms asked for
  uint4 nwr[2][PPL];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
#pragma unroll
    for (int i = 0; i < PPL; ++i) nwr[k][i] = uint4{0u, 0u, 0u, 0u};
    if (k < a.nnorm) {
      const buf_t nb = make_buf(a.nw[k], dbytes);
#pragma unroll
      for (int i = 0; i < PPL; ++i) nwr[k][i] = buf_ld16(nb, (sub + LPT * i) * 16);
    }
  }

  // every source row is loaded before any reduction, so the loads overlap.  Plain loads
  // from per-lane row addresses (a buffer resource per row would differ between the
  // tokens of a wave and turn each load into a loop over them); pieces past D load the
  // row's last piece and are masked to zeros by an AND (a select on the loaded value
  // would become a branch around the load, and a wait for it).  The unpacking runs for
  // every source slot after all loads (absent sources read as zeros): unpacked inside
  // each source's branch, the loads of a source would wait for the previous one.
  uint4 raw[NS][PPL];
#pragma unroll
  for (int n = 0; n < NS; ++n)
#pragma unroll
    for (int i = 0; i < PPL; ++i) raw[n][i] = uint4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    if (n >= a.nsrc) break;
    const T *row = static_cast<const T *>(a.src[n]) + b * a.sb[n] + int64_t(t) * a.st[n];
#pragma unroll
    for (int i = 0; i < PPL; ++i) raw[n][i] = *reinterpret_cast<const uint4 *>(row + min(sub + LPT * i, np - 1) * E);
  }
  float x[NS][PPL][E];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const uint32_t keep = sub + LPT * i < np ? 0xffffffffu : 0u;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      const uint4 u = raw[n][i];
      Piece<T>::unpack(uint4{u.x & keep, u.y & keep, u.z & keep, u.w & keep}, x[n][i]);
    }
  }
  float logit[NS];
  float mx = -INFINITY;
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    logit[n] = -INFINITY;
    if (n < a.nsrc) {
      float ss = 0.f, dot = 0.f;
#pragma unroll
      for (int i = 0; i < PPL; ++i)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          ss = fmaf(x[n][i][e], x[n][i][e], ss);
          dot = fmaf(x[n][i][e], qw[i][e], dot);
        }
      ss = group_sum<LPT>(ss);
      dot = group_sum<LPT>(dot);
      logit[n] = dot * rsqrtf(ss / a.D + a.eps);
      mx = fmaxf(mx, logit[n]);
    }
  }
  float alpha[NS], den = 0.f;
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    alpha[n] = n < a.nsrc ? exp_f(logit[n] - mx) : 0.f;
    den += alpha[n];
  }
  const float inv = 1.f / den;
  float h[PPL][E];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
#pragma unroll
    for (int e = 0; e < E; ++e) h[i][e] = 0.f;
#pragma unroll
    for (int n = 0; n < NS; ++n)
      if (n < a.nsrc) {
#pragma unroll
        for (int e = 0; e < E; ++e) h[i][e] = fmaf(alpha[n] * inv, x[n][i][e], h[i][e]);
      }
  }
  if (a.out && tok_ok) {
    T *orow = static_cast<T *>(a.out) + b * a.ob + int64_t(t) * a.ot;
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int p = sub + LPT * i;
      if (p < np) Piece<T>::store(orow + p * E, h[i]);
    }
  }
  if (a.nnorm == 0) return;
  // RMSNorm of h as the reference computes it on the stored h (rms_norm.py:481-486):
  // y = T(h * rsqrt(mean(h^2) + eps)) * weight, the product rounded to T (pieces past
  // D hold h = 0 and add nothing).
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PPL; ++i)
#pragma unroll
    for (int e = 0; e < E; ++e) {
      h[i][e] = round_to<T>(h[i][e]);
      ss = fmaf(h[i][e], h[i][e], ss);
    }
  const float r = rsqrtf(group_sum<LPT>(ss) / a.D + a.neps);
  if (!tok_ok) return;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (k >= a.nnorm) break;
    T *nrow = static_cast<T *>(a.nout[k]) + b * a.nb[k] + int64_t(t) * a.nt[k];
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int p = sub + LPT * i;
      if (p >= np) continue;
      float w[E], y[E];
      Piece<T>::unpack(nwr[k][i], w);
#pragma unroll
      for (int e = 0; e < E; ++e) y[e] = round_to<T>(h[i][e] * r) * w[e];
      Piece<T>::store(nrow + p * E, y);
    }
  }
}

// Up to 256 tokens (decode batches) each token gets a one-wave workgroup, so the
// launch spreads over as many CUs as there are tokens (64 decode rows: 5.6 us per read
// against 8.2 us with four waves and eight tokens per workgroup).
template <typename T, int LPT, int NS>
int launch_lpt(const AttnResArgs &a, int ppl, hipStream_t s) {
  const int bs = a.B * a.T <= 256 ? LPT : 256;
  const dim3 grid((a.B * a.T + bs / LPT - 1) / (bs / LPT)), block(bs);
  switch (ppl) {
    case 1: attn_res_kernel<T, LPT, 1, NS><<<grid, block, 0, s>>>(a); break;
    case 2: attn_res_kernel<T, LPT, 2, NS><<<grid, block, 0, s>>>(a); break;
    case 3: attn_res_kernel<T, LPT, 3, NS><<<grid, block, 0, s>>>(a); break;
    case 4: attn_res_kernel<T, LPT, 4, NS><<<grid, block, 0, s>>>(a); break;
    default: return set_error(MOTIF_ERR_UNSUPPORTED, "attn_res_read: D too large (at most 256 16-byte pieces)");
  }
  return check_launch("attn_res_kernel");
}

template <typename T>
int launch(const AttnResArgs &a, hipStream_t s) {
  constexpr int E = Piece<T>::N;
  const int np = a.D / E;
  // two tokens a wave (32 lanes each) up to 128 pieces, else one; one token a wave
  // (and a workgroup) for up to 256 tokens
  // source slots in registers: 4 (every read of a block of up to four decoders) or the
  // most the kernel takes
  if (np <= 128 && a.B * a.T > 256)
    return a.nsrc <= 4 ? launch_lpt<T, 32, 4>(a, (np + 31) / 32, s) : launch_lpt<T, 32, kMaxSrc>(a, (np + 31) / 32, s);
  return a.nsrc <= 4 ? launch_lpt<T, 64, 4>(a, (np + 63) / 64, s) : launch_lpt<T, 64, kMaxSrc>(a, (np + 63) / 64, s);
}

}  // namespace

}  // namespace motif

namespace motif {
namespace {

int attn_res_entry(const void *const *sources, const int64_t *src_sb, const int64_t *src_st, int nsrc,
                   const void *query, const void *norm_weight, float eps, void *out, int64_t out_sb,
                   int64_t out_st, int nnorm, const void *const *nw, void *const *nout, const int64_t *nsb,
                   const int64_t *nst, float neps, int B, int T, int D, int dtype, void *stream) {
  if (nsrc < 1 || nsrc > kMaxSrc)
    return set_error(MOTIF_ERR_UNSUPPORTED, "attn_res_read: 1 to 8 sources");
  if (B < 0 || T < 0 || D <= 0 || !sources || !src_sb || !src_st || !query || !norm_weight || (!out && nnorm == 0))
    return set_error(MOTIF_ERR_INVALID, "attn_res_read: bad argument");
  if (dtype != MOTIF_F32 && dtype != MOTIF_BF16) return set_error(MOTIF_ERR_UNSUPPORTED, "attn_res_read: dtype");
  const int esz = dtype == MOTIF_BF16 ? 2 : 4, vec = 16 / esz;
  if (D % vec) return set_error(MOTIF_ERR_UNSUPPORTED, "attn_res_read: D must be a multiple of 16 bytes");
  AttnResArgs a{};
  uintptr_t align = reinterpret_cast<uintptr_t>(query) | reinterpret_cast<uintptr_t>(norm_weight) |
                    reinterpret_cast<uintptr_t>(out);
  int64_t strides = out ? (out_sb | out_st) : 0;
  for (int n = 0; n < nsrc; ++n) {
    if (!sources[n]) return set_error(MOTIF_ERR_INVALID, "attn_res_read: NULL source");
    a.src[n] = sources[n];
    a.sb[n] = src_sb[n];
    a.st[n] = src_st[n];
    align |= reinterpret_cast<uintptr_t>(sources[n]);
    strides |= src_sb[n] | src_st[n];
  }
  for (int k = 0; k < nnorm; ++k) {
    if (!nw[k] || !nout[k]) return set_error(MOTIF_ERR_INVALID, "attn_res_read: NULL norm operand");
    a.nw[k] = nw[k];
    a.nout[k] = nout[k];
    a.nb[k] = nsb[k];
    a.nt[k] = nst[k];
    align |= reinterpret_cast<uintptr_t>(nw[k]) | reinterpret_cast<uintptr_t>(nout[k]);
    strides |= nsb[k] | nst[k];
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
  a.nnorm = nnorm;
  a.neps = neps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == MOTIF_BF16 ? launch<bf16_t>(a, s) : launch<float>(a, s);
}

}  // namespace
}  // namespace motif

extern "C" int motif_attn_res_read(const void *const *sources, const int64_t *src_sb, const int64_t *src_st,
                                   int nsrc, const void *query, const void *norm_weight, float eps, void *out,
                                   int64_t out_sb, int64_t out_st, int B, int T, int D, int dtype, void *stream) {
  return motif::attn_res_entry(sources, src_sb, src_st, nsrc, query, norm_weight, eps, out, out_sb, out_st, 0,
                               nullptr, nullptr, nullptr, nullptr, 0.f, B, T, D, dtype, stream);
}

extern "C" int motif_attn_res_read_norms(const void *const *sources, const int64_t *src_sb,
                                         const int64_t *src_st, int nsrc, const void *query,
                                         const void *norm_weight, float eps, void *out, int64_t out_sb,
                                         int64_t out_st, int nnorm, const void *const *norm_weights,
                                         void *const *norm_outs, const int64_t *norm_sb, const int64_t *norm_st,
                                         float norm_eps, int B, int T, int D, int dtype, void *stream) {
  if (nnorm < 0 || nnorm > 2) return motif::set_error(MOTIF_ERR_INVALID, "attn_res_read: 0 to 2 norms");
  return motif::attn_res_entry(sources, src_sb, src_st, nsrc, query, norm_weight, eps, out, out_sb, out_st, nnorm,
                               norm_weights, norm_outs, norm_sb, norm_st, norm_eps, B, T, D, dtype, stream);
}
