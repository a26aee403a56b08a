// Fused single-token GDN layer step (decode) for gfx950: everything between the
// input projections and o_proj in one launch per layer.
//
// One workgroup per (head, batch row), one thread per value column e (dv <= 128):
//   1. short conv + SiLU of the new token against the conv tails for the head's
//      q / k channels (threads c < 2 dk) and v channels (thread e); the shifted tails
//      and the new state go to their output buffers, which may be the input buffers
//      (every thread reads its own tail channel and state column before writing them);
//   2. q, k L2-normalised over dk (F.normalize, eps 1e-12), q scaled by dk^-1/2;
//   3. gates beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias);
//   4. the delta rule on the fp32 state column S[:, e] held in registers:
//      S *= e^g; S += k (beta (v_e - k^T S)); o_e = q^T S;
//   5. GatedRMSNorm of the head's dv outputs: o * rsqrt(mean(o^2) + eps) * w * SiLU(gate).
// fp32 arithmetic, with every value the reference layer holds in the activation type T
// rounded to T at the same point: the conv output and its SiLU, the norm, quotient and
// scaled q, beta and the g chain (a + dt_bias, softplus, e^A_log, the product), the
// recurrence's output o, and the three products of the GatedRMSNorm (the recurrence
// itself runs in fp32, as the reference's does).  The reference runs these as separate steps
// (motif/block/attention/gdn_attn.py:116-136 conv, :183-209 normalise / gates /
// recurrent_gated_delta_rule (motif/ops/gated_deltanet.py:26-59) / o_norm,
// motif/ops/rms_norm.py:530-553 GatedRMSNorm).
#include "capi_internal.h"
#include "common.h"

namespace motif {

namespace {

struct GdnDecodeArgs {
  const void *proj; int64_t p_sb;            // [B, ncols] projections (q | k | v | gate | a | b)
  int q_off, k_off, v_off, g_off, a_off, b_off;
  const void *wq, *wk, *wv;                  // conv weights [H*dk, K], [H*dk, K], [H*dv, K]
  const void *tq, *tk, *tv;                  // conv tails [B, C, K-1]
  void *oq, *ok, *ov;                        // shifted tails (may alias tq / tk / tv)
  const void *a_log, *dt_bias, *norm_w;      // [H], [H], [dv]
  float norm_eps;
  const float *state;                        // [B, H, dk, dv] fp32
  float *state_out;                          // may alias state
  void *y; int64_t y_sb;                     // [B, H*dv]
  int B, H, dk, dv;
};

template <typename T, int DK, int K>
__global__ void __launch_bounds__(128) gdn_decode_kernel(GdnDecodeArgs a) {
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  __shared__ float sq[DK], sk[DK], sred[2];
  const bool active = tid < a.dv;

  // The state column, the gate and the norm weight do not depend on the conv: issue
  // their loads first so their latency overlaps the conv / normalisation below.  The
  // state block of (b, h) is one buffer; row i sits at the uniform offset i * dv * 4.  The
  // state is streamed once per step: its loads and stores are nontemporal (cache policy 2).
  const buf_t sbuf = make_buf(a.state + (static_cast<size_t>(b) * a.H + h) * DK * a.dv,
                              static_cast<uint32_t>(DK * a.dv * 4));
  const buf_t obuf = make_buf(a.state_out + (static_cast<size_t>(b) * a.H + h) * DK * a.dv,
                              static_cast<uint32_t>(DK * a.dv * 4));
  const uint32_t col = static_cast<uint32_t>(tid) * 4, row = static_cast<uint32_t>(a.dv) * 4;
  float S[DK];
  if (active) {
#pragma unroll
    for (int i = 0; i < DK; ++i)
      S[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sbuf, col, i * row, 2));
  }
  const T *pr = static_cast<const T *>(a.proj) + b * a.p_sb;
  float gt = 0.f, nw = 0.f, xv = 0.f;
  if (active) {
    gt = ld(pr + a.g_off + h * a.dv + tid);
    nw = ld(static_cast<const T *>(a.norm_w) + tid);
    xv = ld(pr + a.v_off + h * a.dv + tid);
  }
  const float av = ld(pr + a.a_off + h), bv = ld(pr + a.b_off + h);
  const float dtb = ld(static_cast<const T *>(a.dt_bias) + h), alog = ld(static_cast<const T *>(a.a_log) + h);

  auto conv = [&](const void *wgt, const void *tails, void *tails_out, int C, int ch, float xnew) {
    const T *wr = static_cast<const T *>(wgt) + static_cast<size_t>(ch) * K;
    const size_t off = (static_cast<size_t>(b) * C + ch) * (K - 1);
    const T *tl = static_cast<const T *>(tails) + off;
    T *to = static_cast<T *>(tails_out) + off;
    float t[K - 1];
#pragma unroll
    for (int r = 0; r < K - 1; ++r) t[r] = ld(tl + r);
    float acc = ld(wr + K - 1) * xnew;
#pragma unroll
    for (int r = 0; r < K - 1; ++r) acc = fmaf(ld(wr + r), t[r], acc);
#pragma unroll
    for (int r = 0; r < K - 2; ++r) st(to + r, t[r + 1]);
    st(to + K - 2, xnew);
    return gdn_conv_act<T>(acc);
  };

  // 1-2. q / k channels: threads [0, DK) -> q, [DK, 2 DK) -> k; an aligned group of
  // DK lanes holds one vector, so its norm is a butterfly over those lanes.
  if (tid < 2 * DK) {
    const bool isq = tid < DK;
    const int c = isq ? tid : tid - DK;
    const int ch = h * DK + c;
    const float x = ld(pr + (isq ? a.q_off : a.k_off) + ch);
    const float y = conv(isq ? a.wq : a.wk, isq ? a.tq : a.tk, isq ? a.oq : a.ok, a.H * DK, ch, x);
    float ss = y * y;
#pragma unroll
    for (int off = 1; off < DK; off <<= 1) ss += __shfl_xor(ss, off, 64);
    // dk^-1/2 as the host's float(dk ** -0.5)
    constexpr float qs = DK == 16 ? 0.25f : DK == 32 ? 0.17677669529663687f : DK == 64 ? 0.125f : 0.08838834764831845f;
    const float inv = gdn_norm_inv<T>(ss);
    if (isq) sq[c] = gdn_normalized<T>(y, inv, qs);
    else sk[c] = gdn_normalized<T>(y, inv, 1.f);
  }
  float vcol = 0.f;
  if (active) vcol = conv(a.wv, a.tv, a.ov, a.H * a.dv, h * a.dv + tid, xv);
  // 3. gates (uniform): beta = T(sigmoid(b)), g = T(-T(e^A_log) * T(softplus(T(a + dt_bias))))
  // (softplus threshold 20), decay = e^g in fp32
  const float beta = round_as<T>(1.f / (1.f + expf(-bv)));
  const float xa = round_as<T>(av + dtb);
  const float sp = round_as<T>(xa > 20.f ? xa : log1pf(expf(xa)));
  const float decay = expf(round_as<T>(-round_as<T>(expf(alog)) * sp));
  __syncthreads();

  // 4. delta rule on column e
  float o = 0.f;
  if (active) {
    float vold = 0.f;
#pragma unroll
    for (int i = 0; i < DK; ++i) {
      S[i] *= decay;
      vold = fmaf(sk[i], S[i], vold);
    }
    const float delta = beta * (vcol - vold);
#pragma unroll
    for (int i = 0; i < DK; ++i) {
      S[i] = fmaf(sk[i], delta, S[i]);
      o = fmaf(sq[i], S[i], o);
    }
#pragma unroll
    for (int i = 0; i < DK; ++i)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, S[i]), obuf, col, i * row, 2);
  }

  // 5. GatedRMSNorm over the head's dv outputs (two waves: partial sums in LDS) of o
  // rounded to T: y = T(T(T(o rsqrt(mean o^2 + eps)) w) T(silu(gate)))
  o = round_as<T>(o);
  const float part = wave_sum(active ? o * o : 0.f);
  if (lane == 0) sred[w] = part;
  __syncthreads();
  const float ms = (sred[0] + (blockDim.x > 64 ? sred[1] : 0.f)) / static_cast<float>(a.dv);
  if (active) {
    const float yv = round_as<T>(round_as<T>(o * rsqrtf(ms + a.norm_eps)) * nw) * round_as<T>(silu_fast(gt));
    st(static_cast<T *>(a.y) + b * a.y_sb + h * a.dv + tid, yv);
  }
}

template <typename T, int DK>
int launch_dk(const GdnDecodeArgs &a, int K, hipStream_t s) {
  const dim3 grid(a.H, a.B), block(a.dv <= 64 && 2 * DK <= 64 ? 64 : 128);
  switch (K) {
    case 2: gdn_decode_kernel<T, DK, 2><<<grid, block, 0, s>>>(a); break;
    case 3: gdn_decode_kernel<T, DK, 3><<<grid, block, 0, s>>>(a); break;
    case 4: gdn_decode_kernel<T, DK, 4><<<grid, block, 0, s>>>(a); break;
    case 5: gdn_decode_kernel<T, DK, 5><<<grid, block, 0, s>>>(a); break;
    default: return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_decode: conv kernel size must be in {2, 3, 4, 5}");
  }
  return check_launch("gdn_decode_kernel");
}

template <typename T>
int launch(const GdnDecodeArgs &a, int K, hipStream_t s) {
  switch (a.dk) {
    case 16: return launch_dk<T, 16>(a, K, s);
    case 32: return launch_dk<T, 32>(a, K, s);
    case 64: return launch_dk<T, 64>(a, K, s);
    default: return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_decode: dk must be 16, 32 or 64");
  }
}

}  // namespace

}  // namespace motif

extern "C" int motif_gdn_decode_fused(
    const void *proj, int64_t proj_sb, int q_off, int k_off, int v_off, int g_off, int a_off, int b_off,
    const void *wq, const void *wk, const void *wv, const void *tail_q, const void *tail_k, const void *tail_v,
    void *tail_q_out, void *tail_k_out, void *tail_v_out,
    const void *a_log, const void *dt_bias, const void *norm_weight, float norm_eps,
    const float *state, float *state_out, void *y, int64_t y_sb, int B, int H, int dk, int dv, int K, int dtype,
    void *stream) {
  using namespace motif;
  if (B < 0 || H <= 0 || dk <= 0 || dv <= 0) return set_error(MOTIF_ERR_INVALID, "gdn_decode: bad size");
  if (dv > 128) return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_decode: dv must be <= 128");
  if (dtype != MOTIF_F32 && dtype != MOTIF_BF16) return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_decode: dtype");
  if (B == 0) return MOTIF_OK;
  if (!proj || !wq || !wk || !wv || !tail_q || !tail_k || !tail_v || !tail_q_out || !tail_k_out || !tail_v_out ||
      !a_log || !dt_bias || !norm_weight || !state || !state_out || !y)
    return set_error(MOTIF_ERR_INVALID, "gdn_decode: NULL pointer");
  GdnDecodeArgs a;
  a.proj = proj; a.p_sb = proj_sb;
  a.q_off = q_off; a.k_off = k_off; a.v_off = v_off; a.g_off = g_off; a.a_off = a_off; a.b_off = b_off;
  a.wq = wq; a.wk = wk; a.wv = wv;
  a.tq = tail_q; a.tk = tail_k; a.tv = tail_v;
  a.oq = tail_q_out; a.ok = tail_k_out; a.ov = tail_v_out;
  a.a_log = a_log; a.dt_bias = dt_bias; a.norm_w = norm_weight; a.norm_eps = norm_eps;
  a.state = state; a.state_out = state_out; a.y = y; a.y_sb = y_sb;
  a.B = B; a.H = H; a.dk = dk; a.dv = dv;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == MOTIF_BF16 ? launch<bf16_t>(a, K, s) : launch<float>(a, K, s);
}
