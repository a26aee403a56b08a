// Elementwise stages around the hot path at prefill sizes, each one pass over HBM
// with 16-byte accesses, rounding to the activation dtype T where the reference's
// separate ops round:
//   gated_rms_norm_kernel  y[b, t, h*dv + e] = T(T(T(o * rsqrt(mean_e o^2 + eps)) * w[e]) *
//                            T(SiLU(gate[b, t, h*dv + e])))   for o = o[b, h, t, :]
//                          GatedRMSNorm over [o || gate] per head (motif/ops/rms_norm.py:530-553,
//                          the GDN layer's output norm, motif/block/attention/gdn_attn.py:206-209)
//                          without materialising the concatenation
//   swiglu_kernel          y = T(x[:, :I] * T(SiLU(x[:, I:])))   (motif/ops/swiglu.py:252-253)
//   add_fold_kernel        f = T(a + b); p_out = T(p + f)        (decoder f_h = attn + mlp and the
//                          block's running sum, motif/block/decoder.py:208-213)
//   gdn_gates_kernel       beta = T(sigmoid(b)), g = T(-T(exp(A_log)) * T(softplus(T(a + dt_bias))))
//                          per (token, head), written as [B, H, L] (motif/block/attention/
//                          gdn_attn.py:193-195; softplus threshold 20)
//   mul_sigmoid_kernel     y = T(x * T(sigmoid(g)))             (Chord output gate,
//                          motif/block/attention/chord_attn.py:254, :313)
//   residual_fold_kernel   f = T(T(a * T(sigmoid(g))) + b) (T(a + b) without a gate) and
//                          p = T(..T(T(c_0 + c_1) + c_2) .. + f) over the block's running-sum
//                          addends c_0 .. c_{n-1} not yet summed: a decoder's output and
//                          every add of the block's running sum since the last one that was
//                          stored, one add (and one rounding) each, in the reference's order
//                          (motif/block/decoder.py:205-213); without a / b only the sum of
//                          the c_j
#include "capi_internal.h"
#include "common.h"

namespace motif {

namespace {

template <typename T> struct V16;
template <> struct V16<bf16_t> {
  static constexpr int N = 8;
  __device__ static void unpack(uint4 u, float *x) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ static uint4 pack(const float *x) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(f32_to_bf16(x[2 * i])) | (static_cast<uint32_t>(f32_to_bf16(x[2 * i + 1])) << 16);
    return uint4{w[0], w[1], w[2], w[3]};
  }
  __device__ static float round(float v) { return bf16_to_f32(f32_to_bf16(v)); }
};
template <> struct V16<float> {
  static constexpr int N = 4;
  __device__ static void unpack(uint4 u, float *x) {
    x[0] = __uint_as_float(u.x); x[1] = __uint_as_float(u.y);
    x[2] = __uint_as_float(u.z); x[3] = __uint_as_float(u.w);
  }
  __device__ static uint4 pack(const float *x) {
    return uint4{__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3])};
  }
  __device__ static float round(float v) { return v; }
};

template <typename T> __device__ __forceinline__ uint4 ld16(const T *p) { return *reinterpret_cast<const uint4 *>(p); }
template <typename T> __device__ __forceinline__ void st16(T *p, uint4 v) { *reinterpret_cast<uint4 *>(p) = v; }

// ------------------------------------------------------------ gated RMSNorm
struct GNormArgs {
  const void *o; int64_t o_sb, o_sh, o_st;   // [B, H, L, dv]
  const void *g; int64_t g_sb, g_st;         // gate [B, L, H*dv]
  const void *w;                             // [dv]
  void *y; int64_t y_sb, y_st;               // [B, L, H*dv]
  float eps;
  int B, L, H, dv;
};

// LPR lanes per (b, t, h) row of dv elements (dv * sizeof(T) / 16, power of two <= 64).
template <typename T, int LPR>
__global__ void __launch_bounds__(256) gated_rms_norm_kernel(GNormArgs a) {
  constexpr int E = V16<T>::N;
  const int sub = threadIdx.x & (LPR - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (256 / LPR) + threadIdx.x / LPR;
  const int64_t nrows = static_cast<int64_t>(a.B) * a.L * a.H;
  const bool valid = row < nrows;
  const int64_t r = valid ? row : 0;
  const int h = static_cast<int>(r % a.H);
  const int64_t bt = r / a.H;
  const int t = static_cast<int>(bt % a.L), b = static_cast<int>(bt / a.L);
  float x[E], g[E], w[E];
  V16<T>::unpack(ld16(static_cast<const T *>(a.o) + b * a.o_sb + h * a.o_sh + int64_t(t) * a.o_st + sub * E), x);
  V16<T>::unpack(ld16(static_cast<const T *>(a.g) + b * a.g_sb + int64_t(t) * a.g_st + h * a.dv + sub * E), g);
  V16<T>::unpack(ld16(static_cast<const T *>(a.w) + sub * E), w);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss = fmaf(x[e], x[e], ss);
#pragma unroll
  for (int off = 1; off < LPR; off <<= 1) ss += __shfl_xor(ss, off, 64);
  if (!valid) return;
  const float rs = rsqrtf(ss / a.dv + a.eps);
  float y[E];
#pragma unroll
  for (int e = 0; e < E; ++e)
    y[e] = V16<T>::round(V16<T>::round(x[e] * rs) * w[e]) * V16<T>::round(silu_fast(g[e]));
  st16(static_cast<T *>(a.y) + b * a.y_sb + int64_t(t) * a.y_st + h * a.dv + sub * E, V16<T>::pack(y));
}

template <typename T>
int launch_gnorm(const GNormArgs &a, hipStream_t s) {
  const int lpr = a.dv * static_cast<int>(sizeof(T)) / 16;
  const int64_t rows = static_cast<int64_t>(a.B) * a.L * a.H;
  const dim3 grid(static_cast<unsigned>((rows * lpr + 255) / 256)), block(256);
  switch (lpr) {
    case 2: gated_rms_norm_kernel<T, 2><<<grid, block, 0, s>>>(a); break;
    case 4: gated_rms_norm_kernel<T, 4><<<grid, block, 0, s>>>(a); break;
    case 8: gated_rms_norm_kernel<T, 8><<<grid, block, 0, s>>>(a); break;
    case 16: gated_rms_norm_kernel<T, 16><<<grid, block, 0, s>>>(a); break;
    case 32: gated_rms_norm_kernel<T, 32><<<grid, block, 0, s>>>(a); break;
    case 64: gated_rms_norm_kernel<T, 64><<<grid, block, 0, s>>>(a); break;
    default: return set_error(MOTIF_ERR_UNSUPPORTED, "gated_rms_norm: dv * sizeof(T) must be 32..1024 bytes");
  }
  return check_launch("gated_rms_norm_kernel");
}

// ------------------------------------------------------------ SwiGLU / add-fold
struct EwArgs {
  const void *x; int64_t x_rs;      // swiglu: [M, 2I]; add_fold: a [M, N]
  const void *x2; int64_t x2_rs;    // add_fold: b
  const void *x3; int64_t x3_rs;    // add_fold: p (may be NULL)
  void *y; int64_t y_rs;            // swiglu: [M, I]; add_fold: f
  void *y2; int64_t y2_rs;          // add_fold: p_out
  int M, N;                         // rows, output columns
};

// One 16-byte chunk of an output row per thread.
template <typename T>
__global__ void __launch_bounds__(256) swiglu_kernel(EwArgs a) {
  constexpr int E = V16<T>::N;
  const int cpr = a.N / E;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(a.M) * cpr) return;
  const int64_t m = i / cpr;
  const int c = static_cast<int>(i - m * cpr) * E;
  const T *xr = static_cast<const T *>(a.x) + m * a.x_rs;
  float o[E], g[E], y[E];
  V16<T>::unpack(ld16(xr + c), o);
  V16<T>::unpack(ld16(xr + a.N + c), g);
#pragma unroll
  for (int e = 0; e < E; ++e) y[e] = o[e] * V16<T>::round(silu_fast(g[e]));
  st16(static_cast<T *>(a.y) + m * a.y_rs + c, V16<T>::pack(y));
}

template <typename T>
__global__ void __launch_bounds__(256) add_fold_kernel(EwArgs a) {
  constexpr int E = V16<T>::N;
  const int cpr = a.N / E;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(a.M) * cpr) return;
  const int64_t m = i / cpr;
  const int c = static_cast<int>(i - m * cpr) * E;
  float u[E], v[E], f[E];
  V16<T>::unpack(ld16(static_cast<const T *>(a.x) + m * a.x_rs + c), u);
  V16<T>::unpack(ld16(static_cast<const T *>(a.x2) + m * a.x2_rs + c), v);
#pragma unroll
  for (int e = 0; e < E; ++e) f[e] = V16<T>::round(u[e] + v[e]);
  st16(static_cast<T *>(a.y) + m * a.y_rs + c, V16<T>::pack(f));
  if (a.x3) {
    float p[E];
    V16<T>::unpack(ld16(static_cast<const T *>(a.x3) + m * a.x3_rs + c), p);
#pragma unroll
    for (int e = 0; e < E; ++e) p[e] = p[e] + f[e];
    st16(static_cast<T *>(a.y2) + m * a.y2_rs + c, V16<T>::pack(p));
  }
}

template <typename T> __device__ __forceinline__ float rnd(float v) { return v; }
template <> __device__ __forceinline__ float rnd<bf16_t>(float v) { return bf16_to_f32(f32_to_bf16(v)); }

struct GateArgs {
  const void *a, *b; int64_t a_sb, a_st, b_sb, b_st;   // [B, L, H] columns (unit head stride)
  const void *a_log, *dt_bias;                         // [H]
  void *beta, *g; int64_t o_sb, o_sh, o_st;            // [B, H, L]
  int B, L, H;
};

template <typename T>
__global__ void __launch_bounds__(256) gdn_gates_kernel(GateArgs p) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(p.B) * p.L * p.H) return;
  const int h = static_cast<int>(i % p.H);
  const int64_t bt = i / p.H;
  const int t = static_cast<int>(bt % p.L), b = static_cast<int>(bt / p.L);
  const float av = ld(static_cast<const T *>(p.a) + b * p.a_sb + int64_t(t) * p.a_st + h);
  const float bv = ld(static_cast<const T *>(p.b) + b * p.b_sb + int64_t(t) * p.b_st + h);
  const float x = rnd<T>(av + ld(static_cast<const T *>(p.dt_bias) + h));
  const float sp = rnd<T>(x > 20.f ? x : log1pf(expf(x)));
  const float A = rnd<T>(expf(ld(static_cast<const T *>(p.a_log) + h)));
  const int64_t o = b * p.o_sb + h * p.o_sh + int64_t(t) * p.o_st;
  st(static_cast<T *>(p.beta) + o, 1.f / (1.f + expf(-bv)));
  st(static_cast<T *>(p.g) + o, -A * sp);
}

template <typename T>
__global__ void __launch_bounds__(256) mul_sigmoid_kernel(EwArgs a) {
  constexpr int E = V16<T>::N;
  const int cpr = a.N / E;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(a.M) * cpr) return;
  const int64_t m = i / cpr;
  const int c = static_cast<int>(i - m * cpr) * E;
  float x[E], g[E];
  V16<T>::unpack(ld16(static_cast<const T *>(a.x) + m * a.x_rs + c), x);
  V16<T>::unpack(ld16(static_cast<const T *>(a.x2) + m * a.x2_rs + c), g);
#pragma unroll
  for (int e = 0; e < E; ++e) x[e] = x[e] * V16<T>::round(1.f / (1.f + expf(-g[e])));
  st16(static_cast<T *>(a.y) + m * a.y_rs + c, V16<T>::pack(x));
}

// ------------------------------------------------------------ residual fold
constexpr int kMaxChain = 8;
struct FoldArgs {
  const void *a; int64_t a_rs;   // branch output (NULL: only the sum of the c_j)
  const void *g; int64_t g_rs;   // gate pre-activation of a (may be NULL)
  const void *b; int64_t b_rs;   // second branch
  const void *c[kMaxChain]; int64_t c_rs[kMaxChain];
  int nc;                        // addends c_j (0: no running sum)
  void *f; int64_t f_rs;
  void *p; int64_t p_rs;
  int M, N;
};

// One 16-byte chunk of a row per thread; every load is issued before the arithmetic.
template <typename T, bool BRANCH, bool GATE>
__global__ void __launch_bounds__(256) residual_fold_kernel(FoldArgs a) {
  constexpr int E = V16<T>::N;
  const int cpr = a.N / E;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(a.M) * cpr) return;
  const int64_t m = i / cpr;
  const int c = static_cast<int>(i - m * cpr) * E;
  uint4 ra{}, rg{}, rb{};
  if (BRANCH) {
    ra = ld16(static_cast<const T *>(a.a) + m * a.a_rs + c);
    if (GATE) rg = ld16(static_cast<const T *>(a.g) + m * a.g_rs + c);
    rb = ld16(static_cast<const T *>(a.b) + m * a.b_rs + c);
  }
  uint4 rc[kMaxChain];
#pragma unroll
  for (int j = 0; j < kMaxChain; ++j)
    rc[j] = j < a.nc ? ld16(static_cast<const T *>(a.c[j]) + m * a.c_rs[j] + c) : uint4{0u, 0u, 0u, 0u};
  float f[E];
  if (BRANCH) {
    float x[E], y[E];
    V16<T>::unpack(ra, x);
    V16<T>::unpack(rb, y);
    if (GATE) {
      float g[E];
      V16<T>::unpack(rg, g);
#pragma unroll
      for (int e = 0; e < E; ++e) x[e] = V16<T>::round(x[e] * V16<T>::round(1.f / (1.f + expf(-g[e]))));
    }
#pragma unroll
    for (int e = 0; e < E; ++e) f[e] = V16<T>::round(x[e] + y[e]);
    st16(static_cast<T *>(a.f) + m * a.f_rs + c, V16<T>::pack(f));
  }
  if (a.nc == 0) return;
  float p[E];
  V16<T>::unpack(rc[0], p);
#pragma unroll
  for (int j = 1; j < kMaxChain; ++j) {
    if (j >= a.nc) break;
    float q[E];
    V16<T>::unpack(rc[j], q);
#pragma unroll
    for (int e = 0; e < E; ++e) p[e] = V16<T>::round(p[e] + q[e]);
  }
  if (BRANCH) {
#pragma unroll
    for (int e = 0; e < E; ++e) p[e] = p[e] + f[e];
  }
  st16(static_cast<T *>(a.p) + m * a.p_rs + c, V16<T>::pack(p));
}

template <typename T>
int launch_fold(const FoldArgs &a, dim3 grid, hipStream_t s) {
  if (!a.a) residual_fold_kernel<T, false, false><<<grid, 256, 0, s>>>(a);
  else if (a.g) residual_fold_kernel<T, true, true><<<grid, 256, 0, s>>>(a);
  else residual_fold_kernel<T, true, false><<<grid, 256, 0, s>>>(a);
  return check_launch("residual_fold_kernel");
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

}  // namespace motif

extern "C" int motif_gated_rms_norm(const void *o, int64_t o_sb, int64_t o_sh, int64_t o_st, const void *gate,
                                    int64_t g_sb, int64_t g_st, const void *weight, float eps, void *y,
                                    int64_t y_sb, int64_t y_st, int B, int L, int H, int dv, int dtype,
                                    void *stream) {
  using namespace motif;
  if (B < 0 || L < 0 || H <= 0 || dv <= 0) return set_error(MOTIF_ERR_INVALID, "gated_rms_norm: bad size");
  if (!o || !gate || !weight || !y) return set_error(MOTIF_ERR_INVALID, "gated_rms_norm: NULL pointer");
  if (dtype != MOTIF_F32 && dtype != MOTIF_BF16) return set_error(MOTIF_ERR_UNSUPPORTED, "gated_rms_norm: dtype");
  const int vec = dtype == MOTIF_BF16 ? 8 : 4;
  if (!aligned16(o) || !aligned16(gate) || !aligned16(weight) || !aligned16(y) ||
      ((o_sb | o_sh | o_st | g_sb | g_st | y_sb | y_st | dv) % vec))
    return set_error(MOTIF_ERR_UNSUPPORTED, "gated_rms_norm: rows must be 16-byte aligned");
  if (B == 0 || L == 0) return MOTIF_OK;
  GNormArgs a{o, o_sb, o_sh, o_st, gate, g_sb, g_st, weight, y, y_sb, y_st, eps, B, L, H, dv};
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == MOTIF_BF16 ? launch_gnorm<bf16_t>(a, s) : launch_gnorm<float>(a, s);
}

extern "C" int motif_swiglu(const void *x, int64_t x_rs, void *y, int64_t y_rs, int M, int I, int dtype,
                            void *stream) {
  using namespace motif;
  if (M < 0 || I <= 0) return set_error(MOTIF_ERR_INVALID, "swiglu: bad size");
  if (!x || !y) return set_error(MOTIF_ERR_INVALID, "swiglu: NULL pointer");
  if (dtype != MOTIF_F32 && dtype != MOTIF_BF16) return set_error(MOTIF_ERR_UNSUPPORTED, "swiglu: dtype");
  const int vec = dtype == MOTIF_BF16 ? 8 : 4;
  if (!aligned16(x) || !aligned16(y) || ((x_rs | y_rs | I) % vec))
    return set_error(MOTIF_ERR_UNSUPPORTED, "swiglu: rows must be 16-byte aligned");
  if (M == 0) return MOTIF_OK;
  EwArgs a{x, x_rs, nullptr, 0, nullptr, 0, y, y_rs, nullptr, 0, M, I};
  const int64_t n = static_cast<int64_t>(M) * (I / vec);
  const dim3 grid(static_cast<unsigned>((n + 255) / 256)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MOTIF_BF16) swiglu_kernel<bf16_t><<<grid, block, 0, s>>>(a);
  else swiglu_kernel<float><<<grid, block, 0, s>>>(a);
  return check_launch("swiglu_kernel");
}

extern "C" int motif_add_fold(const void *a_, int64_t a_rs, const void *b_, int64_t b_rs, const void *p,
                              int64_t p_rs, void *f, int64_t f_rs, void *p_out, int64_t po_rs, int M, int N,
                              int dtype, void *stream) {
  using namespace motif;
  if (M < 0 || N <= 0) return set_error(MOTIF_ERR_INVALID, "add_fold: bad size");
  if (!a_ || !b_ || !f || (p && !p_out)) return set_error(MOTIF_ERR_INVALID, "add_fold: NULL pointer");
  if (dtype != MOTIF_F32 && dtype != MOTIF_BF16) return set_error(MOTIF_ERR_UNSUPPORTED, "add_fold: dtype");
  const int vec = dtype == MOTIF_BF16 ? 8 : 4;
  if (!aligned16(a_) || !aligned16(b_) || !aligned16(f) || (p && (!aligned16(p) || !aligned16(p_out))) ||
      ((a_rs | b_rs | f_rs | (p ? (p_rs | po_rs) : 0) | N) % vec))
    return set_error(MOTIF_ERR_UNSUPPORTED, "add_fold: rows must be 16-byte aligned");
  if (M == 0) return MOTIF_OK;
  EwArgs a{a_, a_rs, b_, b_rs, p, p_rs, f, f_rs, p_out, po_rs, M, N};
  const int64_t n = static_cast<int64_t>(M) * (N / vec);
  const dim3 grid(static_cast<unsigned>((n + 255) / 256)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MOTIF_BF16) add_fold_kernel<bf16_t><<<grid, block, 0, s>>>(a);
  else add_fold_kernel<float><<<grid, block, 0, s>>>(a);
  return check_launch("add_fold_kernel");
}

extern "C" int motif_gdn_gates(const void *a, int64_t a_sb, int64_t a_st, const void *b, int64_t b_sb,
                               int64_t b_st, const void *a_log, const void *dt_bias, void *beta, void *g,
                               int64_t o_sb, int64_t o_sh, int64_t o_st, int B, int L, int H, int dtype,
                               void *stream) {
  using namespace motif;
  if (B < 0 || L < 0 || H <= 0) return set_error(MOTIF_ERR_INVALID, "gdn_gates: bad size");
  if (!a || !b || !a_log || !dt_bias || !beta || !g) return set_error(MOTIF_ERR_INVALID, "gdn_gates: NULL pointer");
  if (dtype != MOTIF_F32 && dtype != MOTIF_BF16) return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_gates: dtype");
  if (B == 0 || L == 0) return MOTIF_OK;
  GateArgs p{a, b, a_sb, a_st, b_sb, b_st, a_log, dt_bias, beta, g, o_sb, o_sh, o_st, B, L, H};
  const int64_t n = static_cast<int64_t>(B) * L * H;
  const dim3 grid(static_cast<unsigned>((n + 255) / 256)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MOTIF_BF16) gdn_gates_kernel<bf16_t><<<grid, block, 0, s>>>(p);
  else gdn_gates_kernel<float><<<grid, block, 0, s>>>(p);
  return check_launch("gdn_gates_kernel");
}

extern "C" int motif_mul_sigmoid(const void *x, int64_t x_rs, const void *g, int64_t g_rs, void *y, int64_t y_rs,
                                 int M, int N, int dtype, void *stream) {
  using namespace motif;
  if (M < 0 || N <= 0) return set_error(MOTIF_ERR_INVALID, "mul_sigmoid: bad size");
  if (!x || !g || !y) return set_error(MOTIF_ERR_INVALID, "mul_sigmoid: NULL pointer");
  if (dtype != MOTIF_F32 && dtype != MOTIF_BF16) return set_error(MOTIF_ERR_UNSUPPORTED, "mul_sigmoid: dtype");
  const int vec = dtype == MOTIF_BF16 ? 8 : 4;
  if (!aligned16(x) || !aligned16(g) || !aligned16(y) || ((x_rs | g_rs | y_rs | N) % vec))
    return set_error(MOTIF_ERR_UNSUPPORTED, "mul_sigmoid: rows must be 16-byte aligned");
  if (M == 0) return MOTIF_OK;
  EwArgs a{x, x_rs, g, g_rs, nullptr, 0, y, y_rs, nullptr, 0, M, N};
  const int64_t n = static_cast<int64_t>(M) * (N / vec);
  const dim3 grid(static_cast<unsigned>((n + 255) / 256)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MOTIF_BF16) mul_sigmoid_kernel<bf16_t><<<grid, block, 0, s>>>(a);
  else mul_sigmoid_kernel<float><<<grid, block, 0, s>>>(a);
  return check_launch("mul_sigmoid_kernel");
}

extern "C" int motif_residual_fold(const void *a_, int64_t a_rs, const void *g, int64_t g_rs, const void *b_,
                                   int64_t b_rs, const void *const *chain, const int64_t *chain_rs, int nchain,
                                   void *f, int64_t f_rs, void *p, int64_t p_rs, int M, int N, int dtype,
                                   void *stream) {
  using namespace motif;
  if (M < 0 || N <= 0) return set_error(MOTIF_ERR_INVALID, "residual_fold: bad size");
  if (nchain < 0 || nchain > kMaxChain) return set_error(MOTIF_ERR_UNSUPPORTED, "residual_fold: 0 to 8 addends");
  if (a_ ? (!b_ || !f) : (nchain < 2 || g || b_ || f))
    return set_error(MOTIF_ERR_INVALID, "residual_fold: a and b together (with f), or only two or more addends");
  if (nchain > 0 && (!chain || !chain_rs || !p)) return set_error(MOTIF_ERR_INVALID, "residual_fold: NULL pointer");
  if (dtype != MOTIF_F32 && dtype != MOTIF_BF16) return set_error(MOTIF_ERR_UNSUPPORTED, "residual_fold: dtype");
  const int vec = dtype == MOTIF_BF16 ? 8 : 4;
  FoldArgs a{};
  a.a = a_; a.a_rs = a_rs; a.g = a_ ? g : nullptr; a.g_rs = g_rs; a.b = b_; a.b_rs = b_rs;
  a.nc = nchain; a.f = f; a.f_rs = f_rs; a.p = nchain > 0 ? p : nullptr; a.p_rs = p_rs; a.M = M; a.N = N;
  bool ok = N % vec == 0;
  if (a_) ok = ok && aligned16(a_) && aligned16(b_) && aligned16(f) && (a_rs | b_rs | f_rs) % vec == 0 &&
               (!a.g || (aligned16(g) && g_rs % vec == 0));
  for (int j = 0; j < nchain; ++j) {
    if (!chain[j]) return set_error(MOTIF_ERR_INVALID, "residual_fold: NULL addend");
    a.c[j] = chain[j];
    a.c_rs[j] = chain_rs[j];
    ok = ok && aligned16(chain[j]) && chain_rs[j] % vec == 0;
  }
  if (nchain > 0) ok = ok && aligned16(p) && p_rs % vec == 0;
  if (!ok) return set_error(MOTIF_ERR_UNSUPPORTED, "residual_fold: rows must be 16-byte aligned");
  if (M == 0) return MOTIF_OK;
  const int64_t n = static_cast<int64_t>(M) * (N / vec);
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == MOTIF_BF16 ? launch_fold<bf16_t>(a, grid, s) : launch_fold<float>(a, grid, s);
}
