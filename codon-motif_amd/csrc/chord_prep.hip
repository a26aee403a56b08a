// ChordAttention input stage for a preallocated KV cache, fused: from the fused
// q | k | v projection rows, per head
//   q_out[b, h, t]              = RMSNorm(q_h; q_norm.weight)
//   k_cache[b, g, pos + t]      = RMSNorm(k_g; k_norm.weight)
//   v_cache[b, g, pos + t]      = v_g
// with RMSNorm as the reference computes it (motif/ops/rms_norm.py:481-486):
// T(x * rsqrt(mean(x^2) + eps)) * weight, the product rounded to T.  Replaces
// motif/block/attention/chord_attn.py:255-265 (q_norm(q_proj h), k_norm(k_proj h),
// v_proj h) and the cache append motif/model/cache.py:170-215.
//
// One group of D * sizeof(T) / 16 lanes per (token, head) row, 16-byte loads and
// stores; the sum of squares is a butterfly inside the group.
#include "capi_internal.h"
#include "common.h"

namespace motif {

namespace {

struct PrepArgs {
  const void *proj; int64_t p_sb, p_st;   // [B, L, ncols]
  int q_off, k_off, v_off;
  const void *qw, *kw;                    // [D]
  float eps;
  void *q; int64_t q_sb, q_sh, q_st;      // [B, H, L, D]
  void *kc; int64_t k_sb, k_sh, k_st;     // [B, Hkv, cap, D]
  void *vc; int64_t v_sb, v_sh, v_st;
  int *len_dev;                           // host position: optional, set to pos + L;
                                          // device position (pos < 0): read, not written
  int pos, capacity, B, L, H, Hkv, D;
};

template <typename T> struct Vec;
template <> struct Vec<bf16_t> {
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
template <> struct Vec<float> {
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

// LPR lanes per row (D * sizeof(T) / 16, a power of two <= 64).
template <typename T, int LPR>
__global__ void __launch_bounds__(256) chord_prep_kernel(PrepArgs a) {
  constexpr int E = Vec<T>::N;
  const int lane = threadIdx.x & 63;
  const int sub = lane & (LPR - 1);
  const int rows_per_block = 256 / LPR;
  const int heads = a.H + 2 * a.Hkv;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * rows_per_block + threadIdx.x / LPR;
  const int64_t nrows = static_cast<int64_t>(a.B) * a.L * heads;
  const bool valid = row < nrows;
  const int64_t r = valid ? row : 0;
  const int hh = static_cast<int>(r % heads);
  const int64_t bt = r / heads;
  const int t = static_cast<int>(bt % a.L), b = static_cast<int>(bt / a.L);

  // column of this row's head in the projection
  int col;
  if (hh < a.H) col = a.q_off + hh * a.D;
  else if (hh < a.H + a.Hkv) col = a.k_off + (hh - a.H) * a.D;
  else col = a.v_off + (hh - a.H - a.Hkv) * a.D;
  const T *src = static_cast<const T *>(a.proj) + b * a.p_sb + static_cast<int64_t>(t) * a.p_st + col;
  // the row, its norm-weight piece (v rows load the q one and ignore it) and the device
  // cache cursor are requested together, ahead of any use
  const uint4 xraw = *reinterpret_cast<const uint4 *>(src + sub * E);
  const uint4 wraw = *reinterpret_cast<const uint4 *>(static_cast<const T *>(hh >= a.H && hh < a.H + a.Hkv ? a.kw : a.qw) +
                                                      sub * E);
  // the cache position of this launch: the host's, or the device cursor (the decode
  // kernel that follows reads the same cursor and advances it)
  const int pos = a.pos >= 0 ? a.pos : __builtin_amdgcn_readfirstlane(*a.len_dev);
  float x[E];
  Vec<T>::unpack(xraw, x);

  const bool is_v = hh >= a.H + a.Hkv;
  // sum of squares over the row's LPR lanes (every lane joins the butterfly)
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss = fmaf(x[e], x[e], ss);
#pragma unroll
  for (int off = 1; off < LPR; off <<= 1) ss += __shfl_xor(ss, off, 64);
  if (!valid) return;

  if (hh >= a.H && pos + t >= a.capacity) return;  // never write past the slab
  T *dst;
  if (hh < a.H) {
    dst = static_cast<T *>(a.q) + b * a.q_sb + hh * a.q_sh + static_cast<int64_t>(t) * a.q_st;
  } else if (!is_v) {
    dst = static_cast<T *>(a.kc) + b * a.k_sb + (hh - a.H) * a.k_sh + static_cast<int64_t>(pos + t) * a.k_st;
  } else {
    dst = static_cast<T *>(a.vc) + b * a.v_sb + (hh - a.H - a.Hkv) * a.v_sh + static_cast<int64_t>(pos + t) * a.v_st;
  }
  if (!is_v) {
    const float rs = rsqrtf(ss / a.D + a.eps);
    float w[E];
    Vec<T>::unpack(wraw, w);
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = Vec<T>::round(x[e] * rs) * w[e];
  }
  *reinterpret_cast<uint4 *>(dst + sub * E) = Vec<T>::pack(x);
  if (a.pos >= 0 && a.len_dev && row == 0) *a.len_dev = a.pos + a.L;
}

template <typename T>
int launch(const PrepArgs &a, hipStream_t s) {
  const int lpr = a.D * static_cast<int>(sizeof(T)) / 16;
  const int64_t rows = static_cast<int64_t>(a.B) * a.L * (a.H + 2 * a.Hkv);
  const int64_t blocks = (rows * lpr + 255) / 256;
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  switch (lpr) {
    case 4: chord_prep_kernel<T, 4><<<grid, block, 0, s>>>(a); break;
    case 8: chord_prep_kernel<T, 8><<<grid, block, 0, s>>>(a); break;
    case 16: chord_prep_kernel<T, 16><<<grid, block, 0, s>>>(a); break;
    case 32: chord_prep_kernel<T, 32><<<grid, block, 0, s>>>(a); break;
    default: return set_error(MOTIF_ERR_UNSUPPORTED, "chord_prep: head_dim must be 32..256 bytes / 16");
  }
  return check_launch("chord_prep_kernel");
}

}  // namespace

}  // namespace motif

extern "C" int motif_chord_qkv_prep(const void *proj, int64_t p_sb, int64_t p_st, int q_off, int k_off, int v_off,
                                    const void *q_norm_weight, const void *k_norm_weight, float eps,
                                    void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                                    void *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                    void *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_st,
                                    int *length_dev, int pos, int capacity, int B, int L, int H, int Hkv,
                                    int D, int dtype, void *stream) {
  using namespace motif;
  if (B < 0 || L < 0 || H <= 0 || Hkv <= 0 || D <= 0 || H % Hkv || capacity < 0)
    return set_error(MOTIF_ERR_INVALID, "chord_prep: bad size");
  if (pos < 0 && !length_dev)
    return set_error(MOTIF_ERR_INVALID, "chord_prep: a device position (pos < 0) needs length_dev");
  if (pos >= 0 && pos + L > capacity)
    return set_error(MOTIF_ERR_INVALID, "chord_prep: pos + L exceeds the cache capacity");
  if (!proj || !q_norm_weight || !k_norm_weight || !q || !k_cache || !v_cache)
    return set_error(MOTIF_ERR_INVALID, "chord_prep: NULL pointer");
  if (dtype != MOTIF_F32 && dtype != MOTIF_BF16) return set_error(MOTIF_ERR_UNSUPPORTED, "chord_prep: dtype");
  const int esz = dtype == MOTIF_BF16 ? 2 : 4, vec = 16 / esz;
  const uintptr_t align = reinterpret_cast<uintptr_t>(proj) | reinterpret_cast<uintptr_t>(q_norm_weight) |
                          reinterpret_cast<uintptr_t>(k_norm_weight) | reinterpret_cast<uintptr_t>(q) |
                          reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache);
  const int64_t strides = p_sb | p_st | q_off | k_off | v_off | q_sb | q_sh | q_st | k_sb | k_sh | k_st | v_sb |
                          v_sh | v_st | D;
  if ((align & 15) || (strides % vec))
    return set_error(MOTIF_ERR_UNSUPPORTED, "chord_prep: rows must be 16-byte aligned");
  PrepArgs a;
  a.proj = proj; a.p_sb = p_sb; a.p_st = p_st;
  a.q_off = q_off; a.k_off = k_off; a.v_off = v_off;
  a.qw = q_norm_weight; a.kw = k_norm_weight; a.eps = eps;
  a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.kc = k_cache; a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.vc = v_cache; a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.len_dev = length_dev; a.pos = pos; a.capacity = capacity;
  a.B = B; a.L = L; a.H = H; a.Hkv = Hkv; a.D = D;
  if (B == 0 || L == 0) return MOTIF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == MOTIF_BF16 ? launch<bf16_t>(a, s) : launch<float>(a, s);
}
