// Short causal depthwise conv + SiLU (the GDN q/k/v front end) for gfx950,
// optionally followed by the per-head L2 normalisation and scale of q / k.
//
// One thread owns one channel over a run of timesteps and slides a K-1 window in
// registers; a wavefront covers 64 consecutive channels of one timestep (coalesced).
// Each run is processed 16 timesteps at a time with all 16 loads issued before the
// arithmetic.  With HD > 0 a head is HD consecutive lanes: the sum of squares is a
// butterfly over those lanes, y / max(||y||, 1e-12) * scale (F.normalize semantics).
// Every intermediate the reference layer rounds to the activation type (conv output,
// SiLU, the norm, the quotient, q's scaled value) is rounded here at the same point.
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
  int hd;    // vector kernel: head L2 normalisation on (HD channels a head) or off (0)
};

// Up to three independent conv problems (the GDN q, k, v front ends) in one launch of
// the vector kernel: blocks [start[p], start[p + 1]) serve problem p.
struct ConvGroup {
  ConvArgs a[3];
  int start[3];
  int n;
};

constexpr int kConvStep = 16;  // timesteps per batch of loads (scalar kernel)
constexpr int kVecStep = 4;    // timesteps per thread (vector kernel)

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

  const T *x = static_cast<const T *>(a.x) + batch * a.x_sb + int64_t(t_begin) * a.x_st;
  T *y = static_cast<T *>(a.y) + batch * a.y_sb + int64_t(t_begin) * a.y_st + dc;
  const T *w = static_cast<const T *>(a.w) + dc * K;
  // Range-checked buffers over this sequence's rows and this batch row's tail_in:
  // positions before the start or past the end read as zeros (packed sequences and
  // a NULL tail_in get zero-sized tail buffers), so every load is unconditional.
  const buf_t xbuf = make_buf(x, len > 0 ? static_cast<uint32_t>(((len - 1) * a.x_st + a.D) * sizeof(T)) : 0u);
  const bool has_tail = a.cu == nullptr && a.tail_in;
  const buf_t tbuf = make_buf(has_tail ? static_cast<const T *>(a.tail_in) + static_cast<size_t>(batch) * a.D * (K - 1)
                                       : static_cast<const T *>(a.x),
                              has_tail ? static_cast<uint32_t>(a.D * (K - 1) * sizeof(T)) : 0u);
  auto xat = [&](int pos) { return buf_ld<T>(xbuf, static_cast<uint32_t>(pos * a.x_st + dc)); };

  // Issue everything the first block needs at once: weights, tail, window, 16 inputs.
  float wr[K], tv[K - 1], xw[K - 1], xs[kConvStep];
#pragma unroll
  for (int r = 0; r < K; ++r) wr[r] = ld(w + r);
#pragma unroll
  for (int u = 0; u < K - 1; ++u) tv[u] = buf_ld<T>(tbuf, dc * (K - 1) + u);
#pragma unroll
  for (int r = 0; r < K - 1; ++r) xw[r] = xat(t_lo - (K - 1) + r);
#pragma unroll
  for (int i = 0; i < kConvStep; ++i) xs[i] = xat(t_lo + i);
  __builtin_amdgcn_sched_barrier(0);  // keep the loads above as one batch

  // Window = inputs at positions t_lo-K+1 .. t_lo-1 (before the start: tail entries);
  // tail_keep = the entries of the last K-1 positions that come from tail_in (taken
  // before anything is written, as tail_out may alias tail_in).
  float win[K - 1], tail_keep[K - 1];
  const bool last_run = t_hi == len;
#pragma unroll
  for (int r = 0; r < K - 1; ++r) {
    const int pos = t_lo - (K - 1) + r, pk = len - (K - 1) + r;
    float tw = 0.f, tk = 0.f;
#pragma unroll
    for (int u = 0; u < K - 1; ++u) {  // tail entry pos + K - 1 (static register index)
      tw = (pos + K - 1 == u) ? tv[u] : tw;
      tk = (pk + K - 1 == u) ? tv[u] : tk;
    }
    win[r] = active ? (pos >= 0 ? xw[r] : tw) : 0.f;
    tail_keep[r] = (active && pk < 0) ? tk : 0.f;
  }
#pragma unroll
  for (int r = 0; r < K; ++r) wr[r] = active ? wr[r] : 0.f;

  for (int t0 = t_lo; t0 < t_hi; t0 += kConvStep) {
    if (t0 != t_lo) {
#pragma unroll
      for (int i = 0; i < kConvStep; ++i) xs[i] = xat(t0 + i);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < kConvStep; ++i) {
      if (!active) xs[i] = 0.f;
      float acc = wr[K - 1] * xs[i];
#pragma unroll
      for (int r = 0; r < K - 1; ++r) acc = fmaf(wr[r], win[r], acc);
      float v = gdn_conv_act<T>(acc);
      if (HD > 0) {
        float ss = v * v;
#pragma unroll
        for (int off = 1; off < HD; off <<= 1) ss += __shfl_xor(ss, off, 64);
        v = gdn_normalized<T>(v, gdn_norm_inv<T>(ss), a.scale);
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
      const float xv = xat(pos);
      st(to + r, pos >= 0 ? xv : tail_keep[r]);
    }
  }
}

// Vector form for row-contiguous 16-byte-aligned channels: one thread owns E = 16 /
// sizeof(T) consecutive channels over kVecStep timesteps (16-byte loads and stores;
// few timesteps per thread keep enough waves in flight to cover the load latency).  With
// HD > 0 a head is HD / E consecutive lanes.  Same arithmetic as the scalar kernel.
template <typename T> struct Vec16;
template <> struct Vec16<bf16_t> {
  static constexpr int E = 8;
  __device__ static void unpack(const uint4 &u, float *x) {
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
};
template <> struct Vec16<float> {
  static constexpr int E = 4;
  __device__ static void unpack(const uint4 &u, float *x) {
    x[0] = __uint_as_float(u.x); x[1] = __uint_as_float(u.y); x[2] = __uint_as_float(u.z); x[3] = __uint_as_float(u.w);
  }
  __device__ static uint4 pack(const float *x) {
    return uint4{__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3])};
  }
};

template <typename T, int K, int HD>
__global__ void __launch_bounds__(256) short_conv_silu_vec_kernel(ConvGroup grp) {
  constexpr int E = Vec16<T>::E;
  constexpr int G = HD / E;  // lanes per head (HD > 0)
  // this block's problem (selects on uniform values: no indexed copy of the group)
  const int bx = blockIdx.x;
  const int p = (grp.n > 2 && bx >= grp.start[2]) ? 2 : (grp.n > 1 && bx >= grp.start[1]) ? 1 : 0;
  const ConvArgs a = p == 2 ? grp.a[2] : p == 1 ? grp.a[1] : grp.a[0];
  const int blk = bx - (p == 2 ? grp.start[2] : p == 1 ? grp.start[1] : 0);
  const bool norm = HD > 0 && a.hd > 0;
  const int nc = a.D / E;
  const int idx = blk * 256 + threadIdx.x;
  const int sq = blockIdx.y;
  const int c = idx % nc, tb = idx / nc;
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
  const int t_lo = tb * kVecStep;
  // Head groups share tb, so a whole group is in or out together.
  if (t_lo >= len && !(tb == 0 && len == 0)) return;
  const int t_hi = min(len, t_lo + kVecStep);
  const int d0 = c * E;

  const T *x = static_cast<const T *>(a.x) + batch * a.x_sb + int64_t(t_begin) * a.x_st;
  T *y = static_cast<T *>(a.y) + batch * a.y_sb + int64_t(t_begin) * a.y_st + d0;
  const buf_t xbuf = make_buf(x, len > 0 ? static_cast<uint32_t>(((len - 1) * a.x_st + a.D) * sizeof(T)) : 0u);
  const bool has_tail = a.cu == nullptr && a.tail_in;
  const T *tail0 = has_tail ? static_cast<const T *>(a.tail_in) + (static_cast<size_t>(batch) * a.D + d0) * (K - 1)
                            : nullptr;

  uint4 raw[K - 1 + kVecStep];
#pragma unroll
  for (int i = 0; i < K - 1 + kVecStep; ++i)
    raw[i] = buf_ld16(xbuf, static_cast<uint32_t>(((t_lo - (K - 1) + i) * a.x_st + d0) * sizeof(T)));
  // The E channels' taps (E * K contiguous values = K 16-byte pieces).
  float wr[E][K];
  {
    const T *wp = static_cast<const T *>(a.w) + d0 * K;
    float wf[E * K];
#pragma unroll
    for (int j = 0; j < K; ++j) Vec16<T>::unpack(*reinterpret_cast<const uint4 *>(wp + j * E), wf + j * E);
#pragma unroll
    for (int e = 0; e < E; ++e)
#pragma unroll
      for (int r = 0; r < K; ++r) wr[e][r] = wf[e * K + r];
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the loads above as one batch

  // window: positions t_lo-K+1 .. t_lo-1 (rows before the sequence start read 0; with
  // a cached tail the first run takes them from tail_in)
  float win[K - 1][E];
#pragma unroll
  for (int r = 0; r < K - 1; ++r) Vec16<T>::unpack(raw[r], win[r]);
  if (has_tail && t_lo < K - 1) {
#pragma unroll
    for (int r = 0; r < K - 1; ++r) {
      const int u = t_lo + r;  // tail entry of position t_lo - (K - 1) + r
      if (u < K - 1) {
#pragma unroll
        for (int e = 0; e < E; ++e) win[r][e] = ld(tail0 + e * (K - 1) + u);
      }
    }
  }
  const bool last_run = t_hi == len;

#pragma unroll
  for (int i = 0; i < kVecStep; ++i) {
    float xt[E], v[E];
    Vec16<T>::unpack(raw[K - 1 + i], xt);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float acc = wr[e][K - 1] * xt[e];
#pragma unroll
      for (int r = 0; r < K - 1; ++r) acc = fmaf(wr[e][r], win[r][e], acc);
      v[e] = gdn_conv_act<T>(acc);
      ss = fmaf(v[e], v[e], ss);
#pragma unroll
      for (int r = 0; r < K - 2; ++r) win[r][e] = win[r + 1][e];
      win[K - 2][e] = xt[e];
    }
    if (norm) {
#pragma unroll
      for (int off = 1; off < G; off <<= 1) ss += __shfl_xor(ss, off, 64);
      const float inv = gdn_norm_inv<T>(ss);
#pragma unroll
      for (int e = 0; e < E; ++e) v[e] = gdn_normalized<T>(v[e], inv, a.scale);
    }
    if (t_lo + i < t_hi) *reinterpret_cast<uint4 *>(y + int64_t(t_lo + i) * a.y_st) = Vec16<T>::pack(v);
  }

  if (last_run && a.tail_out) {
    T *to = static_cast<T *>(a.tail_out) + (static_cast<size_t>(sq) * a.D + d0) * (K - 1);
#pragma unroll
    for (int r = 0; r < K - 1; ++r) {
      const int pos = len - (K - 1) + r;
      float xv[E];
      Vec16<T>::unpack(buf_ld16(xbuf, static_cast<uint32_t>((pos * a.x_st + d0) * sizeof(T))), xv);
      // positions before the sequence start keep the incoming tail entries (0 without one)
#pragma unroll
      for (int e = 0; e < E; ++e)
        st(to + e * (K - 1) + r, pos >= 0 ? xv[e] : has_tail ? ld(tail0 + e * (K - 1) + pos + K - 1) : 0.f);
    }
  }
}

template <typename T, int HD>
static int launch_conv_group(ConvGroup g, int K, int nseq, int max_len, hipStream_t s) {
  const int ntb = max(1, (max_len + kVecStep - 1) / kVecStep);
  int64_t blocks = 0;
  for (int p = 0; p < g.n; ++p) {
    g.start[p] = static_cast<int>(blocks);
    blocks += (static_cast<int64_t>(g.a[p].D / Vec16<T>::E) * ntb + 255) / 256;
  }
  if (blocks > (int64_t(1) << 30)) return set_error(MOTIF_ERR_UNSUPPORTED, "short_conv_silu: grid too large");
  const dim3 grid(static_cast<unsigned>(blocks), nseq), block(256);
  switch (K) {
    case 2: short_conv_silu_vec_kernel<T, 2, HD><<<grid, block, 0, s>>>(g); break;
    case 3: short_conv_silu_vec_kernel<T, 3, HD><<<grid, block, 0, s>>>(g); break;
    case 4: short_conv_silu_vec_kernel<T, 4, HD><<<grid, block, 0, s>>>(g); break;
    case 5: short_conv_silu_vec_kernel<T, 5, HD><<<grid, block, 0, s>>>(g); break;
    default: return set_error(MOTIF_ERR_UNSUPPORTED, "short_conv_silu: K must be in {2, 3, 4, 5}");
  }
  return check_launch("short_conv_silu_vec_kernel");
}

template <typename T, int HD>
static int launch_conv_vec(ConvArgs a, int K, int nseq, int max_len, hipStream_t s) {
  ConvGroup g;
  a.hd = HD;
  g.a[0] = a;
  g.n = 1;
  return launch_conv_group<T, HD>(g, K, nseq, max_len, s);
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
  constexpr int E = Vec16<T>::E;
  const bool aliased = a.tail_out != nullptr && a.tail_out == a.tail_in;
  const bool vec = !aliased && a.D % E == 0 && ((a.x_sb | a.x_st | a.y_sb | a.y_st) % E) == 0 &&
                   ((reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.y) |
                     reinterpret_cast<uintptr_t>(a.w) | reinterpret_cast<uintptr_t>(a.tail_in)) & 15) == 0 &&
                   head_dim % E == 0;
  if (vec) {
    switch (head_dim) {
      case 0: return launch_conv_vec<T, 0>(a, K, nseq, max_len, s);
      case 16: return launch_conv_vec<T, 16>(a, K, nseq, max_len, s);
      case 32: return launch_conv_vec<T, 32>(a, K, nseq, max_len, s);
      case 64: return launch_conv_vec<T, 64>(a, K, nseq, max_len, s);
    }
  }
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
      if (!tail_in) return zero_async(tail_out, n, static_cast<hipStream_t>(stream));
      hipError_t e = hipMemcpyAsync(tail_out, tail_in, n, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream));
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

template <typename T>
static int launch_multi(ConvGroup g, int K, int nseq, int max_len, int hd, hipStream_t s) {
  switch (hd) {
    case 0: return launch_conv_group<T, 0>(g, K, nseq, max_len, s);
    case 16: return launch_conv_group<T, 16>(g, K, nseq, max_len, s);
    case 32: return launch_conv_group<T, 32>(g, K, nseq, max_len, s);
    case 64: return launch_conv_group<T, 64>(g, K, nseq, max_len, s);
  }
  return set_error(MOTIF_ERR_UNSUPPORTED, "short_conv_silu_multi: head_dim must be 0, 16, 32 or 64");
}

extern "C" int motif_short_conv_silu_multi(
    int n, const void *const *x, const int64_t *x_sb, const int64_t *x_st,
    const void *const *weight, const void *const *tail_in, void *const *tail_out,
    void *const *y, const int64_t *y_sb, const int64_t *y_st,
    const int *D, const int *head_dim, const float *scale,
    int B, int L, int K,
    const int32_t *cu_seqlens, int nseq, int max_seqlen,
    int dtype, void *stream) {
  if (n < 1 || n > 3 || !x || !x_sb || !x_st || !weight || !tail_in || !tail_out || !y || !y_sb || !y_st || !D ||
      !head_dim || !scale)
    return set_error(MOTIF_ERR_INVALID, "short_conv_silu_multi: n must be 1..3 and the arrays non-NULL");
  if (B < 1 || L < 1 || K < 2 || K > 5 || nseq < 1 || max_seqlen < 1)
    return set_error(MOTIF_ERR_UNSUPPORTED, "short_conv_silu_multi: needs tokens and K in 2..5");
  const bool packed = cu_seqlens != nullptr;
  if (packed && B != 1) return set_error(MOTIF_ERR_INVALID, "short_conv_silu_multi: packed sequences need B == 1");
  if (!packed && (nseq != B || max_seqlen != L))
    return set_error(MOTIF_ERR_INVALID, "short_conv_silu_multi: padded batches need nseq == B and max_seqlen == L");
  if (dtype != MOTIF_F32 && dtype != MOTIF_BF16) return set_error(MOTIF_ERR_UNSUPPORTED, "short_conv_silu_multi: dtype");
  const int E = dtype == MOTIF_BF16 ? 8 : 4;
  ConvGroup g;
  g.n = n;
  int hd = 0;
  for (int p = 0; p < n; ++p) {
    if (!x[p] || !weight[p] || !y[p] || D[p] <= 0)
      return set_error(MOTIF_ERR_INVALID, "short_conv_silu_multi: NULL pointer or empty channel range");
    // the vector kernel only: 16-byte rows, separate tails, one head size for the
    // normalised problems
    const uintptr_t al = reinterpret_cast<uintptr_t>(x[p]) | reinterpret_cast<uintptr_t>(y[p]) |
                         reinterpret_cast<uintptr_t>(weight[p]) | reinterpret_cast<uintptr_t>(tail_in[p]) |
                         reinterpret_cast<uintptr_t>(tail_out[p]);
    const int h = head_dim[p];
    if ((al & 15) || (tail_out[p] && tail_out[p] == tail_in[p]) || D[p] % E || ((x_sb[p] | x_st[p] | y_sb[p] | y_st[p]) % E) ||
        (h != 0 && (h % E || D[p] % h || (hd != 0 && h != hd))))
      return set_error(MOTIF_ERR_UNSUPPORTED, "short_conv_silu_multi: problem not served by the vector kernel");
    if (h) hd = h;
    ConvArgs &a = g.a[p];
    a.x = x[p]; a.x_sb = x_sb[p]; a.x_st = x_st[p];
    a.w = weight[p]; a.tail_in = tail_in[p]; a.tail_out = tail_out[p];
    a.y = y[p]; a.y_sb = y_sb[p]; a.y_st = y_st[p];
    a.B = B; a.L = L; a.D = D[p]; a.cu = cu_seqlens;
    a.scale = scale[p]; a.tch = kConvStep; a.hd = h;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == MOTIF_BF16 ? launch_multi<bf16_t>(g, K, nseq, max_seqlen, hd, s)
                             : launch_multi<float>(g, K, nseq, max_seqlen, hd, s);
}
