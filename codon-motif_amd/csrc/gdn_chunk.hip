// GDN chunked prefill on bf16 MFMA (gfx950), chunk length 64.
//
// Three kernels.  gdn_prep_mfma runs one workgroup per (chunk, head) and does all
// the work that does not depend on the carried state: gamma = cumsum(g),
// N = strict(beta K K^T * D) and Attn = (Q K^T) * D on MFMA, T = (I + N)^{-1} by a
// blocked inverse (16x16 diagonal blocks by substitution, then 32 and 64 by
// T_ab = -T_aa N_ab T_bb products), and the chunk transition and output operators
//   A_n = e^{gamma_C} I - K~^T W      (dk x dk)      K~ = K e^{gamma_C - gamma}
//   H_n = K~^T U                      (dk x dv)      W = T beta e^gamma K, U = T beta V
//   Q'  = Q e^{gamma} - Attn W        (C x dk)
//   O'  = Attn U                      (C x dv)
// so that for the state S_n entering chunk n
//   S_{n+1} = A_n S_n + H_n,   O_n = O' + Q' S_n.
// gdn_state_scan carries S across the chunks, one workgroup per (16 state columns,
// head, sequence) with one wave per 16-row tile of S in accumulator registers (the
// tiles meet in LDS once per chunk) and a six-chunk-deep register prefetch of
// A_n / H_n (the workgroups of one head share an XCD, so A_n is read from HBM once
// and from that XCD's L2 after); it writes every S_n as MFMA operands.  gdn_chunk_out then
// forms O_n = O' + Q' S_n for all chunks in parallel.
//
// The workspace holds A_n, Q', H_n, O' and S_n in the order the consuming kernel's
// lanes read them (one 16-byte piece per lane per operand tile), so every load of
// the two scan kernels is a coalesced 1 KB wavefront access with no LDS staging.
//
// Inputs are bf16 (exact as MFMA operands).  fp32-derived operands (T, N, Attn, K~,
// M, A_n, Q', the state) are split into bf16 hi + lo and their products take three
// MFMA passes (hi.hi + hi.lo + lo.hi, fp32 accumulation), products with an exact
// bf16 operand two: about 16 mantissa bits per product, fp32 accumulation throughout.
#include <algorithm>
#include <cstdlib>

#include "gdn_internal.h"

namespace motif {

namespace {

constexpr int kC = 64;    // chunk length
constexpr int kPad = 8;   // LDS row padding (bf16 elements)

__device__ __forceinline__ __bf16 bf(float x) { return static_cast<__bf16>(x); }
__device__ __forceinline__ float fl(__bf16 x) { return static_cast<float>(x); }

__device__ __forceinline__ f32x4 mma(const bf16x8 &a, const bf16x8 &b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 16x16x16: A lane (m = l % 16) holds k = 4 (l / 16) .. +3, B lane (n = l % 16) the same k.
__device__ __forceinline__ f32x4 mma16(const bf16x4 &a, const bf16x4 &b, f32x4 c) {
  typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4;
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}

// c += (ah + al)(bh + bl) without the lo.lo term; SA / SB: operand has a lo part.
template <bool SA, bool SB>
__device__ __forceinline__ f32x4 mma3(const bf16x8 &ah, const bf16x8 &al, const bf16x8 &bh,
                                      const bf16x8 &bl, f32x4 c) {
  if (SA) c = mma(al, bh, c);
  if (SB) c = mma(ah, bl, c);
  return mma(ah, bh, c);
}

// 8 contiguous bf16 at row + k0 (k0 multiple of 8, 16-byte aligned rows).
__device__ __forceinline__ bf16x8 rd8(const __bf16 *row, int k0) {
  return *reinterpret_cast<const bf16x8 *>(row + k0);
}

// The A operand matching a B operand converted from a 16x16 accumulator pair:
// elements [k0 + 4g, +4) and [k0 + 16 + 4g, +4).
__device__ __forceinline__ bf16x8 rd_perm(const __bf16 *row, int k0, int g) {
  const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(row + k0 + 4 * g);
  const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(row + k0 + 16 + 4 * g);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

template <typename T> __device__ __forceinline__ float ldf(const T *p) { return ld(p); }

template <bool B> struct BoolC { static constexpr bool value = B; };

// Workspace per (head, chunk) cell, every piece 16 bytes per lane of a 64-lane tile:
//   an [2 planes][DK/16 mt][DK/32 ks][64]  bf16x8  A_n rows 16 mt + (l % 16), k slots
//                                                  32 ks + 4 (l / 16) + {0..3, 16..19}
//   qp [2][4][DK/32][64]                   bf16x8  Q' in the same operand order
//   hn [dv/16 cg][DK/16 mt][64]            f32x4   H_n[16 mt + 4 (l / 16) + r][16 cg + l % 16]
//   op [dv/16 cg][4 mt][64]                f32x4   O'[16 mt + l % 16][16 cg + 4 (l / 16) + r]
//   sn [dv/16 cg][DK/32 ks][2 planes][64]  bf16x8  S_n rows 32 ks + 4 (l / 16) + {0..3, 16..19},
//                                                  column 16 cg + l % 16
struct WsLayout {
  size_t an, qp, hn, op, sn, cell;
  __host__ __device__ WsLayout(int dk, int dv) {
    an = 0;
    qp = an + 2ull * dk * dk * 2;
    hn = qp + 2ull * kC * dk * 2;
    op = hn + 4ull * dk * dv;
    sn = op + 4ull * kC * dv;
    cell = sn + 4ull * dk * dv;
  }
};

// Fused front end of the prefill (motif_gdn_prefill_fused): the prep kernel reads the
// raw input projections of the chunk and computes q, k, v (short causal conv + SiLU,
// q / k L2-normalised, q scaled) and the gates beta, g itself, so they never go
// through HBM.  Conv kernel length kConvK.
constexpr int kConvK = 4;
struct FrontArgs {
  const bf16_t *x; int64_t x_sb, x_st;        // projection rows [B, L, ncols]
  int q_off, k_off, v_off, a_off, b_off;      // column offsets of q, k, v, a, b
  const bf16_t *wq, *wk, *wv;                 // conv weights [C, kConvK]
  const bf16_t *tq, *tk, *tv;                 // incoming conv tails [B, C, K-1] or nullptr
  bf16_t *oq, *ok, *ov;                       // outgoing tails [nseq, C, K-1] or nullptr
  const bf16_t *a_log, *dt_bias;              // [H]
  float q_scale;                              // dk^-1/2
};

// ------------------------------------------------------------------ prep
// LDS planes of [rows][64] bf16 (128-byte rows), 16-byte chunks XOR-swizzled by
// row so that 16 rows read at one column hit distinct banks.  Element offset of
// (row, col); col & 3 == 0 keeps 8-byte accesses aligned, col & 7 == 0 16-byte ones.
__device__ __forceinline__ int swz(int row, int col) {
  return row * 64 + ((((col >> 3) ^ (row & 7)) << 3) | (col & 7));
}
__device__ __forceinline__ bf16x8 rd8s(const __bf16 *p, int row, int col) {
  return *reinterpret_cast<const bf16x8 *>(p + swz(row, col));
}
__device__ __forceinline__ bf16x4 rd4s(const __bf16 *p, int row, int col) {
  return *reinterpret_cast<const bf16x4 *>(p + swz(row, col));
}
// 8 k-values [k0 + 4g, +4) and [k0 + 16 + 4g, +4) of a swizzled row: the A operand
// that pairs with a B operand built from two 16x16 accumulator tiles.
__device__ __forceinline__ bf16x8 rd_perm_s(const __bf16 *p, int row, int k0, int g) {
  return __builtin_shufflevector(rd4s(p, row, k0 + 4 * g), rd4s(p, row, k0 + 16 + 4 * g), 0, 1, 2, 3, 4, 5, 6, 7);
}
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
// two floats -> packed bf16 pair (round to nearest even), one instruction
__device__ __forceinline__ uint32_t pk_bf16(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){x0, x1}, bf16x2v));
}
// hi = RNE(x), lo = RNE(x - hi) for a pair, as packed words
__device__ __forceinline__ void split2(float x0, float x1, uint32_t &h, uint32_t &l) {
  h = pk_bf16(x0, x1);
  l = pk_bf16(x0 - __uint_as_float(h << 16), x1 - __uint_as_float(h & 0xffff0000u));
}
__device__ __forceinline__ void split4(const float *x, bf16x4 &h, bf16x4 &l) {
  uint2 hw, lw;
  split2(x[0], x[1], hw.x, lw.x);
  split2(x[2], x[3], hw.y, lw.y);
  h = __builtin_bit_cast(bf16x4, hw);
  l = __builtin_bit_cast(bf16x4, lw);
}
__device__ __forceinline__ void split8(const float *x, bf16x8 &h, bf16x8 &l) {
  uint4 hw, lw;
  split2(x[0], x[1], hw.x, lw.x);
  split2(x[2], x[3], hw.y, lw.y);
  split2(x[4], x[5], hw.z, lw.z);
  split2(x[6], x[7], hw.w, lw.w);
  h = __builtin_bit_cast(bf16x8, hw);
  l = __builtin_bit_cast(bf16x8, lw);
}
__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}
__device__ __forceinline__ uint16_t bits(__bf16 x) { return __builtin_bit_cast(uint16_t, x); }

// Byte offsets of the prep kernel's LDS.  Phase 7 (the operator products) keeps
//   att hi/lo  [64][64]   Attn = (Q K^T) * D, rows i', columns i
//   tt  hi/lo  [64][64]   T^T, rows j, columns i
//   kt         [DK][64]   K^T (exact), vt [DV][64] V^T (exact), ktt hi/lo [DK][64] K~^T
// Phases 1-5 use the kt.. region for K and Q rows (padded, row-major) and NT, one fp32
// [64][68] array holding N = strict(beta K K^T * D) below the diagonal and T^T on and
// above it; the level-2 product Y^T lives in the tt region until T^T is written there.
template <int DK, int DV>
struct PrepLayout {
  static constexpr int kPlane = 64 * 64 * 2;
  static constexpr int att_h = 0, att_l = kPlane, tt_h = 2 * kPlane, tt_l = 3 * kPlane;
  static constexpr int base = 4 * kPlane;
  static constexpr int kt = base, vt = kt + DK * 128, ktt_h = vt + DV * 128, ktt_l = ktt_h + DK * 128;
  static constexpr int end7 = ktt_l + DK * 128;
  static constexpr int kRow = DK + kPad;  // K / Q rows (bf16 elements)
  static constexpr int kh = base, qh = kh + 64 * kRow * 2, nt = qh + 64 * kRow * 2;
  static constexpr int end1 = nt + 64 * 68 * 4;
  static constexpr int yt = tt_h;  // [32][36] fp32
  static constexpr int small = end7 > end1 ? end7 : end1;  // gam[64], beta[64]
  static constexpr int bytes = small + 2 * 64 * 4;
};

template <int DK, int DV, bool FRONT>
__global__ void __launch_bounds__(256, 2) gdn_prep_mfma(GdnArgs a, ChunkArgs ca, char *ws, FrontArgs fa) {
  using TI = bf16_t;
  using PL = PrepLayout<DK, DV>;
  constexpr int NTS = 68;  // NT row stride (floats)
  extern __shared__ __attribute__((aligned(16))) char smem[];
  __bf16 *att_h = reinterpret_cast<__bf16 *>(smem + PL::att_h), *att_l = reinterpret_cast<__bf16 *>(smem + PL::att_l);
  __bf16 *tt_h = reinterpret_cast<__bf16 *>(smem + PL::tt_h), *tt_l = reinterpret_cast<__bf16 *>(smem + PL::tt_l);
  __bf16 *kt = reinterpret_cast<__bf16 *>(smem + PL::kt), *vt = reinterpret_cast<__bf16 *>(smem + PL::vt);
  __bf16 *ktt_h = reinterpret_cast<__bf16 *>(smem + PL::ktt_h), *ktt_l = reinterpret_cast<__bf16 *>(smem + PL::ktt_l);
  __bf16 *kh = reinterpret_cast<__bf16 *>(smem + PL::kh), *qh = reinterpret_cast<__bf16 *>(smem + PL::qh);
  float *nt = reinterpret_cast<float *>(smem + PL::nt);
  float *yt = reinterpret_cast<float *>(smem + PL::yt);
  float *gam = reinterpret_cast<float *>(smem + PL::small), *bet = gam + 64;

  const int chunk = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int ln = lane & 15, g = lane >> 4;
  const ChunkInfo ci = resolve_chunk(chunk, kC, a.L, ca);

  // variables phase 1 leaves for the later phases (the FRONT form uses its own)
  constexpr int KSEG = DK / 8, VP = 32 * (DV / 8) / 256;
  const int kp = tid & 31, kseg = tid >> 5;
  const bool kval = kseg < KSEG;
  uint4 k0r = {}, k1r = {}, v0r[VP], v1r[VP];
  bf16x4 qe[DK / 16];
  constexpr int RQ = DK / 8, RV = DV / 16, RM = RQ > RV ? RQ : RV;
  uint32_t cv[RM][4];  // FRONT: this thread's conv outputs, bf16 channel pairs per row
  int f_seg = 0, f_r0 = 0;
  if constexpr (!FRONT) {
    const TI *qb = static_cast<const TI *>(a.q) + ci.batch * a.q_sb + h * a.q_sh + int64_t(ci.t0) * a.q_st;
    const TI *kb = static_cast<const TI *>(a.k) + ci.batch * a.k_sb + h * a.k_sh + int64_t(ci.t0) * a.k_st;
    const TI *vb = static_cast<const TI *>(a.v) + ci.batch * a.v_sb + h * a.v_sh + int64_t(ci.t0) * a.v_st;
    const TI *bb = static_cast<const TI *>(a.beta) + ci.batch * a.b_sb + h * a.b_sh + int64_t(ci.t0) * a.b_st;
    const TI *gb = static_cast<const TI *>(a.g) + ci.batch * a.g_sb + h * a.g_sh + int64_t(ci.t0) * a.g_st;

    // ---- phase 1: rows 2p, 2p + 1 of one 8-column segment per thread (zero past len);
    // p = tid % 32, so the 4-byte transposed writes of a wavefront cover 32 distinct
    // column pairs of one LDS row (distinct banks).
    // Loads go through range-checked buffers over the chunk's valid rows: rows past
    // len read as zeros with no branches (so every load of the phase is in flight at once).
    const int last = ci.len - 1;
    const buf_t kbuf = make_buf(kb, (last * a.k_st + DK) * 2), qbuf = make_buf(qb, (last * a.q_st + DK) * 2);
    const buf_t vbuf = make_buf(vb, (last * a.v_st + a.dv) * 2);
    const buf_t gbuf = make_buf(gb, (last * a.g_st + 1) * 2), bbuf = make_buf(bb, (last * a.b_st + 1) * 2);
    // gates (every wavefront loads them; wavefront 0 takes the prefix sum)
    const float gv = buf_ld<TI>(gbuf, lane * a.g_st), bv = buf_ld<TI>(bbuf, lane * a.b_st);
    const int kc = 8 * min(kseg, KSEG - 1);
    k0r = buf_ld16(kbuf, ((2 * kp) * a.k_st + kc) * 2);
    k1r = buf_ld16(kbuf, ((2 * kp + 1) * a.k_st + kc) * 2);
    const uint4 q0r = buf_ld16(qbuf, ((2 * kp) * a.q_st + kc) * 2), q1r = buf_ld16(qbuf, ((2 * kp + 1) * a.q_st + kc) * 2);
#pragma unroll
    for (int r = 0; r < VP; ++r) {
      const int vp = tid & 31, vs = (tid >> 5) + 8 * r;
      const int vc = 8 * min(vs, a.dv / 8 - 1);
      v0r[r] = buf_ld16(vbuf, ((2 * vp) * a.v_st + vc) * 2);
      v1r[r] = buf_ld16(vbuf, ((2 * vp + 1) * a.v_st + vc) * 2);
    }
    // Q rows of this wavefront's Q' row tile (tile w): Q[16 w + ln][16 dt + 4g .. +3].
#pragma unroll
    for (int dt = 0; dt < DK / 16; ++dt)
      qe[dt] = __builtin_bit_cast(bf16x4, buf_ld8(qbuf, ((16 * w + ln) * a.q_st + 16 * dt + 4 * g) * 2));
    if (w == 0) {  // the inclusive prefix sum of g
      float s = gv;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(s, off, 64);
        if (lane >= off) s += y;
      }
      gam[lane] = s;
      bet[lane] = bv;
    }
    if (kval) {
      *reinterpret_cast<uint4 *>(kh + (2 * kp) * PL::kRow + 8 * kseg) = k0r;
      *reinterpret_cast<uint4 *>(kh + (2 * kp + 1) * PL::kRow + 8 * kseg) = k1r;
      *reinterpret_cast<uint4 *>(qh + (2 * kp) * PL::kRow + 8 * kseg) = q0r;
      *reinterpret_cast<uint4 *>(qh + (2 * kp + 1) * PL::kRow + 8 * kseg) = q1r;
    }
  
  } else {
    // ---- phase 1 (fused front end): wave 0 convolves q, wave 1 k, waves 2-3 v.  A
    // thread walks R consecutive chunk rows of one 8-channel segment with the conv
    // window in registers; the S segments of a row are S adjacent lanes, so the q / k
    // L2 norm of a row is a butterfly over them.  Arithmetic as the standalone conv
    // kernel: fp32 conv, SiLU, norm, one rounding to bf16.
    constexpr int KC = kConvK;
    const int prob = w < 2 ? w : 2;
    const int C = prob < 2 ? DK : DV;
    const int S = C / 8;
    const int t = prob < 2 ? lane : tid - 128;
    const int rows = prob < 2 ? RQ : RV;  // wave-uniform
    f_seg = t % S;
    f_r0 = (t / S) * rows;
    const int chan = h * C + 8 * f_seg;
    const int col = (prob == 0 ? fa.q_off : prob == 1 ? fa.k_off : fa.v_off) + chan;
    const bf16_t *wgt = (prob == 0 ? fa.wq : prob == 1 ? fa.wk : fa.wv) + static_cast<size_t>(chan) * KC;
    const bf16_t *tin = ca.cu ? nullptr : (prob == 0 ? fa.tq : prob == 1 ? fa.tk : fa.tv);
    const int s_lo = ca.cu ? ca.cu[ci.seq] : 0, s_hi = ca.cu ? ca.cu[ci.seq + 1] : a.L;
    const bf16_t *xs = fa.x + ci.batch * fa.x_sb + int64_t(s_lo) * fa.x_st + col;
    // rows outside [s_lo, s_hi) read zeros (a token before the start wraps to a huge offset)
    const buf_t xbuf = make_buf(xs, s_hi > s_lo ? static_cast<uint32_t>(((s_hi - s_lo - 1) * fa.x_st + 8) * 2) : 0u);
    const int rel0 = ci.t0 - s_lo + f_r0;  // sequence offset of this thread's first row
    uint4 raw[KC - 1 + RM];
#pragma unroll
    for (int i = 0; i < KC - 1 + RM; ++i)
      if (i < KC - 1 + rows)
        raw[i] = buf_ld16(xbuf, static_cast<uint32_t>((rel0 - (KC - 1) + i) * fa.x_st * 2));
    float wr[8][KC];
    {
      float wf[8 * KC];
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        const uint4 u = *reinterpret_cast<const uint4 *>(wgt + 8 * j);
        const uint32_t ww[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          wf[8 * j + 2 * e] = __uint_as_float(ww[e] << 16);
          wf[8 * j + 2 * e + 1] = __uint_as_float(ww[e] & 0xffff0000u);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int r = 0; r < KC; ++r) wr[e][r] = wf[e * KC + r];
    }
    __builtin_amdgcn_sched_barrier(0);  // the loads above stay one batch
    auto unpack8 = [](const uint4 &u, float *x) {
      const uint32_t ww[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[2 * e] = __uint_as_float(ww[e] << 16);
        x[2 * e + 1] = __uint_as_float(ww[e] & 0xffff0000u);
      }
    };
    float win[KC - 1][8];
#pragma unroll
    for (int r = 0; r < KC - 1; ++r) {
      unpack8(raw[r], win[r]);
      const int tok = rel0 - (KC - 1) + r;
      if (tin && tok < 0) {  // before the start of a batch row: the cached tail
#pragma unroll
        for (int e = 0; e < 8; ++e)
          win[r][e] = bf16_to_f32(tin[(static_cast<size_t>(ci.batch) * a.H * C + chan + e) * (KC - 1) + (KC - 1) + tok]);
      }
    }
    const float scale = prob == 0 ? fa.q_scale : 1.f;
#pragma unroll
    for (int i = 0; i < RM; ++i) {
      if (i < rows) {
        float xt[8], v[8];
        unpack8(raw[KC - 1 + i], xt);
        const bool live = f_r0 + i < ci.len;
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float acc = wr[e][KC - 1] * xt[e];
#pragma unroll
          for (int r = 0; r < KC - 1; ++r) acc = fmaf(wr[e][r], win[r][e], acc);
          v[e] = live ? silu_fast(acc) : 0.f;
          ss = fmaf(v[e], v[e], ss);
#pragma unroll
          for (int r = 0; r < KC - 2; ++r) win[r][e] = win[r + 1][e];
          win[KC - 2][e] = xt[e];
        }
        if (prob < 2) {
#pragma unroll
          for (int off = 1; off < 8; off <<= 1)
            if (off < S) ss += __shfl_xor(ss, off, 64);
          const float f = scale * rcp_fast(fmaxf(sqrtf(ss), 1e-12f));
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] *= f;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) cv[i][e] = pk_bf16(v[2 * e], v[2 * e + 1]);
        if (prob < 2)
          *reinterpret_cast<uint4 *>((prob == 0 ? qh : kh) + (f_r0 + i) * PL::kRow + 8 * f_seg) =
              uint4{cv[i][0], cv[i][1], cv[i][2], cv[i][3]};
      }
    }
    // gates of the chunk's rows (zero past len, as the unfused loads read them)
    if (w == 0) {
      float gv = 0.f, bv = 0.f;
      if (lane < ci.len) {
        const bf16_t *xr = fa.x + ci.batch * fa.x_sb + int64_t(ci.t0 + lane) * fa.x_st;
        const float av = bf16_to_f32(xr[fa.a_off + h]), braw = bf16_to_f32(xr[fa.b_off + h]);
        // beta = T(sigmoid(b)), g = T(-T(exp(A_log)) * T(softplus(T(a + dt_bias)))), threshold 20
        const float xa = fl(bf(av + bf16_to_f32(fa.dt_bias[h])));
        const float sp = fl(bf(xa > 20.f ? xa : log1pf(expf(xa))));
        const float A = fl(bf(expf(bf16_to_f32(fa.a_log[h]))));
        bv = fl(bf(1.f / (1.f + expf(-braw))));
        gv = fl(bf(-A * sp));
      }
      float sacc = gv;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(sacc, off, 64);
        if (lane >= off) sacc += y;
      }
      gam[lane] = sacc;
      bet[lane] = bv;
    }
    // the sequence's last chunk writes the outgoing conv tails (the last K-1 inputs)
    if (fa.oq && ci.t0 + ci.len == s_hi) {
      for (int idx = tid; idx < (2 * DK + DV) * (KC - 1); idx += 256) {
        const int ca_ = idx / (KC - 1), r = idx % (KC - 1);
        const int pb = ca_ < DK ? 0 : ca_ < 2 * DK ? 1 : 2;
        const int Cp = pb < 2 ? DK : DV, c = ca_ - (pb == 0 ? 0 : pb == 1 ? DK : 2 * DK);
        const int ch = h * Cp + c;
        const int rel = (s_hi - s_lo) - (KC - 1) + r;
        const bf16_t *tp = ca.cu ? nullptr : (pb == 0 ? fa.tq : pb == 1 ? fa.tk : fa.tv);
        bf16_t val = 0;
        if (rel >= 0)
          val = fa.x[ci.batch * fa.x_sb + int64_t(s_lo + rel) * fa.x_st + (pb == 0 ? fa.q_off : pb == 1 ? fa.k_off : fa.v_off) + ch];
        else if (tp)
          val = tp[(static_cast<size_t>(ci.batch) * a.H * Cp + ch) * (KC - 1) + (KC - 1) + rel];
        bf16_t *op_ = pb == 0 ? fa.oq : pb == 1 ? fa.ok : fa.ov;
        op_[(static_cast<size_t>(ci.seq) * a.H * Cp + ch) * (KC - 1) + r] = val;
      }
    }
  }
  __syncthreads();
  if constexpr (FRONT) {
#pragma unroll
    for (int dt = 0; dt < DK / 16; ++dt)
      qe[dt] = *reinterpret_cast<const bf16x4 *>(qh + (16 * w + ln) * PL::kRow + 16 * dt + 4 * g);
  }

  // ---- phase 2: G = K K^T -> N, and K Q^T -> Attn, on 16x16 tiles (bi <= bj).
  // Tile (bi, bj) of G holds G[16 bi + 4g + r][16 bj + ln] = G[16 bj + ln][16 bi + 4g + r]
  // (symmetric), i.e. N row 16 bj + ln, columns 16 bi + 4g .. +3: one float4 per lane.
  // Tile (bi, bj) of K Q^T holds (Q K^T)[16 bj + ln][16 bi + 4g + r]: Attn row 16 bj + ln.
  // Wave w takes Attn row block w and N row block 3 - w (all four column blocks, the
  // ones above the diagonal masked to zero); operand reads are issued before the products.
  {
    const int ba = w, bn = 3 - w;
    bf16x8 kop[4][DK / 32], qop[DK / 32], nop[DK / 32];
#pragma unroll
    for (int ks = 0; ks < DK / 32; ++ks) {
      const int k0 = 32 * ks + 8 * g;
#pragma unroll
      for (int bi = 0; bi < 4; ++bi) kop[bi][ks] = rd8(kh + (16 * bi + ln) * PL::kRow, k0);
      qop[ks] = rd8(qh + (16 * ba + ln) * PL::kRow, k0);
      nop[ks] = rd8(kh + (16 * bn + ln) * PL::kRow, k0);
    }
    f32x4 at[4], nt4[4];
#pragma unroll
    for (int bi = 0; bi < 4; ++bi) {
      at[bi] = f32x4{0.f, 0.f, 0.f, 0.f};
      nt4[bi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < DK / 32; ++ks) {  // tiles above the diagonal are masked below
        at[bi] = mma(kop[bi][ks], qop[ks], at[bi]);
        nt4[bi] = mma(kop[bi][ks], nop[ks], nt4[bi]);
      }
    }
    const int rowa = 16 * ba + ln, rown = 16 * bn + ln;
    const float ga = gam[rowa], gn = gam[rown], bn_ = bet[rown];
#pragma unroll
    for (int bi = 0; bi < 4; ++bi) {
      const int col = 16 * bi + 4 * g;
      float x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = (col + r <= rowa) ? at[bi][r] * exp_fast(ga - gam[col + r]) : 0.f;
      bf16x4 hv, lv;
      split4(x, hv, lv);
      *reinterpret_cast<bf16x4 *>(att_h + swz(rowa, col)) = hv;
      *reinterpret_cast<bf16x4 *>(att_l + swz(rowa, col)) = lv;
      // (the zeros written above the diagonal land where T is written later)
      f32x4 y;
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = (col + r < rown) ? bn_ * nt4[bi][r] * exp_fast(gn - gam[col + r]) : 0.f;
      *reinterpret_cast<f32x4 *>(nt + rown * NTS + col) = y;
    }
  }
  __syncthreads();

  // ---- phase 3: diagonal 16x16 blocks of T = (I + N)^{-1} by forward substitution,
  // wave w -> block w, lane c < 16 -> column c; T[16w + i][16w + c] goes to NT row 16w + c.
  if (ln == lane) {
    const int b = w, c = lane;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float *nrow = nt + (16 * b + i) * NTS + 16 * b;
      float s = (i == c) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) s = fmaf(-nrow[j], x[j], s);
      x[i] = s;
    }
    float *trow = nt + (16 * b + c) * NTS + 16 * b;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (i >= c) trow[i] = x[i];
  }
  __syncthreads();

  // ---- phase 4: 32x32 inverses: T_ab = -T_aa N_ab T_bb for (a, b) = (1, 0), (3, 2).
  if (w < 2) {
    const int a_ = 2 * w + 1, b_ = 2 * w;
    // X = N_ab T_bb (16x16x16 products in three passes)
    float av[4], bv[4];
    {
      const f32x4 n4 = *reinterpret_cast<const f32x4 *>(nt + (16 * a_ + ln) * NTS + 16 * b_ + 4 * g);
      const f32x4 t4 = *reinterpret_cast<const f32x4 *>(nt + (16 * b_ + ln) * NTS + 16 * b_ + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        av[r] = n4[r];
        bv[r] = (4 * g + r >= ln) ? t4[r] : 0.f;  // T_bb[4g + r][ln], lower triangular
      }
    }
    bf16x4 ah, al, bh, bl;
    split4(av, ah, al);
    split4(bv, bh, bl);
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
    x = mma16(al, bh, x);
    x = mma16(ah, bl, x);
    x = mma16(ah, bh, x);
    // T_ab = -T_aa X: A = T_aa[ln][4g + r] (stored at NT[16a + 4g + r][16a + ln]), B = X.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int k = 4 * g + r;
      av[r] = (k <= ln) ? nt[(16 * a_ + k) * NTS + 16 * a_ + ln] : 0.f;
      bv[r] = x[r];
    }
    split4(av, ah, al);
    split4(bv, bh, bl);
    f32x4 y = {0.f, 0.f, 0.f, 0.f};
    y = mma16(al, bh, y);
    y = mma16(ah, bl, y);
    y = mma16(ah, bh, y);
    // y[r] = (T_aa X)[4g + r][ln] -> T[16a + 4g + r][16b + ln] at NT[16b + ln][16a + 4g + r]
    *reinterpret_cast<f32x4 *>(nt + (16 * b_ + ln) * NTS + 16 * a_ + 4 * g) = -y;
  }
  __syncthreads();

  // ---- phase 5: the 64x64 inverse: T[32:, :32] = -T[32:, 32:] N[32:, :32] T[:32, :32].
  {
    const int ti = w >> 1, tj = w & 1;
    // Y = N[32:, :32] T[:32, :32], tile (ti, tj), K = 32.
    float av[8], bv[8];
    {
      const float *nrow = nt + (32 + 16 * ti + ln) * NTS + 8 * g;
      const float *trow = nt + (16 * tj + ln) * NTS + 8 * g;  // T[8g + t][16 tj + ln]
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        av[t] = nrow[t];
        bv[t] = (8 * g + t >= 16 * tj + ln) ? trow[t] : 0.f;
      }
    }
    bf16x8 ah, al, bh, bl;
    split8(av, ah, al);
    split8(bv, bh, bl);
    f32x4 y = {0.f, 0.f, 0.f, 0.f};
    y = mma3<true, true>(ah, al, bh, bl, y);
    *reinterpret_cast<f32x4 *>(yt + (16 * tj + ln) * 36 + 16 * ti + 4 * g) = y;  // Y^T
    __syncthreads();
    // T[32 + 16 ti + m][16 tj + n] = -sum_k T[32 + 16 ti + m][32 + k] Y[k][16 tj + n]
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int k = 8 * g + t;
      av[t] = (k <= 16 * ti + ln) ? nt[(32 + k) * NTS + 32 + 16 * ti + ln] : 0.f;
      bv[t] = yt[(16 * tj + ln) * 36 + k];
    }
    split8(av, ah, al);
    split8(bv, bh, bl);
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    o = mma3<true, true>(ah, al, bh, bl, o);
    *reinterpret_cast<f32x4 *>(nt + (16 * tj + ln) * NTS + 32 + 16 * ti + 4 * g) = -o;
  }
  __syncthreads();

  // ---- phase 6: T^T (bf16 hi/lo), then the transposed K, K~ and V planes.
  {
    const int j = tid >> 2, i0 = 16 * (tid & 3);
    float x[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) x[t] = (i0 + t >= j) ? nt[j * NTS + i0 + t] : 0.f;
    bf16x8 h0, l0, h1, l1;
    split8(x, h0, l0);
    split8(x + 8, h1, l1);
    *reinterpret_cast<bf16x8 *>(tt_h + swz(j, i0)) = h0;
    *reinterpret_cast<bf16x8 *>(tt_l + swz(j, i0)) = l0;
    *reinterpret_cast<bf16x8 *>(tt_h + swz(j, i0 + 8)) = h1;
    *reinterpret_cast<bf16x8 *>(tt_l + swz(j, i0 + 8)) = l1;
  }
  const float glast = gam[kC - 1];
  __syncthreads();  // NT and the K / Q rows are dead from here on
  if constexpr (!FRONT) {
    if (kval) {
      const int j = 2 * kp;
      const float f0 = exp_fast(glast - gam[j]), f1 = exp_fast(glast - gam[j + 1]);
      const bf16x8 ka = __builtin_bit_cast(bf16x8, k0r), kb_ = __builtin_bit_cast(bf16x8, k1r);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int d = 8 * kseg + t;
        *reinterpret_cast<uint32_t *>(kt + swz(d, j)) = pack2(bits(ka[t]), bits(kb_[t]));
        const float x0 = fl(ka[t]) * f0, x1 = fl(kb_[t]) * f1;
        uint32_t hw, lw;
        split2(x0, x1, hw, lw);
        *reinterpret_cast<uint32_t *>(ktt_h + swz(d, j)) = hw;
        *reinterpret_cast<uint32_t *>(ktt_l + swz(d, j)) = lw;
      }
    }
#pragma unroll
    for (int r = 0; r < VP; ++r) {
      const int vp = tid & 31, vs = (tid >> 5) + 8 * r;
      if (vs < a.dv / 8) {
        const bf16x8 va = __builtin_bit_cast(bf16x8, v0r[r]), vb_ = __builtin_bit_cast(bf16x8, v1r[r]);
#pragma unroll
        for (int t = 0; t < 8; ++t)
          *reinterpret_cast<uint32_t *>(vt + swz(8 * vs + t, 2 * vp)) = pack2(bits(va[t]), bits(vb_[t]));
      }
    }
  
  } else if (w == 1) {  // K^T and K~^T planes from this thread's K rows (pairs of rows)
#pragma unroll
    for (int i = 0; i < RQ; i += 2) {
      const int j = f_r0 + i;
      const float f0 = exp_fast(glast - gam[j]), f1 = exp_fast(glast - gam[j + 1]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 8 * f_seg + e;
        const uint16_t b0 = static_cast<uint16_t>(cv[i][e >> 1] >> (16 * (e & 1)));
        const uint16_t b1 = static_cast<uint16_t>(cv[i + 1][e >> 1] >> (16 * (e & 1)));
        *reinterpret_cast<uint32_t *>(kt + swz(d, j)) = pack2(b0, b1);
        uint32_t hw, lw;
        split2(bf16_to_f32(b0) * f0, bf16_to_f32(b1) * f1, hw, lw);
        *reinterpret_cast<uint32_t *>(ktt_h + swz(d, j)) = hw;
        *reinterpret_cast<uint32_t *>(ktt_l + swz(d, j)) = lw;
      }
    }
  } else if (w >= 2) {  // V^T plane
#pragma unroll
    for (int i = 0; i < RV; i += 2) {
      const int j = f_r0 + i;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint16_t b0 = static_cast<uint16_t>(cv[i][e >> 1] >> (16 * (e & 1)));
        const uint16_t b1 = static_cast<uint16_t>(cv[i + 1][e >> 1] >> (16 * (e & 1)));
        *reinterpret_cast<uint32_t *>(vt + swz(8 * f_seg + e, j)) = pack2(b0, b1);
      }
    }
  }
  __syncthreads();

  // ---- phase 7: M = [K~^T ; Attn] T, computed as M^T tiles (rows j, columns m) and fed
  // straight from the accumulators into  Z^T = K^T (diag(beta e^gamma) M^T)  and
  // Y = (M diag(beta)) V  (or Y^T).  m-tiles 0 .. DK/16-1 give A_n and H_n, the rest Q' and O'.
  const WsLayout Lw(DK, a.dv);
  char *cell = ws + (static_cast<size_t>(h) * ca.total_chunks + chunk) * Lw.cell;
  float *hn = reinterpret_cast<float *>(cell + Lw.hn);
  float *op = reinterpret_cast<float *>(cell + Lw.op);
  const float eC = exp_fast(glast);
  float sk[4][4], sv[4][4];  // per-row scales of M^T for rows j = 16 jt + 4g + r
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * jt + 4 * g + r;
      sv[jt][r] = bet[j];
      sk[jt][r] = bet[j] * exp_fast(gam[j]);
    }
  // One m-tile: TOP -> rows d' = 16 mti + ln of A_n / H_n, else rows i' of Q' / O'.
  auto mtile = [&](auto top_c, int mti, const bf16x4 *qrow) {
    constexpr bool top = decltype(top_c)::value;
    const int mrow = 16 * mti + ln;  // d' (top) or i' (bottom)
    const __bf16 *Lh = top ? ktt_h : att_h, *Ll = top ? ktt_l : att_l;
    bf16x8 lh[2], ll[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      lh[ks] = rd8s(Lh, mrow, 32 * ks + 8 * g);
      ll[ks] = rd8s(Ll, mrow, 32 * ks + 8 * g);
    }
    bf16x4 mkh[4], mkl[4], mvh[4], mvl[4];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks == 0 && jt >= 2) continue;  // T^T rows j >= 32 vanish on columns i < 32
        acc = mma3<true, true>(rd8s(tt_h, 16 * jt + ln, 32 * ks + 8 * g), rd8s(tt_l, 16 * jt + ln, 32 * ks + 8 * g),
                               lh[ks], ll[ks], acc);
      }
      float xk[4], xv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        xk[r] = acc[r] * sk[jt][r];
        xv[r] = acc[r] * sv[jt][r];
      }
      split4(xk, mkh[jt], mkl[jt]);
      split4(xv, mvh[jt], mvl[jt]);
    }
    bf16x8 bkh[2], bkl[2], bvh[2], bvl[2];
#pragma unroll
    for (int jp = 0; jp < 2; ++jp) {
      bkh[jp] = __builtin_shufflevector(mkh[2 * jp], mkh[2 * jp + 1], 0, 1, 2, 3, 4, 5, 6, 7);
      bkl[jp] = __builtin_shufflevector(mkl[2 * jp], mkl[2 * jp + 1], 0, 1, 2, 3, 4, 5, 6, 7);
      bvh[jp] = __builtin_shufflevector(mvh[2 * jp], mvh[2 * jp + 1], 0, 1, 2, 3, 4, 5, 6, 7);
      bvl[jp] = __builtin_shufflevector(mvl[2 * jp], mvl[2 * jp + 1], 0, 1, 2, 3, 4, 5, 6, 7);
    }
    const float eq = top ? eC : exp_fast(gam[mrow]);
    char *base = cell + (top ? Lw.an : Lw.qp);
    constexpr int ntile = top ? DK / 16 : kC / 16;
#pragma unroll
    for (int dt = 0; dt < DK / 16; ++dt) {
      f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jp = 0; jp < 2; ++jp) {
        const bf16x8 ak = rd_perm_s(kt, 16 * dt + ln, 32 * jp, g);
        z = mma(ak, bkl[jp], z);
        z = mma(ak, bkh[jp], z);
      }
      // z[r] = Z^T[16 dt + 4g + r][m] = (M_k K)[m][16 dt + 4g + r]
      const int col = 16 * dt + 4 * g;
      float x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        x[r] = (top ? (col + r == mrow ? eq : 0.f) : fl(qrow[dt][r]) * eq) - z[r];
      bf16x4 hv, lv;
      split4(x, hv, lv);
      // operand order: tile (plane, mti, ks = dt / 2), lane, half dt % 2
      const size_t o_h = ((static_cast<size_t>(0 * ntile + mti) * (DK / 32) + dt / 2) * 64 + lane) * 16 + 8 * (dt & 1);
      const size_t o_l = ((static_cast<size_t>(1 * ntile + mti) * (DK / 32) + dt / 2) * 64 + lane) * 16 + 8 * (dt & 1);
      *reinterpret_cast<bf16x4 *>(base + o_h) = hv;
      *reinterpret_cast<bf16x4 *>(base + o_l) = lv;
    }
    // H_n as Y = M_v V (accumulator layout of the state), O' as Y^T (layout of O^T).
    float *dst0 = top ? hn + mti * 256 : op + mti * 256;
#pragma unroll
    for (int et = 0; et < DV / 16; ++et) {
      if (et < a.dv / 16) {
        f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jp = 0; jp < 2; ++jp) {
          const bf16x8 avv = rd_perm_s(vt, 16 * et + ln, 32 * jp, g);
          if (top) {
            y = mma(bvl[jp], avv, y);
            y = mma(bvh[jp], avv, y);
          } else {
            y = mma(avv, bvl[jp], y);
            y = mma(avv, bvh[jp], y);
          }
        }
        *reinterpret_cast<f32x4 *>(dst0 + static_cast<size_t>(et) * ntile * 256 + 4 * lane) = y;
      }
    }
  };
  // wave w: A_n / H_n row tile w (when w < DK/16) and Q' / O' row tile w
  if (w < DK / 16) mtile(BoolC<true>{}, w, nullptr);
  mtile(BoolC<false>{}, w, qe);
}

// ------------------------------------------------------------------ state scan
// One wave per 16-row tile of S.
template <int DK>
struct ScanStage {
  uint4 an[2][DK / 32];  // A_n hi / lo operand rows of this wave's tile
  f32x4 hn;              // H_n tile, accumulator layout
};

template <int DK>
__device__ __forceinline__ void scan_load(ScanStage<DK> &st, const char *cell, const WsLayout &Lw, int cg, int mt,
                                          int lane) {
  constexpr int TDK = DK / 16, KS = DK / 32;
  const uint4 *an = reinterpret_cast<const uint4 *>(cell + Lw.an) + lane;
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) st.an[p][ks] = an[((p * TDK + mt) * KS + ks) * 64];
  st.hn = reinterpret_cast<const f32x4 *>(cell + Lw.hn)[(static_cast<size_t>(cg) * TDK + mt) * 64 + lane];
}

// One workgroup per (16 state columns, head, sequence), one wave per 16-row tile mt of
// S: S[r] = S[16 mt + 4g + r][16 cg + l % 16].  Per chunk every wave turns its tile
// into hi / lo bf16 halves of the B operand (slots 0..3 of a 32-row k-step come from
// tile 2 ks, slots 4..7 from tile 2 ks + 1), exchanges them through LDS (double
// buffered: one barrier per chunk) and forms its tile of S_{n+1} = A_n S_n + H_n: a
// chain of 3 (DK / 32) MFMAs per wave instead of 3 DK^2 / 512 for one wave per column
// group.
// Workgroups of a scan launch: ngroups (head, sequence) groups of ncg column-group
// workgroups that all read the same A_n.  Workgroups go to the 8 XCDs round-robin by
// linear id, so a group is placed on one XCD (its A_n then comes from that XCD's L2
// after the first read): linear id L runs on XCD L % 8, and slot L / 8 of that XCD
// holds column group slot % ncg of group 8 (slot / ncg) + L % 8.  The grid is padded
// to whole groups per XCD; padding workgroups exit at once.
struct ScanGrid {
  int ncg, ngroups;
  static constexpr int kXcd = 8;
  int blocks() const { return kXcd * ((ngroups + kXcd - 1) / kXcd) * ncg; }
};

template <int DK>
__global__ void __launch_bounds__(64 * (DK / 16)) gdn_state_scan(GdnArgs a, ChunkArgs ca, char *ws, ScanGrid sgrid) {
  constexpr int TDK = DK / 16, KS = DK / 32;
  const int slot = blockIdx.x / ScanGrid::kXcd;
  const int group = (slot / sgrid.ncg) * ScanGrid::kXcd + blockIdx.x % ScanGrid::kXcd;
  if (group >= sgrid.ngroups) return;
  const int cg = slot % sgrid.ncg, h = group % a.H, sq = group / a.H;
  const int lane = threadIdx.x & 63, mt = threadIdx.x >> 6;
  const int ln = lane & 15, g = lane >> 4;
  const int col = 16 * cg + ln;
  const int ks_own = mt >> 1, half = mt & 1;  // where this tile sits in the B operand

  int first, count;
  if (ca.cu == nullptr) {
    first = sq * ca.nper;
    count = ca.nper;
  } else {
    first = ca.coff[sq];
    count = ca.coff[sq + 1] - first;
  }
  const WsLayout Lw(DK, a.dv);
  char *cell0 = ws + (static_cast<size_t>(h) * ca.total_chunks + first) * Lw.cell;

  f32x4 S;
  const size_t sbase = (static_cast<size_t>(sq) * a.H + h) * DK * a.dv;
#pragma unroll
  for (int r = 0; r < 4; ++r)
    S[r] = a.s_in ? a.s_in[sbase + static_cast<size_t>(16 * mt + 4 * g + r) * a.dv + col] : 0.f;

  // [buffer][plane][ks][lane] bf16x8 B operands of S
  __shared__ __attribute__((aligned(16))) uint4 sB[2][2][KS][64];

  // kScanDepth stages of A_n / H_n in flight (chunk n + kScanDepth is requested while
  // chunk n is computed)
  constexpr int kScanDepth = 6;
  ScanStage<DK> st[kScanDepth];
  if (count > 0) {
#pragma unroll
    for (int j = 0; j < kScanDepth; ++j)
      scan_load<DK>(st[j], cell0 + static_cast<size_t>(min(j, count - 1)) * Lw.cell, Lw, cg, mt, lane);
  }

  // S_n as hi / lo operands (shared, and stored for the output kernel), then this
  // wave's tile of S_{n+1}; the stage is then refilled with chunk
  // min(n + kScanDepth, count - 1) (a repeat load of the last chunk near the end keeps
  // the loop free of branches).
  auto step = [&](ScanStage<DK> &stg, int n) {
    char *cell = cell0 + static_cast<size_t>(n) * Lw.cell;
    const int buf = n & 1;
    uint2 hv, lv;
    {
      bf16_t hb[4], lb[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const __bf16 hh = bf(S[r]);
        hb[r] = __builtin_bit_cast(bf16_t, hh);
        lb[r] = __builtin_bit_cast(bf16_t, bf(S[r] - fl(hh)));
      }
      hv = uint2{hb[0] | (static_cast<uint32_t>(hb[1]) << 16), hb[2] | (static_cast<uint32_t>(hb[3]) << 16)};
      lv = uint2{lb[0] | (static_cast<uint32_t>(lb[1]) << 16), lb[2] | (static_cast<uint32_t>(lb[3]) << 16)};
    }
    reinterpret_cast<uint2 *>(&sB[buf][0][ks_own][lane])[half] = hv;
    reinterpret_cast<uint2 *>(&sB[buf][1][ks_own][lane])[half] = lv;
    __syncthreads();
    // S_n for the output kernel: the 2 KS = TDK operand arrays, one full 1 KB array per
    // wave (array mt = plane mt % 2 of k-step mt / 2)
    reinterpret_cast<uint4 *>(cell + Lw.sn)[(static_cast<size_t>(cg) * KS * 2 + mt) * 64 + lane] =
        sB[buf][mt & 1][mt >> 1][lane];
    f32x4 acc = stg.hn;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const bf16x8 sh = __builtin_bit_cast(bf16x8, sB[buf][0][ks][lane]);
      const bf16x8 sl = __builtin_bit_cast(bf16x8, sB[buf][1][ks][lane]);
      acc = mma(__builtin_bit_cast(bf16x8, stg.an[1][ks]), sh, acc);
      acc = mma(__builtin_bit_cast(bf16x8, stg.an[0][ks]), sl, acc);
      acc = mma(__builtin_bit_cast(bf16x8, stg.an[0][ks]), sh, acc);
    }
    S = acc;
    scan_load<DK>(stg, cell0 + static_cast<size_t>(min(n + kScanDepth, count - 1)) * Lw.cell, Lw, cg, mt, lane);
  };
  int n = 0;
  for (; n + kScanDepth <= count; n += kScanDepth) {
#pragma unroll
    for (int j = 0; j < kScanDepth; ++j) step(st[j], n + j);
  }
#pragma unroll
  for (int j = 0; j < kScanDepth - 1; ++j)
    if (n + j < count) step(st[j], n + j);

#pragma unroll
  for (int r = 0; r < 4; ++r) a.s_out[sbase + static_cast<size_t>(16 * mt + 4 * g + r) * a.dv + col] = S[r];
}

// ------------------------------------------------------------------ chunk output
// O_n = O' + Q' S_n for every chunk in parallel, computed transposed so that each lane
// ends with four consecutive columns of one row: O^T = S_n^T Q'^T, accumulator
// lane l holding O[16 mt + l % 16][16 cg + 4 (l / 16) + r].
template <typename TO, int DK>
__global__ void __launch_bounds__(256) gdn_chunk_out(GdnArgs a, ChunkArgs ca, const char *ws, int vec_store) {
  constexpr int KS = DK / 32;
  constexpr int kMaxCg = 2;  // 16-column groups per wave (dv <= 128)
  const int chunk = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, g = lane >> 4;
  const ChunkInfo ci = resolve_chunk(chunk, kC, a.L, ca);
  const WsLayout Lw(DK, a.dv);
  const char *cell = ws + (static_cast<size_t>(h) * ca.total_chunks + chunk) * Lw.cell;
  const int ncg = a.dv / 16;

  // gate pieces of the fused GatedRMSNorm, requested before the products
  uint2 gv[kMaxCg][4];
  if (a.gate) {
    const bf16_t *gp = static_cast<const bf16_t *>(a.gate) + ci.batch * a.gt_sb + int64_t(ci.t0) * a.gt_st + h * a.dv;
#pragma unroll
    for (int i = 0; i < kMaxCg; ++i)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = min(16 * mt + ln, ci.len - 1), c0 = 16 * min(w + 4 * i, ncg - 1) + 4 * g;
        gv[i][mt] = *reinterpret_cast<const uint2 *>(gp + int64_t(row) * a.gt_st + c0);
      }
  }

  bf16x8 qh[4][KS], ql[4][KS];
  const uint4 *qp = reinterpret_cast<const uint4 *>(cell + Lw.qp) + lane;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qh[mt][ks] = __builtin_bit_cast(bf16x8, qp[((0 * 4 + mt) * KS + ks) * 64]);
      ql[mt][ks] = __builtin_bit_cast(bf16x8, qp[((1 * 4 + mt) * KS + ks) * 64]);
    }
  // O tiles of this wave's column groups cg = w + 4 i: lane holds O[16 mt + ln][16 cg + 4 g + r]
  f32x4 res[kMaxCg][4];
#pragma unroll
  for (int i = 0; i < kMaxCg; ++i) {
    const int cg = w + 4 * i;
    if (cg >= ncg) break;
    const uint4 *sn = reinterpret_cast<const uint4 *>(cell + Lw.sn) + static_cast<size_t>(cg) * KS * 2 * 64 + lane;
    const f32x4 *op = reinterpret_cast<const f32x4 *>(cell + Lw.op) + static_cast<size_t>(cg) * 4 * 64 + lane;
    bf16x8 sh[KS], sl[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      sh[ks] = __builtin_bit_cast(bf16x8, sn[(2 * ks) * 64]);
      sl[ks] = __builtin_bit_cast(bf16x8, sn[(2 * ks + 1) * 64]);
    }
    f32x4 acc[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[mt] = op[mt * 64];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) acc[mt] = mma(sl[ks], qh[mt][ks], acc[mt]);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) acc[mt] = mma(sh[ks], ql[mt][ks], acc[mt]);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) acc[mt] = mma(sh[ks], qh[mt][ks], acc[mt]);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) res[i][mt] = acc[mt];
    if (a.o) {
      TO *ob = static_cast<TO *>(a.o) + ci.batch * a.o_sb + h * a.o_sh + int64_t(ci.t0) * a.o_st;
      const int c0 = 16 * cg + 4 * g;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = 16 * mt + ln;
        if (row >= ci.len) continue;
        TO *dst = ob + int64_t(row) * a.o_st + c0;
        if (vec_store) {
          bf16x4 v;
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = bf(acc[mt][r]);
          *reinterpret_cast<bf16x4 *>(dst) = v;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) st(dst + r, acc[mt][r]);
        }
      }
    }
  }
  if (!a.gate) return;

  // GatedRMSNorm of the head rows: sums of squares of the bf16-rounded O over this
  // wave's columns, then over the lane groups and, through LDS, over the 4 waves.
  __shared__ float sred[4][64];
  float ss[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kMaxCg; ++i) {
    if (w + 4 * i >= ncg) break;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        res[i][mt][r] = fl(bf(res[i][mt][r]));
        ss[mt] = fmaf(res[i][mt][r], res[i][mt][r], ss[mt]);
      }
  }
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    ss[mt] += __shfl_xor(ss[mt], 16, 64);
    ss[mt] += __shfl_xor(ss[mt], 32, 64);
  }
  if (g == 0) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) sred[w][16 * mt + ln] = ss[mt];
  }
  __syncthreads();
  float rs[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int row = 16 * mt + ln;
    rs[mt] = rsqrtf((sred[0][row] + sred[1][row] + sred[2][row] + sred[3][row]) / a.dv + a.neps);
  }
  bf16_t *yb = static_cast<bf16_t *>(a.y) + ci.batch * a.y_sb + int64_t(ci.t0) * a.y_st + h * a.dv;
#pragma unroll
  for (int i = 0; i < kMaxCg; ++i) {
    const int cg = w + 4 * i;
    if (cg >= ncg) break;
    const int c0 = 16 * cg + 4 * g;
    const uint2 wraw = *reinterpret_cast<const uint2 *>(static_cast<const bf16_t *>(a.nw) + c0);
    const float wv[4] = {__uint_as_float(wraw.x << 16), __uint_as_float(wraw.x & 0xffff0000u),
                         __uint_as_float(wraw.y << 16), __uint_as_float(wraw.y & 0xffff0000u)};
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int row = 16 * mt + ln;
      if (row >= ci.len) continue;
      const float gf[4] = {__uint_as_float(gv[i][mt].x << 16), __uint_as_float(gv[i][mt].x & 0xffff0000u),
                           __uint_as_float(gv[i][mt].y << 16), __uint_as_float(gv[i][mt].y & 0xffff0000u)};
      bf16x4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[r] = bf(fl(bf(fl(bf(res[i][mt][r] * rs[mt])) * wv[r])) * fl(bf(silu_fast(gf[r]))));
      *reinterpret_cast<bf16x4 *>(yb + int64_t(row) * a.y_st + c0) = v;
    }
  }
}

template <int DK, int DV, bool FRONT = false>
int launch_prep(const GdnArgs &a, const ChunkArgs &ca, char *ws, hipStream_t s, const FrontArgs &fa = FrontArgs{}) {
  const size_t smem = PrepLayout<DK, DV>::bytes;
  auto kern = gdn_prep_mfma<DK, DV, FRONT>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
  if (e != hipSuccess) return set_error(MOTIF_ERR_HIP, std::string("gdn_prep_mfma smem: ") + hipGetErrorString(e));
  kern<<<dim3(ca.total_chunks, a.H), dim3(256), smem, s>>>(a, ca, ws, fa);
  return check_launch("gdn_prep_mfma");
}

template <int DK>
int launch_dk(const GdnArgs &a, const ChunkArgs &ca, char *ws, hipStream_t s) {
  int rc;
  // the prep's V^T plane is sized for the padded dv bound of its template
  if (a.dv <= 64) rc = launch_prep<DK, 64>(a, ca, ws, s);
  else rc = launch_prep<DK, 128>(a, ca, ws, s);
  if (rc) return rc;
  const ScanGrid sgrid{a.dv / 16, a.H * ca.nseq};
  gdn_state_scan<DK><<<sgrid.blocks(), dim3(64 * (DK / 16)), 0, s>>>(a, ca, ws, sgrid);
  if ((rc = check_launch("gdn_state_scan"))) return rc;
  // 8-byte output stores when every row start is 8-byte aligned
  const int vec = ((a.o_sb | a.o_sh | a.o_st) & 3) == 0 && (reinterpret_cast<uintptr_t>(a.o) & 7) == 0;
  gdn_chunk_out<bf16_t, DK><<<dim3(ca.total_chunks, a.H), dim3(256), 0, s>>>(a, ca, ws, vec);
  return check_launch("gdn_chunk_out");
}

}  // namespace

bool chunk_mfma_supported(int dk, int dv, int chunk) {
  return chunk == kC && (dk == 32 || dk == 64) && dv % 16 == 0 && dv > 0 && dv <= 128;
}

size_t chunk_mfma_workspace_bytes(int H, int dk, int dv, int total_chunks) {
  return WsLayout(dk, dv).cell * static_cast<size_t>(H) * total_chunks;
}

bool chunk_mfma_eligible(const GdnArgs &a, int chunk, int in_dtype, int out_dtype) {
  if (in_dtype != MOTIF_BF16 || out_dtype != MOTIF_BF16 || !chunk_mfma_supported(a.dk, a.dv, chunk)) return false;
  // 16-byte row loads of q / k / v
  const int64_t st = a.q_sb | a.q_sh | a.q_st | a.k_sb | a.k_sh | a.k_st | a.v_sb | a.v_sh | a.v_st;
  const uintptr_t p = reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.k) | reinterpret_cast<uintptr_t>(a.v);
  // chunk-relative byte offsets of the range-checked buffer loads stay below 2^31
  const int64_t tmax = std::max({std::abs(a.q_st), std::abs(a.k_st), std::abs(a.v_st), std::abs(a.b_st), std::abs(a.g_st)});
  return (st & 7) == 0 && (p & 15) == 0 && tmax * kC * 2 < (int64_t(1) << 30);
}

int launch_chunk_mfma(const GdnArgs &a, const ChunkArgs &ca, void *workspace, hipStream_t s) {
  char *ws = static_cast<char *>(workspace);
  return a.dk == 32 ? launch_dk<32>(a, ca, ws, s) : launch_dk<64>(a, ca, ws, s);
}
namespace {

template <int DK, int DV>
int launch_fused(const GdnArgs &a, const ChunkArgs &ca, const FrontArgs &fa, char *ws, hipStream_t s) {
  int rc = launch_prep<DK, DV, true>(a, ca, ws, s, fa);
  if (rc) return rc;
  const ScanGrid sgrid{a.dv / 16, a.H * ca.nseq};
  gdn_state_scan<DK><<<sgrid.blocks(), dim3(64 * (DK / 16)), 0, s>>>(a, ca, ws, sgrid);
  if ((rc = check_launch("gdn_state_scan"))) return rc;
  gdn_chunk_out<bf16_t, DK><<<dim3(ca.total_chunks, a.H), dim3(256), 0, s>>>(a, ca, ws, 0);
  return check_launch("gdn_chunk_out");
}

}  // namespace

}  // namespace motif

extern "C" int motif_gdn_prefill_fused(
    const void *proj, int64_t p_sb, int64_t p_st, int q_off, int k_off, int v_off, int g_off, int a_off, int b_off,
    const void *wq, const void *wk, const void *wv, int conv_k,
    const void *tail_q, const void *tail_k, const void *tail_v, void *tail_q_out, void *tail_k_out, void *tail_v_out,
    const void *a_log, const void *dt_bias, float q_scale, const void *norm_weight, float norm_eps,
    const float *state_in, float *state_out, void *y, int64_t y_sb, int64_t y_st,
    int B, int H, int L, int dk, int dv,
    const int32_t *cu_seqlens, const int32_t *chunk_offsets, int nseq, int total_chunks,
    void *workspace, size_t workspace_bytes, void *stream) {
  using namespace motif;
  if (B < 0 || H <= 0 || L < 0 || dk <= 0 || dv <= 0) return set_error(MOTIF_ERR_INVALID, "gdn_prefill: bad size");
  if (!((dk == 32 || dk == 64) && (dv == 64 || dv == 128) && conv_k == kConvK))
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_prefill: dk in {32, 64}, dv in {64, 128} and conv kernel 4 only");
  const bool packed = cu_seqlens != nullptr;
  if (packed && (B != 1 || !chunk_offsets || nseq <= 0))
    return set_error(MOTIF_ERR_INVALID, "gdn_prefill: packed sequences need B == 1, chunk_offsets and nseq > 0");
  if (!packed && nseq != B) return set_error(MOTIF_ERR_INVALID, "gdn_prefill: nseq must equal B");
  if (packed && (tail_q || tail_k || tail_v))
    return set_error(MOTIF_ERR_INVALID, "gdn_prefill: packed sequences start from zero conv tails");
  const int nper = packed ? 0 : (L + kC - 1) / kC;
  if (!packed && total_chunks != B * nper)
    return set_error(MOTIF_ERR_INVALID, "gdn_prefill: total_chunks must be B * ceil(L / 64)");
  if (!proj || !wq || !wk || !wv || !a_log || !dt_bias || !norm_weight || !state_out || !y)
    return set_error(MOTIF_ERR_INVALID, "gdn_prefill: NULL pointer");
  if ((tail_q_out || tail_k_out || tail_v_out) && !(tail_q_out && tail_k_out && tail_v_out))
    return set_error(MOTIF_ERR_INVALID, "gdn_prefill: give all three outgoing tails or none");
  if ((tail_q || tail_k || tail_v) && !(tail_q && tail_k && tail_v))
    return set_error(MOTIF_ERR_INVALID, "gdn_prefill: give all three incoming tails or none");
  const uintptr_t al16 = reinterpret_cast<uintptr_t>(proj) | reinterpret_cast<uintptr_t>(wq) |
                         reinterpret_cast<uintptr_t>(wk) | reinterpret_cast<uintptr_t>(wv);
  const uintptr_t al8 = reinterpret_cast<uintptr_t>(norm_weight) | reinterpret_cast<uintptr_t>(y);
  if ((al16 & 15) || (al8 & 7) || ((p_sb | p_st | q_off | k_off | v_off) & 7) || ((g_off | y_sb | y_st) & 3))
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_prefill: misaligned rows");
  // sequence-relative byte offsets of the range-checked projection loads stay below 2^32
  if ((static_cast<int64_t>(L) + kConvK) * p_st * 2 >= (int64_t(1) << 32))
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_prefill: projection rows too long for the range-checked loads");
  if (nseq == 0 || total_chunks == 0) {
    if (total_chunks != 0 || L != 0) return set_error(MOTIF_ERR_INVALID, "gdn_prefill: inconsistent sizes");
    return MOTIF_OK;
  }
  const size_t need = motif_gdn_chunk_workspace_bytes(H, dk, dv, kC, total_chunks);
  if (!workspace || workspace_bytes < need)
    return set_error(MOTIF_ERR_INVALID, "gdn_prefill: workspace too small (need " + std::to_string(need) + " bytes)");

  GdnArgs a{};
  a.q = a.k = a.v = a.beta = a.g = proj;  // the prep reads the projections through FrontArgs
  a.s_in = state_in; a.s_out = state_out;
  a.o = nullptr;
  a.B = B; a.H = H; a.L = L; a.dk = dk; a.dv = dv;
  a.gate = static_cast<const bf16_t *>(proj) + g_off; a.gt_sb = p_sb; a.gt_st = p_st;
  a.nw = norm_weight; a.neps = norm_eps;
  a.y = y; a.y_sb = y_sb; a.y_st = y_st;
  ChunkArgs ca{};
  ca.cu = cu_seqlens; ca.coff = chunk_offsets; ca.nseq = nseq; ca.nper = nper; ca.total_chunks = total_chunks;
  FrontArgs fa{};
  fa.x = static_cast<const bf16_t *>(proj); fa.x_sb = p_sb; fa.x_st = p_st;
  fa.q_off = q_off; fa.k_off = k_off; fa.v_off = v_off; fa.a_off = a_off; fa.b_off = b_off;
  fa.wq = static_cast<const bf16_t *>(wq); fa.wk = static_cast<const bf16_t *>(wk); fa.wv = static_cast<const bf16_t *>(wv);
  fa.tq = static_cast<const bf16_t *>(tail_q); fa.tk = static_cast<const bf16_t *>(tail_k);
  fa.tv = static_cast<const bf16_t *>(tail_v);
  fa.oq = static_cast<bf16_t *>(tail_q_out); fa.ok = static_cast<bf16_t *>(tail_k_out);
  fa.ov = static_cast<bf16_t *>(tail_v_out);
  fa.a_log = static_cast<const bf16_t *>(a_log); fa.dt_bias = static_cast<const bf16_t *>(dt_bias);
  fa.q_scale = q_scale;
  char *ws = static_cast<char *>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dk == 64) return dv == 128 ? launch_fused<64, 128>(a, ca, fa, ws, s) : launch_fused<64, 64>(a, ca, fa, ws, s);
  return dv == 128 ? launch_fused<32, 128>(a, ca, fa, ws, s) : launch_fused<32, 64>(a, ca, fa, ws, s);
}

namespace motif {


}  // namespace motif
