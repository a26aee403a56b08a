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
// gdn_state_scan carries S across the chunks, one wavefront per (16 state columns,
// head, sequence) holding all dk rows of its columns in accumulator registers (the
// columns of S evolve independently, so no wavefront waits on another), with a
// register prefetch of A_n / H_n several chunks deep (the wavefronts of one head share
// an XCD, so A_n is read from HBM once and from that XCD's L2 after); it writes every
// S_n as MFMA operands.  gdn_chunk_out then forms O_n = O' + Q' S_n for all chunks in
// parallel, with the GatedRMSNorm of each head row fused.
//
// The workspace holds A_n, Q', H_n, O' and S_n as bf16 in the order the consuming
// kernel's lanes read them (one 8- or 16-byte piece per lane per operand tile), so
// every load of the two later kernels is a coalesced wavefront access with no LDS
// staging.  Rounding these five to bf16 moves the output by about 2^-9 of its size
// and the final state by ~2e-3 (relative), inside the bf16 bar.
//
// Inputs are bf16 (exact as MFMA operands).  Inside the prep, fp32-derived operands
// (T, N, Attn, K~, M) are split into bf16 hi + lo and their products take three MFMA
// passes (hi.hi + hi.lo + lo.hi, fp32 accumulation), products with an exact bf16
// operand two: about 16 mantissa bits per product, fp32 accumulation throughout.
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

// Workspace per (head, chunk) cell, bf16, every piece 8 or 16 bytes per lane of a
// 64-lane tile:
//   an [DK/16 mt][DK/32 ks][64]   bf16x8  A_n rows 16 mt + (l % 16), k slots
//                                         32 ks + 4 (l / 16) + {0..3, 16..19}
//   qp [4 mt][DK/32 ks][64]       bf16x8  Q' in the same operand order
//   hn [dv/16 cg][DK/16 mt][64]   bf16x4  H_n[16 mt + 4 (l / 16) + r][16 cg + l % 16]
//   op [dv/16 cg][4 mt][64]       bf16x4  O'[16 mt + l % 16][16 cg + 4 (l / 16) + r]
//   sn [dv/16 cg][DK/32 ks][64]   bf16x8  S_n rows 32 ks + 4 (l / 16) + {0..3, 16..19},
//                                         column 16 cg + l % 16
struct WsLayout {
  size_t an, qp, hn, op, sn, cell;
  __host__ __device__ WsLayout(int dk, int dv) {
    an = 0;
    qp = an + 2ull * dk * dk;
    hn = qp + 2ull * kC * dk;
    op = hn + 2ull * dk * dv;
    sn = op + 2ull * kC * dv;
    cell = sn + 2ull * dk * dv;
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

// Byte offsets of the prep kernel's LDS (planes of [rows][64] bf16 are swizzled, swz):
//   A: [K rows | spare | Q rows | K^T] 8 KB each.  The K and Q rows and the exact K^T
//      plane are written in phase 1; after phase 2 the exact V^T plane [DV][64] goes
//      over the K rows and the spare piece.  The Q rows stay for phase 7 (Q').
//   B: NT, one fp32 [64][68] array holding N = strict(beta K K^T * D) below the
//      diagonal and T^T on and above it (phases 2-6), then T^T as bf16 hi / lo planes
//      [64][64], rows j, columns i (phases 6-7).
// 49.5 KB at dk = 64, dv = 128: three workgroups per CU.
template <int DK, int DV>
struct PrepLayout {
  static constexpr int kPlane = 64 * 64 * 2;
  static constexpr int kh = 0, vt = 0, qh = 2 * kPlane, kt = 3 * kPlane;
  static_assert(DV * 128 <= 2 * kPlane && DK * 128 <= kPlane, "V^T / K^T planes exceed their pieces");
  static constexpr int nt = 4 * kPlane, tt_h = nt, tt_l = nt + kPlane;
  // gam[64], beta[64], ek[64] = e^{gamma_C - gamma}, sb[64] = beta e^gamma
  static constexpr int small = nt + (64 * 68 * 4 > 2 * kPlane ? 64 * 68 * 4 : 2 * kPlane);
  static constexpr int bytes = small + 4 * 64 * 4;
};

// v_mfma_f32_32x32x16_bf16: A lane l holds row l % 32, k 8 (l / 32) + 0..7; B lane l
// column l % 32, the same k; accumulator register r of lane l holds row
// 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
__device__ __forceinline__ f32x16 mma32(const bf16x8 &a, const bf16x8 &b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// The 16 k of one 32x32x16 step as an operand built from accumulator rows: slot s of
// lane half h stands for k = 16 ks + 8 (s / 4) + 4 h + s % 4, so a B operand comes
// straight from accumulator registers 8 (ks % 2) .. +7 of the same lane.  A row-major
// LDS operand in that order is two 8-byte reads, columns 16 ks + 4 h and + 8.
__device__ __forceinline__ bf16x8 rd_pair_s(const __bf16 *p, int row, int c0) {
  return __builtin_shufflevector(rd4s(p, row, c0), rd4s(p, row, c0 + 8), 0, 1, 2, 3, 4, 5, 6, 7);
}

template <int DK, int DV, bool FRONT>
__global__ void __launch_bounds__(256, 3) gdn_prep_mfma(GdnArgs a, ChunkArgs ca, char *ws, FrontArgs fa) {
  using TI = bf16_t;
  using PL = PrepLayout<DK, DV>;
  constexpr int NTS = 68;  // NT row stride (floats)
  extern __shared__ __attribute__((aligned(16))) char smem[];
  __bf16 *tt_h = reinterpret_cast<__bf16 *>(smem + PL::tt_h), *tt_l = reinterpret_cast<__bf16 *>(smem + PL::tt_l);
  __bf16 *kt = reinterpret_cast<__bf16 *>(smem + PL::kt), *vt = reinterpret_cast<__bf16 *>(smem + PL::vt);
  __bf16 *kh = reinterpret_cast<__bf16 *>(smem + PL::kh), *qh = reinterpret_cast<__bf16 *>(smem + PL::qh);
  float *nt = reinterpret_cast<float *>(smem + PL::nt);
  float *gam = reinterpret_cast<float *>(smem + PL::small), *bet = gam + 64, *ek = gam + 128, *sb = gam + 192;

  const int chunk = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, g = lane >> 4;
  const ChunkInfo ci = resolve_chunk(chunk, kC, a.L, ca);
  // wavefront 0, lane = chunk row: the gates and the per-row decay factors phase 7 scales by
  auto put_gates = [&](float gsum, float b) {
    gam[lane] = gsum;
    bet[lane] = b;
    ek[lane] = exp_fast(__shfl(gsum, 63, 64) - gsum);
    sb[lane] = b * exp_fast(gsum);
  };

  // variables phase 1 leaves for the later phases (the FRONT form uses its own)
  constexpr int KSEG = DK / 8, VP = 32 * (DV / 8) / 256;
  const int kp = tid & 31, kseg = tid >> 5;
  const bool kval = kseg < KSEG;
  uint4 k0r = {}, k1r = {}, v0r[VP], v1r[VP];
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
    if (w == 0) {  // the inclusive prefix sum of g
      float s = gv;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(s, off, 64);
        if (lane >= off) s += y;
      }
      put_gates(s, bv);
    }
    if (kval) {
      *reinterpret_cast<uint4 *>(kh + swz(2 * kp, 8 * kseg)) = k0r;
      *reinterpret_cast<uint4 *>(kh + swz(2 * kp + 1, 8 * kseg)) = k1r;
      *reinterpret_cast<uint4 *>(qh + swz(2 * kp, 8 * kseg)) = q0r;
      *reinterpret_cast<uint4 *>(qh + swz(2 * kp + 1, 8 * kseg)) = q1r;
      // the K^T plane (its own region) from the same registers
      const bf16x8 ka = __builtin_bit_cast(bf16x8, k0r), kb_ = __builtin_bit_cast(bf16x8, k1r);
#pragma unroll
      for (int t = 0; t < 8; ++t)
        *reinterpret_cast<uint32_t *>(kt + swz(8 * kseg + t, 2 * kp)) = pack2(bits(ka[t]), bits(kb_[t]));
    }
  
  } else {
    // ---- phase 1 (fused front end): wave 0 convolves q, wave 1 k, waves 2-3 v.  A
    // thread walks R consecutive chunk rows of one 8-channel segment with the conv
    // window in registers; the S segments of a row are S adjacent lanes, so the q / k
    // L2 norm of a row is a butterfly over them.  Arithmetic as the standalone conv
    // kernel: fp32 conv accumulation, then the reference layer's bf16 roundings (conv
    // output, SiLU, norm, quotient, scaled q).
    constexpr int KC = kConvK;
    const int prob = w < 2 ? w : 2;
    const int C = prob < 2 ? DK : DV;
    const int S = C / 8;
    const int t = prob < 2 ? lane : tid - 128;
    const int rows = prob < 2 ? RQ : RV;  // wave-uniform
    f_seg = t % S;
    f_r0 = (t / S) * rows;
    const int chan = h * C + 8 * f_seg;
    const int col0 = (prob == 0 ? fa.q_off : prob == 1 ? fa.k_off : fa.v_off) + h * C;  // the wave's head slice
    const bf16_t *wgt = (prob == 0 ? fa.wq : prob == 1 ? fa.wk : fa.wv) + static_cast<size_t>(chan) * KC;
    const bf16_t *tin = ca.cu ? nullptr : (prob == 0 ? fa.tq : prob == 1 ? fa.tk : fa.tv);
    const int s_lo = ca.cu ? ca.cu[ci.seq] : 0, s_hi = ca.cu ? ca.cu[ci.seq + 1] : a.L;
    // one buffer over the wave's head slice of the sequence's rows (a uniform resource:
    // a per-lane base would make every load a loop over the lanes' distinct bases); rows
    // outside [s_lo, s_hi) read zeros (a token before the start wraps to a huge offset,
    // the segment's 16 f_seg bytes staying below one row)
    const bf16_t *xs = fa.x + ci.batch * fa.x_sb + int64_t(s_lo) * fa.x_st + col0;
    const buf_t xbuf = make_buf(xs, s_hi > s_lo ? static_cast<uint32_t>(((s_hi - s_lo - 1) * fa.x_st + C) * 2) : 0u);
    const int rel0 = ci.t0 - s_lo + f_r0;  // sequence offset of this thread's first row
    // the gate inputs of row `lane` (clamped to the chunk; zeroed past len below), issued
    // ahead of the conv inputs so that wave 0 forms the gates while those are in flight
    // (every wave loads them: no branch around the batch of loads)
    const bf16_t *xg = fa.x + ci.batch * fa.x_sb + int64_t(ci.t0 + min(lane, ci.len - 1)) * fa.x_st;
    const bf16_t g_a = xg[fa.a_off + h], g_b = xg[fa.b_off + h];
    const bf16_t g_dt = fa.dt_bias[h], g_al = fa.a_log[h];
    uint4 raw[KC - 1 + RM];
#pragma unroll
    for (int i = 0; i < KC - 1 + RM; ++i)
      if (i < KC - 1 + rows)
        raw[i] = buf_ld16(xbuf, static_cast<uint32_t>((rel0 - (KC - 1) + i) * fa.x_st * 2 + 16 * f_seg));
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
    // gates of the chunk's rows (zero past len, as the unfused loads read them)
    if (w == 0) {
      float gv = 0.f, bv = 0.f;
      if (lane < ci.len) {
        // beta = T(sigmoid(b)), g = T(-T(exp(A_log)) * T(softplus(T(a + dt_bias)))), threshold 20
        const float xa = fl(bf(bf16_to_f32(g_a) + bf16_to_f32(g_dt)));
        const float sp = fl(bf(xa > 20.f ? xa : log1pf(expf(xa))));
        const float A = fl(bf(expf(bf16_to_f32(g_al))));
        bv = fl(bf(1.f / (1.f + expf(-bf16_to_f32(g_b)))));
        gv = fl(bf(-A * sp));
      }
      float sacc = gv;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(sacc, off, 64);
        if (lane >= off) sacc += y;
      }
      put_gates(sacc, bv);
    }
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
          v[e] = live ? gdn_conv_act<bf16_t>(acc) : 0.f;
          ss = fmaf(v[e], v[e], ss);
#pragma unroll
          for (int r = 0; r < KC - 2; ++r) win[r][e] = win[r + 1][e];
          win[KC - 2][e] = xt[e];
        }
        if (prob < 2) {
#pragma unroll
          for (int off = 1; off < 8; off <<= 1)
            if (off < S) ss += __shfl_xor(ss, off, 64);
          const float inv = gdn_norm_inv<bf16_t>(ss);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = gdn_normalized<bf16_t>(v[e], inv, scale);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) cv[i][e] = pk_bf16(v[2 * e], v[2 * e + 1]);
        if (prob < 2)
          *reinterpret_cast<uint4 *>((prob == 0 ? qh : kh) + swz(f_r0 + i, 8 * f_seg)) =
              uint4{cv[i][0], cv[i][1], cv[i][2], cv[i][3]};
      }
    }
    if (w == 1) {  // the K^T plane (its own region) from this thread's K rows, in pairs
#pragma unroll
      for (int i = 0; i < RQ; i += 2) {
        const int j = f_r0 + i;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint16_t b0 = static_cast<uint16_t>(cv[i][e >> 1] >> (16 * (e & 1)));
          const uint16_t b1 = static_cast<uint16_t>(cv[i + 1][e >> 1] >> (16 * (e & 1)));
          *reinterpret_cast<uint32_t *>(kt + swz(8 * f_seg + e, j)) = pack2(b0, b1);
        }
      }
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

  // ---- phase 2 on 32x32x16 products (k = the dk columns of the K / Q rows in LDS).
  // Waves 0, 1: N = strict(beta K K^T * D), rows 32 w .. +31, into NT (the tile right
  // of the diagonal block is zero and skipped; entries on and above the diagonal are
  // written as zeros, where T goes later).  Waves 2, 3: Attn^T = (K Q^T) * D^T for the
  // 32 queries m = 32 (w - 2) + l % 32, kept in registers as the hi / lo B operands
  // of phase 7 (k = key row i, in the slot order of rd_pair_s), plus the Q row pieces
  // that Q' needs.
  const int lc = lane & 31, hh = lane >> 5;
  bf16x8 ath[4], atl[4];    // Attn^T B operands, k-step ks
  if (w < 2) {
    const int i0 = 32 * w;
    for (int jt = 0; jt <= w; ++jt) {
      f32x16 acc = {};
#pragma unroll
      for (int kd = 0; kd < DK / 16; ++kd)
        acc = mma32(rd8s(kh, i0 + lc, 16 * kd + 8 * hh), rd8s(kh, 32 * jt + lc, 16 * kd + 8 * hh), acc);
      const int j = 32 * jt + lc;
      const float gj = gam[j];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = i0 + 8 * (r >> 2) + 4 * hh + (r & 3);
        const float val = bet[i] * acc[r] * exp_fast(gam[i] - gj);
        nt[i * NTS + j] = j < i ? val : 0.f;
      }
    }
  } else {
    const int m = 32 * (w - 2) + lc;
    const float gm = gam[m];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      f32x16 acc = {};
      if (it <= w - 2) {  // key tiles past the query tile are masked whole
#pragma unroll
        for (int kd = 0; kd < DK / 16; ++kd)
          acc = mma32(rd8s(kh, 32 * it + lc, 16 * kd + 8 * hh), rd8s(qh, m, 16 * kd + 8 * hh), acc);
      }
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * it + 8 * (r >> 2) + 4 * hh + (r & 3);
        const float val = acc[r] * exp_fast(gm - gam[i]);
        x[r] = i <= m ? val : 0.f;
      }
      split8(x, ath[2 * it], atl[2 * it]);
      split8(x + 8, ath[2 * it + 1], atl[2 * it + 1]);
    }
  }
  __syncthreads();

  // ---- V^T plane over the dead K rows and the spare piece (read in phase 7 only,
  // after several barriers), freeing the registers that hold V.
  if constexpr (!FRONT) {
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
  // Wave w = (ti, tj) forms both row tiles of column tile tj of Y = N[32:, :32] T[:32, :32]
  // itself, so the second product takes Y from its own registers (k in the slot order
  // {4g .. 4g + 3, 16 + 4g .. + 3}), with no exchange.  Phase 5 reads NT rows 32.. and
  // the block T[:32, :32] and writes only the block T[32:, :32] (NT rows 0-31, columns
  // 32-63), so it needs no barrier inside.
  {
    const int ti = w >> 1, tj = w & 1;
    f32x4 y[2];
#pragma unroll
    for (int yi = 0; yi < 2; ++yi) {
      float av[8], bv[8];
      const float *nrow = nt + (32 + 16 * yi + ln) * NTS + 8 * g;
      const float *trow = nt + (16 * tj + ln) * NTS + 8 * g;  // T[8g + t][16 tj + ln]
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        av[t] = nrow[t];
        bv[t] = (8 * g + t >= 16 * tj + ln) ? trow[t] : 0.f;
      }
      bf16x8 ah, al, bh, bl;
      split8(av, ah, al);
      split8(bv, bh, bl);
      y[yi] = mma3<true, true>(ah, al, bh, bl, f32x4{0.f, 0.f, 0.f, 0.f});  // Y[16 yi + 4g + r][16 tj + ln]
    }
    // T[32 + 16 ti + m][16 tj + n] = -sum_k T[32 + 16 ti + m][32 + k] Y[k][16 tj + n]
    float av[8], bv[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int k = t < 4 ? 4 * g + t : 16 + 4 * g + (t - 4);
      av[t] = (k <= 16 * ti + ln) ? nt[(32 + k) * NTS + 32 + 16 * ti + ln] : 0.f;
      bv[t] = t < 4 ? y[0][t] : y[1][t - 4];
    }
    bf16x8 ah, al, bh, bl;
    split8(av, ah, al);
    split8(bv, bh, bl);
    const f32x4 o = mma3<true, true>(ah, al, bh, bl, f32x4{0.f, 0.f, 0.f, 0.f});
    *reinterpret_cast<f32x4 *>(nt + (16 * tj + ln) * NTS + 32 + 16 * ti + 4 * g) = -o;
  }
  __syncthreads();

  // ---- phase 6: T^T as bf16 hi / lo planes, written over NT once every thread holds
  // its 16 entries.
  {
    const int j = tid >> 2, i0 = 16 * (tid & 3);
    float x[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) x[t] = (i0 + t >= j) ? nt[j * NTS + i0 + t] : 0.f;
    bf16x8 h0, l0, h1, l1;
    split8(x, h0, l0);
    split8(x + 8, h1, l1);
    __syncthreads();
    *reinterpret_cast<bf16x8 *>(tt_h + swz(j, i0)) = h0;
    *reinterpret_cast<bf16x8 *>(tt_l + swz(j, i0)) = l0;
    *reinterpret_cast<bf16x8 *>(tt_h + swz(j, i0 + 8)) = h1;
    *reinterpret_cast<bf16x8 *>(tt_l + swz(j, i0 + 8)) = l1;
  }
  const float glast = gam[kC - 1];
  __syncthreads();
  // ---- phase 7: wave w takes a 32-row tile of M = [K~^T ; Attn] T: top tiles
  // (w < DK / 32) rows d' of K~^T T, bottom tiles (waves 2, 3) rows i' of Attn T.
  // M^T (rows j, columns m) = T^T L^T on 32x32x16 MFMAs, A = T^T (hi / lo planes), B =
  // K~ (K^T plane times e^{gamma_C - gamma_i}, split here) or Attn^T (registers).  The
  // M^T accumulator, scaled per row j, is already in the slot order of a B operand
  // (and, for the same lane, of an A operand over k = j), so
  //   Z^T = K^T (diag(beta e^gamma) M^T)    -> A_n = e^{gamma_C} I - Z,  Q' = Q e^gamma - Z
  //   Y   = (M diag(beta)) V (top: H_n),  Y^T = V^T (diag(beta) M^T) (bottom: O')
  // take their M operands straight from registers.  Each result goes to the workspace
  // as bf16 in 8-byte pieces of the consuming kernel's operand order.
  const WsLayout Lw(DK, a.dv);
  char *cell = ws + (static_cast<size_t>(h) * ca.total_chunks + chunk) * Lw.cell;
  // (one specialised body per tile kind: no wave-uniform branches inside its loops)
  auto phase7 = [&](auto top_c) {
    constexpr bool top = decltype(top_c)::value;
    const int tile = top ? w : w - 2;
    const int m = 32 * tile + lc;  // d' (top) or i' (bottom): this lane's column of M^T
    bf16x8 bh[4], bl[4];
    if (top) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 kv = rd_pair_s(kt, m, 16 * ks + 4 * hh);
        float x[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) x[t] = fl(kv[t]) * ek[16 * ks + 8 * (t >> 2) + 4 * hh + (t & 3)];
        split8(x, bh[ks], bl[ks]);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        bh[ks] = ath[ks];
        bl[ks] = atl[ks];
      }
    }
    // M^T rows j = 32 jt + 8 (r / 4) + 4 hh + r % 4
    f32x16 mt2[2];
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) {
      f32x16 acc = {};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (jt == 1 && ks < 2) continue;  // T^T rows j >= 32 vanish on columns i < 32
        const bf16x8 th = rd_pair_s(tt_h, 32 * jt + lc, 16 * ks + 4 * hh);
        const bf16x8 tl = rd_pair_s(tt_l, 32 * jt + lc, 16 * ks + 4 * hh);
        acc = mma32(tl, bh[ks], acc);
        acc = mma32(th, bl[ks], acc);
        acc = mma32(th, bh[ks], acc);
      }
      mt2[jt] = acc;
    }
    // operands over k = j of diag(s) M^T, s = beta e^gamma (K side) or beta (V side)
    auto m_operands = [&](bool kside, bf16x8 *oh, bf16x8 *ol) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        float x[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const int r = 8 * (ks & 1) + t, j = 16 * ks + 8 * (t >> 2) + 4 * hh + (t & 3);
          x[t] = mt2[ks >> 1][r] * (kside ? sb[j] : bet[j]);
        }
        split8(x, oh[ks], ol[ks]);
      }
    };
    bf16x8 oh[4], ol[4];
    m_operands(true, oh, ol);
    // Z^T[d][m] = sum_j K^T[d][j] (s M^T)[j][m]; z[r]: d = 32 dt + 8 (r / 4) + 4 hh + r % 4
    const float eq = top ? exp_fast(glast) : exp_fast(gam[m]);
    char *zbase = cell + (top ? Lw.an : Lw.qp);
#pragma unroll
    for (int dt = 0; dt < DK / 32; ++dt) {
      f32x16 z = {};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 ka = rd_pair_s(kt, 32 * dt + lc, 16 * ks + 4 * hh);
        z = mma32(ka, ol[ks], z);
        z = mma32(ka, oh[ks], z);
      }
      // rows m, columns d = 32 dt + 8 q + 4 hh + p (p = 0..3): tile mt = m / 16, k-step
      // dt, lane (m % 16) + 16 (2 (q % 2) + hh), half q / 2
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bf16x4 qrow = top ? bf16x4{} : rd4s(qh, m, 32 * dt + 8 * q + 4 * hh);
        float x[4];
#pragma unroll
        for (int p4 = 0; p4 < 4; ++p4) {
          const int d = 32 * dt + 8 * q + 4 * hh + p4;
          x[p4] = (top ? (d == m ? eq : 0.f) : fl(qrow[p4]) * eq) - z[4 * q + p4];
        }
        const size_t o = ((static_cast<size_t>(m >> 4) * (DK / 32) + dt) * 64 + (m & 15) + 16 * (2 * (q & 1) + hh)) * 16 +
                         8 * (q >> 1);
        *reinterpret_cast<uint2 *>(zbase + o) = uint2{pk_bf16(x[0], x[1]), pk_bf16(x[2], x[3])};
      }
    }
    m_operands(false, oh, ol);
    bf16_t *yb = reinterpret_cast<bf16_t *>(cell + (top ? Lw.hn : Lw.op));
    for (int vt2 = 0; vt2 < a.dv / 32; ++vt2) {
      f32x16 y = {};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 vv = rd_pair_s(vt, 32 * vt2 + lc, 16 * ks + 4 * hh);
        if (top) {
          y = mma32(ol[ks], vv, y);
          y = mma32(oh[ks], vv, y);
        } else {
          y = mma32(vv, ol[ks], y);
          y = mma32(vv, oh[ks], y);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        size_t o;
        if (top) {  // H_n[d' = 32 tile + 8 q + 4 hh + p][v = 32 vt2 + lc], layout [cg][DK/16][64] x 4
          const int cg = 2 * vt2 + (lc >> 4), mt = 2 * tile + (q >> 1);
          o = ((static_cast<size_t>(cg) * (DK / 16) + mt) * 64 + (lc & 15) + 16 * (2 * (q & 1) + hh)) * 4;
        } else {    // O'[m][v = 32 vt2 + 8 q + 4 hh + p], layout [cg][4][64] x 4
          const int cg = 2 * vt2 + (q >> 1), mt = m >> 4;
          o = ((static_cast<size_t>(cg) * 4 + mt) * 64 + (m & 15) + 16 * (2 * (q & 1) + hh)) * 4;
        }
        *reinterpret_cast<uint2 *>(yb + o) = uint2{pk_bf16(y[4 * q], y[4 * q + 1]), pk_bf16(y[4 * q + 2], y[4 * q + 3])};
      }
    }
  };
  if (w < DK / 32) phase7(BoolC<true>{});
  else if (w >= 2) phase7(BoolC<false>{});
}

// ------------------------------------------------------------------ state scan
// A_n / H_n of one chunk as one wavefront of the scan needs them.
template <int DK>
struct ScanStage {
  uint4 an[DK / 16][DK / 32];  // A_n operand rows, every row tile
  uint2 hn[DK / 16];           // H_n tiles of this column group (bf16, accumulator layout)
};

// Loads of one chunk through a buffer over the group's cells: the chunk's byte offset
// is the (uniform) soffset, so a stage costs no address registers.
template <int DK>
__device__ __forceinline__ void scan_load(ScanStage<DK> &st, buf_t cells, uint32_t cell_off, uint32_t an_v,
                                          uint32_t hn_v) {
  constexpr int TDK = DK / 16, KS = DK / 32;
#pragma unroll
  for (int mt = 0; mt < TDK; ++mt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      st.an[mt][ks] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(cells, an_v + (mt * KS + ks) * 1024, cell_off, 0));
#pragma unroll
  for (int mt = 0; mt < TDK; ++mt)
    st.hn[mt] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(cells, hn_v + mt * 512, cell_off, 0));
}

// One wavefront per (16 state columns, head, sequence) holds all DK rows of its columns:
// tile mt, S[mt][r] = S[16 mt + 4g + r][16 cg + l % 16].  S_{n+1} = A_n S_n + H_n mixes
// rows only, so the wavefront needs no other's columns: the B operand of k-step ks is
// the bf16 rounding of its own tiles 2 ks (slots 0..3) and 2 ks + 1 (slots 4..7), i.e.
// k slots 32 ks + 4g + {0..3, 16..19} in the order A_n's operand rows are stored, and
// that same operand is the S_n piece the output kernel reads.  Per chunk DK/16 x DK/32
// MFMAs in DK/16 independent chains, no LDS and no barrier.
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
__global__ void __launch_bounds__(64) gdn_state_scan(GdnArgs a, ChunkArgs ca, char *ws, ScanGrid sgrid) {
  constexpr int TDK = DK / 16, KS = DK / 32;
  const int slot = blockIdx.x / ScanGrid::kXcd;
  const int group = (slot / sgrid.ncg) * ScanGrid::kXcd + blockIdx.x % ScanGrid::kXcd;
  if (group >= sgrid.ngroups) return;
  const int cg = slot % sgrid.ncg, h = group % a.H, sq = group / a.H;

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

  const int lane = threadIdx.x;
  const int ln = lane & 15, g = lane >> 4;
  const int col = 16 * cg + ln;

  f32x4 S[TDK];
  const size_t sbase = (static_cast<size_t>(sq) * a.H + h) * DK * a.dv;
#pragma unroll
  for (int mt = 0; mt < TDK; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      S[mt][r] = a.s_in ? a.s_in[sbase + static_cast<size_t>(16 * mt + 4 * g + r) * a.dv + col] : 0.f;

  // kScanDepth stages of A_n / H_n in flight (chunk n + kScanDepth is requested while
  // chunk n is computed)
  constexpr int kScanDepth = DK == 64 ? 4 : 8;
  const uint32_t cell_bytes = static_cast<uint32_t>(Lw.cell);
  const buf_t cells = make_buf(cell0, static_cast<uint32_t>(count) * cell_bytes);
  const uint32_t an_v = static_cast<uint32_t>(Lw.an) + 16u * lane;
  const uint32_t hn_v = static_cast<uint32_t>(Lw.hn) + static_cast<uint32_t>(cg) * TDK * 512u + 8u * lane;
  ScanStage<DK> st[kScanDepth];
  if (count > 0) {
#pragma unroll
    for (int j = 0; j < kScanDepth; ++j) scan_load<DK>(st[j], cells, min(j, count - 1) * cell_bytes, an_v, hn_v);
  }

  // S_n as bf16 operands (stored for the output kernel), then S_{n+1}; the stage is
  // then refilled with chunk min(n + kScanDepth, count - 1) (a repeat load of the last
  // chunk near the end keeps the loop free of branches).
  auto step = [&](ScanStage<DK> &stg, int n) {
    char *cell = cell0 + static_cast<size_t>(n) * Lw.cell;
    uint4 sb[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      sb[ks] = uint4{pk_bf16(S[2 * ks][0], S[2 * ks][1]), pk_bf16(S[2 * ks][2], S[2 * ks][3]),
                     pk_bf16(S[2 * ks + 1][0], S[2 * ks + 1][1]), pk_bf16(S[2 * ks + 1][2], S[2 * ks + 1][3])};
    uint4 *sn = reinterpret_cast<uint4 *>(cell + Lw.sn) + static_cast<size_t>(cg) * KS * 64 + lane;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) sn[ks * 64] = sb[ks];
#pragma unroll
    for (int mt = 0; mt < TDK; ++mt) {
      const uint2 hv = stg.hn[mt];
      f32x4 acc = {__uint_as_float(hv.x << 16), __uint_as_float(hv.x & 0xffff0000u),
                   __uint_as_float(hv.y << 16), __uint_as_float(hv.y & 0xffff0000u)};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        acc = mma(__builtin_bit_cast(bf16x8, stg.an[mt][ks]), __builtin_bit_cast(bf16x8, sb[ks]), acc);
      S[mt] = acc;
    }
    scan_load<DK>(stg, cells, min(n + kScanDepth, count - 1) * cell_bytes, an_v, hn_v);
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
  for (int mt = 0; mt < TDK; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) a.s_out[sbase + static_cast<size_t>(16 * mt + 4 * g + r) * a.dv + col] = S[mt][r];
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

  // gate and norm-weight pieces of the fused GatedRMSNorm, requested before the products
  uint2 gv[kMaxCg][4], nwv[kMaxCg];
  if (a.gate) {
#pragma unroll
    for (int i = 0; i < kMaxCg; ++i)
      nwv[i] = *reinterpret_cast<const uint2 *>(static_cast<const bf16_t *>(a.nw) + 16 * min(w + 4 * i, ncg - 1) + 4 * g);
    const bf16_t *gp = static_cast<const bf16_t *>(a.gate) + ci.batch * a.gt_sb + int64_t(ci.t0) * a.gt_st + h * a.dv;
#pragma unroll
    for (int i = 0; i < kMaxCg; ++i)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = min(16 * mt + ln, ci.len - 1), c0 = 16 * min(w + 4 * i, ncg - 1) + 4 * g;
        gv[i][mt] = *reinterpret_cast<const uint2 *>(gp + int64_t(row) * a.gt_st + c0);
      }
  }

  bf16x8 qh[4][KS];
  const uint4 *qp = reinterpret_cast<const uint4 *>(cell + Lw.qp) + lane;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qh[mt][ks] = __builtin_bit_cast(bf16x8, qp[(mt * KS + ks) * 64]);
  // O tiles of this wave's column groups cg = w + 4 i: lane holds O[16 mt + ln][16 cg + 4 g + r]
  // S_n and O' pieces of every column group of the wave, requested before any product
  // (a group whose index passes ncg loads the last group again and is skipped below)
  uint4 snv[kMaxCg][KS];
  uint2 opv[kMaxCg][4];
#pragma unroll
  for (int i = 0; i < kMaxCg; ++i) {
    const int cgl = min(w + 4 * i, ncg - 1);
    const uint4 *sn = reinterpret_cast<const uint4 *>(cell + Lw.sn) + static_cast<size_t>(cgl) * KS * 64 + lane;
    const uint2 *op = reinterpret_cast<const uint2 *>(cell + Lw.op) + static_cast<size_t>(cgl) * 4 * 64 + lane;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) snv[i][ks] = sn[ks * 64];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) opv[i][mt] = op[mt * 64];
  }
  f32x4 res[kMaxCg][4];
#pragma unroll
  for (int i = 0; i < kMaxCg; ++i) {
    const int cg = w + 4 * i;
    if (cg >= ncg) break;
    bf16x8 sh[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) sh[ks] = __builtin_bit_cast(bf16x8, snv[i][ks]);
    f32x4 acc[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const uint2 ov = opv[i][mt];
      acc[mt] = f32x4{__uint_as_float(ov.x << 16), __uint_as_float(ov.x & 0xffff0000u),
                      __uint_as_float(ov.y << 16), __uint_as_float(ov.y & 0xffff0000u)};
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) acc[mt] = mma(sh[ks], qh[mt][ks], acc[mt]);
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
    const uint2 wraw = nwv[i];
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
  gdn_state_scan<DK><<<sgrid.blocks(), dim3(64), 0, s>>>(a, ca, ws, sgrid);
  if ((rc = check_launch("gdn_state_scan"))) return rc;
  // 8-byte output stores when every row start is 8-byte aligned
  const int vec = ((a.o_sb | a.o_sh | a.o_st) & 3) == 0 && (reinterpret_cast<uintptr_t>(a.o) & 7) == 0;
  gdn_chunk_out<bf16_t, DK><<<dim3(ca.total_chunks, a.H), dim3(256), 0, s>>>(a, ca, ws, vec);
  return check_launch("gdn_chunk_out");
}

}  // namespace

bool chunk_mfma_supported(int dk, int dv, int chunk) {
  return chunk == kC && (dk == 32 || dk == 64) && dv % 32 == 0 && dv > 0 && dv <= 128;
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
  gdn_state_scan<DK><<<sgrid.blocks(), dim3(64), 0, s>>>(a, ca, ws, sgrid);
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
