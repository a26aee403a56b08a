// GDN chunked prefill on bf16 MFMA (gfx950), chunk length 64.
//
// Two kernels.  gdn_prep_mfma runs one workgroup per (chunk, head) and does all
// the work that does not depend on the carried state: gamma = cumsum(g),
// G = K K^T and Q K^T on MFMA, A = -strict(beta G * D), W and U by forward
// substitution (I - A) [W | U] = [beta e^gamma K | beta V], and then the chunk
// transition and output operators on MFMA:
//   A_n = e^{gamma_C} I - K~^T W      (dk x dk)      K~ = K e^{gamma_C - gamma}
//   H_n = K~^T U                      (dk x dv)
//   Q'  = Q e^{gamma} - Attn W        (C x dk)       Attn = (Q K^T) * D
//   O'  = Attn U                      (C x dv)
// so that for the state S_n entering chunk n
//   S_{n+1} = A_n S_n + H_n,   O_n = O' + Q' S_n.
// gdn_scan_mfma then carries S across the chunks: one workgroup per (64-column
// value tile, head, sequence), one wave per 16 columns, S held in MFMA
// accumulator layout in registers; each chunk is one A_n S and one Q' S product
// (next chunk's operators prefetched into LDS while the current one computes).
//
// Inputs are bf16 (exact as MFMA operands).  fp32-derived operands (T-solved W
// and U, Attn, K~, A_n, Q', the state) are split into bf16 hi + lo and products
// take three MFMA passes (hi.hi + hi.lo + lo.hi, fp32 accumulation): about 16
// mantissa bits per product, fp32 accumulation everywhere.
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

// Workspace layout per (head, chunk) cell: An hi/lo [dk][dk] bf16, Qp hi/lo
// [C][dk] bf16, Hn [dk][dv] fp32, Op [C][dv] fp32.
struct WsLayout {
  size_t an, qp, hn, op, cell;
  __host__ __device__ WsLayout(int dk, int dv) {
    an = 0;
    qp = an + 2ull * dk * dk * 2;
    hn = qp + 2ull * kC * dk * 2;
    op = hn + 4ull * dk * dv;
    cell = op + 4ull * kC * dv;
  }
};

// ------------------------------------------------------------------ prep
template <int DK, int DV>
struct PrepSmem {
  __bf16 kh[kC][DK + kPad];                        // K rows (bf16 inputs are exact)
  __bf16 qh[kC][DK + kPad];                        // Q rows
  __bf16 kth[DK][kC + kPad], ktl[DK][kC + kPad];   // K~^T
  __bf16 ath[kC][kC + kPad], atl[kC][kC + kPad];   // Attn
  __bf16 wth[DK][kC + kPad], wtl[DK][kC + kPad];   // W^T
  __bf16 uth[DV][kC + kPad], utl[DV][kC + kPad];   // U^T
  float A[kC][kC + 4];                             // strictly lower A (16-byte rows)
  float gam[kC], beta[kC], zk[kC], eg[kC];
};

template <int DK, int DV>
__global__ void __launch_bounds__(256) gdn_prep_mfma(GdnArgs a, ChunkArgs ca, char *ws) {
  using TI = bf16_t;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  PrepSmem<DK, DV> &sm = *reinterpret_cast<PrepSmem<DK, DV> *>(smem_raw);

  const int chunk = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int ln = lane & 15, g = lane >> 4;
  const ChunkInfo ci = resolve_chunk(chunk, kC, a.L, ca);

  const TI *qb = static_cast<const TI *>(a.q) + ci.batch * a.q_sb + h * a.q_sh + int64_t(ci.t0) * a.q_st;
  const TI *kb = static_cast<const TI *>(a.k) + ci.batch * a.k_sb + h * a.k_sh + int64_t(ci.t0) * a.k_st;
  const TI *vb = static_cast<const TI *>(a.v) + ci.batch * a.v_sb + h * a.v_sh + int64_t(ci.t0) * a.v_st;
  const TI *bb = static_cast<const TI *>(a.beta) + ci.batch * a.b_sb + h * a.b_sh + int64_t(ci.t0) * a.b_st;
  const TI *gb = static_cast<const TI *>(a.g) + ci.batch * a.g_sb + h * a.g_sh + int64_t(ci.t0) * a.g_st;

  // K, Q rows (zero past the chunk's valid length): 16-byte loads, all in flight together.
  constexpr int PT = kC * DK / 8 / 256;  // 16-byte pieces per thread and matrix
  uint4 kr[PT], qr[PT];
#pragma unroll
  for (int r = 0; r < PT; ++r) {
    const int p = tid + 256 * r, i = p / (DK / 8), c8 = p % (DK / 8);
    const bool ok = i < ci.len;
    kr[r] = ok ? *reinterpret_cast<const uint4 *>(kb + int64_t(i) * a.k_st + 8 * c8) : uint4{0, 0, 0, 0};
    qr[r] = ok ? *reinterpret_cast<const uint4 *>(qb + int64_t(i) * a.q_st + 8 * c8) : uint4{0, 0, 0, 0};
  }
  if (w == 0) {  // gates and the inclusive prefix sum of g
    float gv = 0.f, bv = 0.f;
    if (lane < ci.len) {
      gv = ldf(gb + int64_t(lane) * a.g_st);
      bv = ldf(bb + int64_t(lane) * a.b_st);
    }
    float s = gv;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(s, off, 64);
      if (lane >= off) s += y;
    }
    sm.gam[lane] = s;
    sm.beta[lane] = bv;
    sm.eg[lane] = exp_f(s);
    sm.zk[lane] = bv * exp_f(s);
  }
#pragma unroll
  for (int r = 0; r < PT; ++r) {
    const int p = tid + 256 * r, i = p / (DK / 8), c8 = p % (DK / 8);
    *reinterpret_cast<uint4 *>(&sm.kh[i][8 * c8]) = kr[r];
    *reinterpret_cast<uint4 *>(&sm.qh[i][8 * c8]) = qr[r];
  }
  __syncthreads();

  const float glast = sm.gam[kC - 1];
  // K~^T = (K e^{gamma_C - gamma})^T, split.
  for (int e = tid; e < kC * DK; e += 256) {
    const int i = e / DK, d = e - i * DK;
    const float x = fl(sm.kh[i][d]) * exp_f(glast - sm.gam[i]);
    const __bf16 x1 = bf(x);
    sm.kth[d][i] = x1;
    sm.ktl[d][i] = bf(x - fl(x1));
  }

  // G = K K^T and QK = Q K^T: wave w owns row tile mt = w (rows 16w .. 16w+15).
  {
    const int mt = w;
#pragma unroll
    for (int nt = 0; nt < kC / 16; ++nt) {
      f32x4 gacc = {0.f, 0.f, 0.f, 0.f}, qacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < DK / 32; ++ks) {
        const int k0 = 32 * ks + 8 * g;
        const bf16x8 bk = rd8(sm.kh[16 * nt + ln], k0);
        gacc = mma(rd8(sm.kh[16 * mt + ln], k0), bk, gacc);
        qacc = mma(rd8(sm.qh[16 * mt + ln], k0), bk, qacc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * mt + 4 * g + r, j = 16 * nt + ln;
        float av = 0.f, atv = 0.f;
        if (j <= i) {
          const float dec = exp_f(sm.gam[i] - sm.gam[j]);
          atv = qacc[r] * dec;
          if (j < i) av = -sm.beta[i] * dec * gacc[r];
        }
        sm.A[i][j] = av;
        const __bf16 t1 = bf(atv);
        sm.ath[i][j] = t1;
        sm.atl[i][j] = bf(atv - fl(t1));
      }
    }
  }
  __syncthreads();

  // Forward substitution, one column of [W | U] per thread.
  for (int col = tid; col < DK + a.dv; col += 256) {
    float x[kC];
    if (col < DK) {
#pragma unroll
      for (int i = 0; i < kC; ++i) x[i] = sm.zk[i] * fl(sm.kh[i][col]);
    } else {
      const int e = col - DK;
#pragma unroll
      for (int i = 0; i < kC; ++i) x[i] = (i < ci.len) ? sm.beta[i] * ldf(vb + int64_t(i) * a.v_st + e) : 0.f;
    }
#pragma unroll
    for (int i = 1; i < kC; ++i) {
      // four independent partial sums over j, A row read 4 floats at a time
      float p0 = x[i], p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
      for (int j0 = 0; j0 < i; j0 += 4) {
        const float4 av = *reinterpret_cast<const float4 *>(&sm.A[i][j0]);
        p0 = fmaf(av.x, x[j0], p0);
        if (j0 + 1 < i) p1 = fmaf(av.y, x[j0 + 1], p1);
        if (j0 + 2 < i) p2 = fmaf(av.z, x[j0 + 2], p2);
        if (j0 + 3 < i) p3 = fmaf(av.w, x[j0 + 3], p3);
      }
      x[i] = (p0 + p1) + (p2 + p3);
    }
    __bf16 *rh = col < DK ? sm.wth[col] : sm.uth[col - DK];
    __bf16 *rl = col < DK ? sm.wtl[col] : sm.utl[col - DK];
#pragma unroll
    for (int i0 = 0; i0 < kC; i0 += 8) {
      bf16x8 vh, vl;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        vh[t] = bf(x[i0 + t]);
        vl[t] = bf(x[i0 + t] - fl(vh[t]));
      }
      *reinterpret_cast<bf16x8 *>(rh + i0) = vh;
      *reinterpret_cast<bf16x8 *>(rl + i0) = vl;
    }
  }
  __syncthreads();

  // Output operators.  Tiles: An (DK/16)^2, Hn (DK/16)(DV/16), Qp 4 (DK/16), Op 4 (DV/16).
  const WsLayout L(DK, a.dv);
  char *cell = ws + (static_cast<size_t>(h) * ca.total_chunks + chunk) * L.cell;
  __bf16 *an_h = reinterpret_cast<__bf16 *>(cell + L.an), *an_l = an_h + DK * DK;
  __bf16 *qp_h = reinterpret_cast<__bf16 *>(cell + L.qp), *qp_l = qp_h + kC * DK;
  float *hn = reinterpret_cast<float *>(cell + L.hn);
  float *op = reinterpret_cast<float *>(cell + L.op);
  constexpr int TDK = DK / 16, TC = kC / 16;
  const int tdv = a.dv / 16;
  const int n_an = TDK * TDK, n_hn = TDK * tdv, n_qp = TC * TDK, n_op = TC * tdv;
  const int ntiles = n_an + n_hn + n_qp + n_op;
  const float eC = exp_f(glast);
  for (int t = w; t < ntiles; t += 4) {
    int kind, mt, nt;
    if (t < n_an) { kind = 0; mt = t / TDK; nt = t % TDK; }
    else if (t < n_an + n_hn) { kind = 1; mt = (t - n_an) / tdv; nt = (t - n_an) % tdv; }
    else if (t < n_an + n_hn + n_qp) { kind = 2; mt = (t - n_an - n_hn) / TDK; nt = (t - n_an - n_hn) % TDK; }
    else { kind = 3; mt = (t - n_an - n_hn - n_qp) / tdv; nt = (t - n_an - n_hn - n_qp) % tdv; }
    // A rows: K~^T rows (kinds 0, 1) or Attn rows (kinds 2, 3); B rows: W^T (0, 2) or U^T (1, 3).
    const __bf16 *arh = kind < 2 ? sm.kth[16 * mt + ln] : sm.ath[16 * mt + ln];
    const __bf16 *arl = kind < 2 ? sm.ktl[16 * mt + ln] : sm.atl[16 * mt + ln];
    const __bf16 *brh = (kind & 1) ? sm.uth[16 * nt + ln] : sm.wth[16 * nt + ln];
    const __bf16 *brl = (kind & 1) ? sm.utl[16 * nt + ln] : sm.wtl[16 * nt + ln];
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kC / 32; ++ks) {
      const int k0 = 32 * ks + 8 * g;
      acc = mma3<true, true>(rd8(arh, k0), rd8(arl, k0), rd8(brh, k0), rd8(brl, k0), acc);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * mt + 4 * g + r, col = 16 * nt + ln;
      if (kind == 0) {
        const float x = (row == col ? eC : 0.f) - acc[r];
        const __bf16 x1 = bf(x);
        an_h[row * DK + col] = x1;
        an_l[row * DK + col] = bf(x - fl(x1));
      } else if (kind == 1) {
        hn[row * a.dv + col] = acc[r];
      } else if (kind == 2) {
        const float qv = fl(sm.qh[row][col]) * sm.eg[row];
        const float x = qv - acc[r];
        const __bf16 x1 = bf(x);
        qp_h[row * DK + col] = x1;
        qp_l[row * DK + col] = bf(x - fl(x1));
      } else {
        op[row * a.dv + col] = acc[r];
      }
    }
  }
}

// ------------------------------------------------------------------ scan
template <int DK>
struct ScanSmem {
  __bf16 anh[2][DK][DK + kPad], anl[2][DK][DK + kPad];  // A_n hi / lo
  __bf16 qph[2][kC][DK + kPad], qpl[2][kC][DK + kPad];  // Q' hi / lo
  float hn[2][DK][64 + 4];                              // H_n, this workgroup's 64 columns
  float op[2][kC][64 + 4];                              // O', this workgroup's 64 columns
};

template <typename TO, int DK>
__global__ void __launch_bounds__(256) gdn_scan_mfma(GdnArgs a, ChunkArgs ca, const char *ws) {
  constexpr int TDK = DK / 16;  // state row tiles
  constexpr int KS = DK / 32;   // k-steps over the state rows
  constexpr int N_AN = DK * DK / 8, N_QP = kC * DK / 8;  // 16-byte pieces per bf16 plane
  constexpr int N_HN = DK * 16, N_OP = kC * 16;          // 16-byte pieces of the fp32 tiles
  constexpr int PIECES = 2 * N_AN + 2 * N_QP + N_HN + N_OP;
  constexpr int PER_T = (PIECES + 255) / 256;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  ScanSmem<DK> &sm = *reinterpret_cast<ScanSmem<DK> *>(smem_raw);

  const int tile = blockIdx.x, h = blockIdx.y, sq = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int ln = lane & 15, g = lane >> 4;
  const int c_base = tile * 64;
  const int col = c_base + 16 * w + ln;
  const bool active = c_base + 16 * w < a.dv;  // wave-uniform

  int first, count, batch, t_begin, t_end;
  if (ca.cu == nullptr) {
    batch = sq; first = sq * ca.nper; count = ca.nper; t_begin = 0; t_end = a.L;
  } else {
    batch = 0; first = ca.coff[sq]; count = ca.coff[sq + 1] - first; t_begin = ca.cu[sq]; t_end = ca.cu[sq + 1];
  }
  const WsLayout Lw(DK, a.dv);
  const char *cell0 = ws + (static_cast<size_t>(h) * ca.total_chunks + first) * Lw.cell;

  // Each thread's staging pieces: byte offset inside a workspace cell and inside one
  // LDS buffer (both fixed across chunks); pieces of columns past dv are skipped.
  constexpr size_t BUF = sizeof(ScanSmem<DK>) / 2;  // the buffers interleave per array; offsets below
  uint32_t src_off[PER_T], dst_off[PER_T];
  uint32_t valid = 0;
#pragma unroll
  for (int r = 0; r < PER_T; ++r) {
    int p = tid + 256 * r;
    uint32_t so = 0, dof = 0;
    bool ok = p < PIECES;
    if (p < 2 * N_AN) {
      const int plane = p / N_AN, q = p % N_AN;
      so = Lw.an + p * 16;
      dof = static_cast<uint32_t>(reinterpret_cast<char *>((plane ? sm.anl[0] : sm.anh[0])[q / (DK / 8)] + 8 * (q % (DK / 8))) - smem_raw);
    } else if ((p -= 2 * N_AN) < 2 * N_QP) {
      const int plane = p / N_QP, q = p % N_QP;
      so = Lw.qp + p * 16;
      dof = static_cast<uint32_t>(reinterpret_cast<char *>((plane ? sm.qpl[0] : sm.qph[0])[q / (DK / 8)] + 8 * (q % (DK / 8))) - smem_raw);
    } else if ((p -= 2 * N_QP) < N_HN) {
      const int row = p / 16, c4 = p % 16;
      ok = ok && c_base + 4 * c4 < a.dv;
      so = Lw.hn + (static_cast<uint32_t>(row) * a.dv + c_base + 4 * c4) * 4;
      dof = static_cast<uint32_t>(reinterpret_cast<char *>(&sm.hn[0][row][4 * c4]) - smem_raw);
    } else if ((p -= N_HN) < N_OP) {
      const int row = p / 16, c4 = p % 16;
      ok = ok && c_base + 4 * c4 < a.dv;
      so = Lw.op + (static_cast<uint32_t>(row) * a.dv + c_base + 4 * c4) * 4;
      dof = static_cast<uint32_t>(reinterpret_cast<char *>(&sm.op[0][row][4 * c4]) - smem_raw);
    }
    src_off[r] = so;
    dst_off[r] = dof;
    valid |= ok ? (1u << r) : 0u;
  }
  // Byte distance between buffer 0 and buffer 1 of each array (identical for all arrays
  // only if laid out [2][...]; computed per array class below).
  const uint32_t d_an = static_cast<uint32_t>(reinterpret_cast<char *>(sm.anh[1]) - reinterpret_cast<char *>(sm.anh[0]));
  const uint32_t d_qp = static_cast<uint32_t>(reinterpret_cast<char *>(sm.qph[1]) - reinterpret_cast<char *>(sm.qph[0]));
  const uint32_t d_hn = static_cast<uint32_t>(reinterpret_cast<char *>(sm.hn[1]) - reinterpret_cast<char *>(sm.hn[0]));
  const uint32_t d_op = static_cast<uint32_t>(reinterpret_cast<char *>(sm.op[1]) - reinterpret_cast<char *>(sm.op[0]));
  uint32_t dbuf[PER_T];
#pragma unroll
  for (int r = 0; r < PER_T; ++r) {
    const int p = tid + 256 * r;
    dbuf[r] = p < 2 * N_AN ? d_an : p < 2 * N_AN + 2 * N_QP ? d_qp : p < 2 * N_AN + 2 * N_QP + N_HN ? d_hn : d_op;
  }
  (void)BUF;

  uint4 stg[PER_T];
  auto stage_load = [&](int n) {
    const char *c = cell0 + static_cast<size_t>(n) * Lw.cell;
#pragma unroll
    for (int r = 0; r < PER_T; ++r)
      stg[r] = (valid >> r) & 1 ? *reinterpret_cast<const uint4 *>(c + src_off[r]) : uint4{0, 0, 0, 0};
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int r = 0; r < PER_T; ++r)
      if (tid + 256 * r < PIECES)
        *reinterpret_cast<uint4 *>(smem_raw + dst_off[r] + (buf ? dbuf[r] : 0)) = stg[r];
  };

  // State S[:, col] in accumulator layout: S[mt][r] = S[16 mt + 4 g + r][col].
  f32x4 S[TDK];
  const size_t sbase = (static_cast<size_t>(sq) * a.H + h) * DK * a.dv;
#pragma unroll
  for (int mt = 0; mt < TDK; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      S[mt][r] = (active && a.s_in) ? a.s_in[sbase + static_cast<size_t>(16 * mt + 4 * g + r) * a.dv + col] : 0.f;

  TO *ob = static_cast<TO *>(a.o) + batch * a.o_sb + h * a.o_sh;
  const int lc = 16 * w + ln;  // column inside the workgroup tile

  if (count > 0) {
    stage_load(0);
    stage_store(0);
  }
  __syncthreads();

  for (int n = 0; n < count; ++n) {
    const int buf = n & 1;
    const bool more = n + 1 < count;
    if (more) stage_load(n + 1);
    if (active) {
      // Operands first (LDS reads in flight together), then the MFMA passes
      // interleaved over independent tiles.
      bf16x8 anh[TDK][KS], anl[TDK][KS], qph[kC / 16][KS], qpl[kC / 16][KS];
#pragma unroll
      for (int mt = 0; mt < TDK; ++mt)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          anh[mt][ks] = rd_perm(sm.anh[buf][16 * mt + ln], 32 * ks, g);
          anl[mt][ks] = rd_perm(sm.anl[buf][16 * mt + ln], 32 * ks, g);
        }
      f32x4 sacc[TDK], oacc[kC / 16];
#pragma unroll
      for (int mt = 0; mt < TDK; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sacc[mt][r] = sm.hn[buf][16 * mt + 4 * g + r][lc];
#pragma unroll
      for (int mt = 0; mt < kC / 16; ++mt)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          qph[mt][ks] = rd_perm(sm.qph[buf][16 * mt + ln], 32 * ks, g);
          qpl[mt][ks] = rd_perm(sm.qpl[buf][16 * mt + ln], 32 * ks, g);
        }
#pragma unroll
      for (int mt = 0; mt < kC / 16; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) oacc[mt][r] = sm.op[buf][16 * mt + 4 * g + r][lc];
      // B operands from S: k-step ks covers state rows 32 ks .. 32 ks + 31.
      bf16x8 sh[KS], sl[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float x = S[2 * ks + i / 4][i % 4];
          sh[ks][i] = bf(x);
          sl[ks][i] = bf(x - fl(sh[ks][i]));
        }
      // S_{n+1} = H_n + A_n S_n ; O_n = O' + Q' S_n   (small passes first)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int mt = 0; mt < TDK; ++mt) sacc[mt] = mma(anl[mt][ks], sh[ks], sacc[mt]);
#pragma unroll
        for (int mt = 0; mt < TDK; ++mt) sacc[mt] = mma(anh[mt][ks], sl[ks], sacc[mt]);
#pragma unroll
        for (int mt = 0; mt < TDK; ++mt) sacc[mt] = mma(anh[mt][ks], sh[ks], sacc[mt]);
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int mt = 0; mt < kC / 16; ++mt) oacc[mt] = mma(qpl[mt][ks], sh[ks], oacc[mt]);
#pragma unroll
        for (int mt = 0; mt < kC / 16; ++mt) oacc[mt] = mma(qph[mt][ks], sl[ks], oacc[mt]);
#pragma unroll
        for (int mt = 0; mt < kC / 16; ++mt) oacc[mt] = mma(qph[mt][ks], sh[ks], oacc[mt]);
      }
#pragma unroll
      for (int mt = 0; mt < TDK; ++mt) S[mt] = sacc[mt];
      const int t0 = t_begin + n * kC;
      const int len = min(kC, t_end - t0);
#pragma unroll
      for (int mt = 0; mt < kC / 16; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * mt + 4 * g + r;
          if (i < len) st(ob + int64_t(t0 + i) * a.o_st + col, oacc[mt][r]);
        }
    }
    if (more) stage_store(buf ^ 1);
    __syncthreads();
  }

  if (active) {
#pragma unroll
    for (int mt = 0; mt < TDK; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        a.s_out[sbase + static_cast<size_t>(16 * mt + 4 * g + r) * a.dv + col] = S[mt][r];
  }
}

template <int DK, int DV>
int launch_prep(const GdnArgs &a, const ChunkArgs &ca, char *ws, hipStream_t s) {
  const size_t smem = sizeof(PrepSmem<DK, DV>);
  auto kern = gdn_prep_mfma<DK, DV>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
  if (e != hipSuccess) return set_error(MOTIF_ERR_HIP, std::string("gdn_prep_mfma smem: ") + hipGetErrorString(e));
  kern<<<dim3(ca.total_chunks, a.H), dim3(256), smem, s>>>(a, ca, ws);
  return check_launch("gdn_prep_mfma");
}

template <typename TO, int DK>
int launch_scan(const GdnArgs &a, const ChunkArgs &ca, const char *ws, hipStream_t s) {
  const size_t smem = sizeof(ScanSmem<DK>);
  auto kern = gdn_scan_mfma<TO, DK>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
  if (e != hipSuccess) return set_error(MOTIF_ERR_HIP, std::string("gdn_scan_mfma smem: ") + hipGetErrorString(e));
  kern<<<dim3((a.dv + 63) / 64, a.H, ca.nseq), dim3(256), smem, s>>>(a, ca, ws);
  return check_launch("gdn_scan_mfma");
}

template <int DK>
int launch_dk(const GdnArgs &a, const ChunkArgs &ca, char *ws, hipStream_t s) {
  int rc;
  // the prep's U^T plane is sized for the padded dv bound of its template
  if (a.dv <= 64) rc = launch_prep<DK, 64>(a, ca, ws, s);
  else rc = launch_prep<DK, 128>(a, ca, ws, s);
  if (rc) return rc;
  return launch_scan<bf16_t, DK>(a, ca, ws, s);
}

}  // namespace

bool chunk_mfma_supported(int dk, int dv, int chunk) {
  return chunk == kC && (dk == 32 || dk == 64) && dv % 16 == 0 && dv > 0 && dv <= 128;
}

size_t chunk_mfma_workspace_bytes(int H, int dk, int dv, int total_chunks) {
  return WsLayout(dk, dv).cell * static_cast<size_t>(H) * total_chunks;
}

int launch_chunk_mfma(const GdnArgs &a, const ChunkArgs &ca, void *workspace, int in_dtype, hipStream_t s) {
  if (in_dtype != MOTIF_BF16) return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_chunk MFMA path takes bf16 inputs");
  // 16-byte row loads of q / k
  const int64_t st = a.q_sb | a.q_sh | a.q_st | a.k_sb | a.k_sh | a.k_st;
  if ((st & 7) || ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.k)) & 15))
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_chunk MFMA path needs 16-byte aligned q / k rows");
  char *ws = static_cast<char *>(workspace);
  return a.dk == 32 ? launch_dk<32>(a, ca, ws, s) : launch_dk<64>(a, ca, ws, s);
}

}  // namespace motif
