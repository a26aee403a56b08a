// Gated DeltaNet (GDN) delta-rule kernels for gfx950.
//
// * gdn_recurrent_kernel: token recurrence (decode and short sequences).  One
//   thread owns one value column of the fp32 state S[:, col] in registers, so
//   the k^T S and q^T S reductions are thread-local; the state is read once and
//   written once per launch (HBM-bound at decode batch sizes).
// * gdn_chunk_prep_kernel: chunk-parallel WY preparation.  One workgroup per
//   (chunk, head) builds gamma = cumsum(g), the strictly-lower A, the masked
//   intra-chunk attention (Q K^T) * D, and W = T Zk, U = T Zv by forward
//   substitution (T = (I - A)^-1 never materialised: one thread per column).
// * gdn_chunk_scan_kernel: the serial inter-chunk pass.  One workgroup per
//   (value tile of 32 columns, head, sequence) carries S[:, tile] across the
//   chunks and emits the chunk outputs O = (Q e^gamma) S + Attn X in the same
//   pass (X = U - W S), so neither the prefix states nor X round-trip HBM.
#include <algorithm>

#include "gdn_internal.h"

namespace motif {

// ------------------------------------------------------------------ recurrence
template <typename TI, typename TO, int DK>
__global__ void __launch_bounds__(128) gdn_recurrent_kernel(GdnArgs a) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int col = blockIdx.x * 128 + threadIdx.x;
  const bool active = col < a.dv;
  __shared__ float sq[2][DK], sk[2][DK], sbg[2][2];

  const TI *q = static_cast<const TI *>(a.q) + b * a.q_sb + h * a.q_sh;
  const TI *k = static_cast<const TI *>(a.k) + b * a.k_sb + h * a.k_sh;
  const TI *v = static_cast<const TI *>(a.v) + b * a.v_sb + h * a.v_sh;
  const TI *beta = static_cast<const TI *>(a.beta) + b * a.b_sb + h * a.b_sh;
  const TI *g = static_cast<const TI *>(a.g) + b * a.g_sb + h * a.g_sh;
  TO *o = static_cast<TO *>(a.o) + b * a.o_sb + h * a.o_sh;

  const size_t sbase = (static_cast<size_t>(b) * a.H + h) * DK * a.dv;
  float S[DK];
#pragma unroll
  for (int i = 0; i < DK; ++i)
    S[i] = (active && a.s_in) ? a.s_in[sbase + static_cast<size_t>(i) * a.dv + col] : 0.f;

  for (int t = 0; t < a.L; ++t) {
    const int buf = t & 1;
    for (int i = threadIdx.x; i < 2 * DK; i += blockDim.x) {
      if (i < DK) sq[buf][i] = ld(q + t * a.q_st + i);
      else sk[buf][i - DK] = ld(k + t * a.k_st + (i - DK));
    }
    if (threadIdx.x == 0) {
      sbg[buf][0] = ld(beta + t * a.b_st);
      sbg[buf][1] = ld(g + t * a.g_st);
    }
    __syncthreads();
    if (active) {
      const float decay = exp_f(sbg[buf][1]);
      const float bt = sbg[buf][0];
      const float vt = ld(v + t * a.v_st + col);
      float vold = 0.f;
#pragma unroll
      for (int i = 0; i < DK; ++i) {
        S[i] *= decay;
        vold = fmaf(sk[buf][i], S[i], vold);
      }
      const float delta = bt * (vt - vold);
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < DK; ++i) {
        S[i] = fmaf(sk[buf][i], delta, S[i]);
        acc = fmaf(sq[buf][i], S[i], acc);
      }
      st(o + t * a.o_st + col, acc);
    }
  }
  if (active) {
#pragma unroll
    for (int i = 0; i < DK; ++i) a.s_out[sbase + static_cast<size_t>(i) * a.dv + col] = S[i];
  }
}

// ---------------------------------------------------------------- chunk prep
template <typename TI, int C, int DK>
__global__ void __launch_bounds__(256) gdn_chunk_prep_kernel(GdnArgs a, ChunkArgs ca) {
  const int chunk = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x;
  const ChunkInfo ci = resolve_chunk(chunk, C, a.L, ca);

  __shared__ float sK[C][DK + 1], sQ[C][DK + 1];
  __shared__ __attribute__((aligned(16))) float sA[C][C];
  __shared__ float sGam[C], sBeta[C], sZk[C];

  const TI *qb = static_cast<const TI *>(a.q) + ci.batch * a.q_sb + h * a.q_sh + int64_t(ci.t0) * a.q_st;
  const TI *kb = static_cast<const TI *>(a.k) + ci.batch * a.k_sb + h * a.k_sh + int64_t(ci.t0) * a.k_st;
  const TI *vb = static_cast<const TI *>(a.v) + ci.batch * a.v_sb + h * a.v_sh + int64_t(ci.t0) * a.v_st;
  const TI *bb = static_cast<const TI *>(a.beta) + ci.batch * a.b_sb + h * a.b_sh + int64_t(ci.t0) * a.b_st;
  const TI *gb = static_cast<const TI *>(a.g) + ci.batch * a.g_sb + h * a.g_sh + int64_t(ci.t0) * a.g_st;

  for (int e = tid; e < C * DK; e += 256) {
    const int i = e / DK, d = e - i * DK;
    float kv = 0.f, qv = 0.f;
    if (i < ci.len) {
      kv = ld(kb + i * a.k_st + d);
      qv = ld(qb + i * a.q_st + d);
    }
    sK[i][d] = kv;
    sQ[i][d] = qv;
  }

  const size_t cidx = static_cast<size_t>(h) * ca.total_chunks + chunk;
  if (tid < 64) {  // one wave: gates and the inclusive prefix sum of g
    float gv = 0.f, bv = 0.f;
    if (tid < C && tid < ci.len) {
      gv = ld(gb + tid * a.g_st);
      bv = ld(bb + tid * a.b_st);
    }
    float s = gv;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(s, off, 64);
      if (tid >= off) s += y;
    }
    if (tid < C) {
      sGam[tid] = s;
      sBeta[tid] = bv;
      sZk[tid] = bv * exp_f(s);
      ca.gam[cidx * C + tid] = s;
    }
  }
  __syncthreads();

  float *attn_out = ca.attn + cidx * C * C;
  for (int e = tid; e < C * C; e += 256) {
    const int i = e / C, j = e - i * C;
    float av = 0.f, atv = 0.f;
    if (j <= i) {
      float dkk = 0.f, dqk = 0.f;
#pragma unroll 8
      for (int d = 0; d < DK; ++d) {
        dkk = fmaf(sK[i][d], sK[j][d], dkk);
        dqk = fmaf(sQ[i][d], sK[j][d], dqk);
      }
      const float dec = exp_f(sGam[i] - sGam[j]);
      atv = dqk * dec;
      if (j < i) av = -sBeta[i] * dec * dkk;
    }
    sA[i][j] = av;
    attn_out[e] = atv;
  }
  __syncthreads();

  // Forward substitution: column x of [W | U] solves (I - A) x = z.
  for (int col = tid; col < DK + a.dv; col += 256) {
    float x[C];
    if (col < DK) {
#pragma unroll
      for (int i = 0; i < C; ++i) x[i] = sZk[i] * sK[i][col];
    } else {
      const int e = col - DK;
#pragma unroll
      for (int i = 0; i < C; ++i) x[i] = (i < ci.len) ? sBeta[i] * ld(vb + i * a.v_st + e) : 0.f;
    }
#pragma unroll
    for (int i = 1; i < C; ++i) {
      float acc = x[i];
#pragma unroll
      for (int j = 0; j < i; ++j) acc = fmaf(sA[i][j], x[j], acc);
      x[i] = acc;
    }
    if (col < DK) {
      float *w = ca.W + cidx * C * DK + col;
#pragma unroll
      for (int i = 0; i < C; ++i) w[i * DK] = x[i];
    } else {
      float *u = ca.U + cidx * C * a.dv + (col - DK);
#pragma unroll
      for (int i = 0; i < C; ++i) u[i * a.dv] = x[i];
    }
  }
}

// ---------------------------------------------------------------- chunk scan
template <typename TI, typename TO, int C, int DK>
__global__ void __launch_bounds__(256) gdn_chunk_scan_kernel(GdnArgs a, ChunkArgs ca) {
  constexpr int VT = 32;      // value columns per workgroup
  constexpr int RI = C / 8;   // chunk rows per thread group
  constexpr int RD = DK / 8;  // state rows per thread group
  const int tile = blockIdx.x, h = blockIdx.y, sq = blockIdx.z;
  const int c0 = tile * VT;
  const int tid = threadIdx.x;
  const int cc = tid % VT, grp = tid / VT;

  __shared__ __attribute__((aligned(16))) float sW[C][DK];
  __shared__ __attribute__((aligned(16))) float sQt[C][DK];
  __shared__ __attribute__((aligned(16))) float sKt[C][DK];
  __shared__ __attribute__((aligned(16))) float sAt[C][C];
  __shared__ float sX[C][VT];
  __shared__ float sS[DK][VT];

  int first, count, batch, t_begin, t_end;
  if (ca.cu == nullptr) {
    batch = sq;
    first = sq * ca.nper;
    count = ca.nper;
    t_begin = 0;
    t_end = a.L;
  } else {
    batch = 0;
    first = ca.coff[sq];
    count = ca.coff[sq + 1] - first;
    t_begin = ca.cu[sq];
    t_end = ca.cu[sq + 1];
  }

  const TI *qb = static_cast<const TI *>(a.q) + batch * a.q_sb + h * a.q_sh;
  const TI *kb = static_cast<const TI *>(a.k) + batch * a.k_sb + h * a.k_sh;
  TO *ob = static_cast<TO *>(a.o) + batch * a.o_sb + h * a.o_sh;

  const size_t sbase = (static_cast<size_t>(sq) * a.H + h) * DK * a.dv;
  float Snew[RD];
#pragma unroll
  for (int r = 0; r < RD; ++r) {
    const int d = grp * RD + r;
    Snew[r] = a.s_in ? a.s_in[sbase + static_cast<size_t>(d) * a.dv + c0 + cc] : 0.f;
  }

  for (int n = 0; n < count; ++n) {
    const int chunk = first + n;
    const int t0 = t_begin + n * C;
    const int len = min(C, t_end - t0);
    const size_t cidx = static_cast<size_t>(h) * ca.total_chunks + chunk;
    const float *gam = ca.gam + cidx * C;
    const float glast = gam[C - 1];

#pragma unroll
    for (int r = 0; r < RD; ++r) sS[grp * RD + r][cc] = Snew[r];
    const float *wsrc = ca.W + cidx * C * DK;
#pragma unroll 2
    for (int e = tid; e < C * DK; e += 256) {
      const int i = e / DK, d = e - i * DK;
      const float gi = gam[i];
      float qv = 0.f, kv = 0.f;
      if (i < len) {
        qv = ld(qb + int64_t(t0 + i) * a.q_st + d);
        kv = ld(kb + int64_t(t0 + i) * a.k_st + d);
      }
      sQt[i][d] = qv * exp_f(gi);
      sKt[i][d] = kv * exp_f(glast - gi);
      sW[i][d] = wsrc[e];
    }
    const float *asrc = ca.attn + cidx * C * C;
    for (int e = tid; e < C * C; e += 256) sAt[e / C][e % C] = asrc[e];
    __syncthreads();

    // X = U - W S  (rows grp*RI + r, column cc)
    float xr[RI];
    const float *usrc = ca.U + cidx * C * a.dv + c0 + cc;
#pragma unroll
    for (int r = 0; r < RI; ++r) xr[r] = usrc[(grp * RI + r) * a.dv];
#pragma unroll 2
    for (int d = 0; d < DK; d += 4) {
      const float s0 = sS[d][cc], s1 = sS[d + 1][cc], s2 = sS[d + 2][cc], s3 = sS[d + 3][cc];
#pragma unroll
      for (int r = 0; r < RI; ++r) {
        const float4 w = *reinterpret_cast<const float4 *>(&sW[grp * RI + r][d]);
        xr[r] -= w.x * s0 + w.y * s1 + w.z * s2 + w.w * s3;
      }
    }
#pragma unroll
    for (int r = 0; r < RI; ++r) sX[grp * RI + r][cc] = xr[r];
    __syncthreads();

    // O = (Q e^gamma) S + Attn X
    float orow[RI];
#pragma unroll
    for (int r = 0; r < RI; ++r) orow[r] = 0.f;
#pragma unroll 2
    for (int d = 0; d < DK; d += 4) {
      const float s0 = sS[d][cc], s1 = sS[d + 1][cc], s2 = sS[d + 2][cc], s3 = sS[d + 3][cc];
#pragma unroll
      for (int r = 0; r < RI; ++r) {
        const float4 qv = *reinterpret_cast<const float4 *>(&sQt[grp * RI + r][d]);
        orow[r] += qv.x * s0 + qv.y * s1 + qv.z * s2 + qv.w * s3;
      }
    }
#pragma unroll 2
    for (int j = 0; j < C; j += 4) {
      const float x0 = sX[j][cc], x1 = sX[j + 1][cc], x2 = sX[j + 2][cc], x3 = sX[j + 3][cc];
#pragma unroll
      for (int r = 0; r < RI; ++r) {
        const float4 at = *reinterpret_cast<const float4 *>(&sAt[grp * RI + r][j]);
        orow[r] += at.x * x0 + at.y * x1 + at.z * x2 + at.w * x3;
      }
    }
#pragma unroll
    for (int r = 0; r < RI; ++r) {
      const int i = grp * RI + r;
      if (i < len) st(ob + int64_t(t0 + i) * a.o_st + c0 + cc, orow[r]);
    }

    // S <- e^{gamma_last} S + K~^T X  (rows grp*RD + r)
    const float el = exp_f(glast);
#pragma unroll
    for (int r = 0; r < RD; ++r) Snew[r] = el * sS[grp * RD + r][cc];
#pragma unroll 4
    for (int i = 0; i < C; ++i) {
      const float xv = sX[i][cc];
#pragma unroll
      for (int r = 0; r < RD; r += 4) {
        const float4 kt = *reinterpret_cast<const float4 *>(&sKt[i][grp * RD + r]);
        Snew[r] = fmaf(kt.x, xv, Snew[r]);
        Snew[r + 1] = fmaf(kt.y, xv, Snew[r + 1]);
        Snew[r + 2] = fmaf(kt.z, xv, Snew[r + 2]);
        Snew[r + 3] = fmaf(kt.w, xv, Snew[r + 3]);
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int r = 0; r < RD; ++r) {
    const int d = grp * RD + r;
    a.s_out[sbase + static_cast<size_t>(d) * a.dv + c0 + cc] = Snew[r];
  }
}

// ------------------------------------------------------------------ launchers
static GdnArgs make_args(const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                         const void *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                         const void *v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                         const void *beta, int64_t b_sb, int64_t b_sh, int64_t b_st,
                         const void *g, int64_t g_sb, int64_t g_sh, int64_t g_st,
                         const float *state_in, float *state_out,
                         void *o, int64_t o_sb, int64_t o_sh, int64_t o_st,
                         int B, int H, int L, int dk, int dv) {
  GdnArgs a;
  a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.k = k; a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v = v; a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.beta = beta; a.b_sb = b_sb; a.b_sh = b_sh; a.b_st = b_st;
  a.g = g; a.g_sb = g_sb; a.g_sh = g_sh; a.g_st = g_st;
  a.s_in = state_in; a.s_out = state_out;
  a.o = o; a.o_sb = o_sb; a.o_sh = o_sh; a.o_st = o_st;
  a.B = B; a.H = H; a.L = L; a.dk = dk; a.dv = dv;
  a.gate = nullptr; a.gt_sb = a.gt_st = 0;
  a.nw = nullptr; a.neps = 0.f;
  a.y = nullptr; a.y_sb = a.y_st = 0;
  return a;
}

template <typename TI, typename TO>
static int launch_recurrent(const GdnArgs &a, hipStream_t s) {
  dim3 grid((a.dv + 127) / 128, a.H, a.B), block(128);
  switch (a.dk) {
    case 16: gdn_recurrent_kernel<TI, TO, 16><<<grid, block, 0, s>>>(a); break;
    case 32: gdn_recurrent_kernel<TI, TO, 32><<<grid, block, 0, s>>>(a); break;
    case 64: gdn_recurrent_kernel<TI, TO, 64><<<grid, block, 0, s>>>(a); break;
    case 128: gdn_recurrent_kernel<TI, TO, 128><<<grid, block, 0, s>>>(a); break;
    default: return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_recurrent: dk must be 16, 32, 64 or 128");
  }
  return check_launch("gdn_recurrent_kernel");
}

template <typename TI, int C, int DK>
static int launch_chunk_t(const GdnArgs &a, const ChunkArgs &ca, hipStream_t s) {
  gdn_chunk_prep_kernel<TI, C, DK><<<dim3(ca.total_chunks, a.H), dim3(256), 0, s>>>(a, ca);
  int rc = check_launch("gdn_chunk_prep_kernel");
  if (rc) return rc;
  gdn_chunk_scan_kernel<TI, TI, C, DK><<<dim3(a.dv / 32, a.H, ca.nseq), dim3(256), 0, s>>>(a, ca);
  return check_launch("gdn_chunk_scan_kernel");
}

template <typename TI, int C>
static int launch_chunk_c(const GdnArgs &a, const ChunkArgs &ca, hipStream_t s) {
  switch (a.dk) {
    case 32: return launch_chunk_t<TI, C, 32>(a, ca, s);
    case 64: return launch_chunk_t<TI, C, 64>(a, ca, s);
    case 128: return launch_chunk_t<TI, C, 128>(a, ca, s);
    default: return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_chunk: dk must be 32, 64 or 128");
  }
}

template <typename TI>
static int launch_chunk(const GdnArgs &a, const ChunkArgs &ca, int C, hipStream_t s) {
  switch (C) {
    case 16: return launch_chunk_c<TI, 16>(a, ca, s);
    case 32: return launch_chunk_c<TI, 32>(a, ca, s);
    case 64: return launch_chunk_c<TI, 64>(a, ca, s);
    default: return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_chunk: chunk must be 16, 32 or 64");
  }
}

}  // namespace motif

using namespace motif;

extern "C" int motif_gdn_recurrent_fwd(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    const void *beta, int64_t b_sb, int64_t b_sh, int64_t b_st,
    const void *g, int64_t g_sb, int64_t g_sh, int64_t g_st,
    const float *state_in, float *state_out,
    void *o, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int L, int dk, int dv, int in_dtype, int out_dtype, void *stream) {
  if (B < 0 || H < 0 || L < 0 || dk <= 0 || dv <= 0)
    return set_error(MOTIF_ERR_INVALID, "gdn_recurrent: negative or zero size");
  if (!state_out) return set_error(MOTIF_ERR_INVALID, "gdn_recurrent: state_out is NULL");
  if (B == 0 || H == 0) return MOTIF_OK;
  if (L > 0 && (!q || !k || !v || !beta || !g || !o))
    return set_error(MOTIF_ERR_INVALID, "gdn_recurrent: NULL input pointer");
  GdnArgs a = make_args(q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, v, v_sb, v_sh, v_st,
                        beta, b_sb, b_sh, b_st, g, g_sb, g_sh, g_st, state_in, state_out,
                        o, o_sb, o_sh, o_st, B, H, L, dk, dv);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (in_dtype == MOTIF_F32 && out_dtype == MOTIF_F32) return launch_recurrent<float, float>(a, s);
  if (in_dtype == MOTIF_BF16 && out_dtype == MOTIF_BF16) return launch_recurrent<bf16_t, bf16_t>(a, s);
  if (in_dtype == MOTIF_BF16 && out_dtype == MOTIF_F32) return launch_recurrent<bf16_t, float>(a, s);
  return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_recurrent: unsupported dtype combination");
}

extern "C" size_t motif_gdn_chunk_workspace_bytes(int H, int dk, int dv, int chunk, int total_chunks) {
  if (H <= 0 || dk <= 0 || dv <= 0 || chunk <= 0 || total_chunks <= 0) return 0;
  // bf16 inputs on the MFMA path need its layout; fp32 inputs use the fp32 kernels.
  size_t mfma = chunk_mfma_supported(dk, dv, chunk) ? chunk_mfma_workspace_bytes(H, dk, dv, total_chunks) : 0;
  const size_t per = static_cast<size_t>(chunk) * (1 + dk + dv + chunk);
  return std::max(mfma, per * H * total_chunks * sizeof(float));
}

static int chunk_fwd_impl(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    const void *beta, int64_t b_sb, int64_t b_sh, int64_t b_st,
    const void *g, int64_t g_sb, int64_t g_sh, int64_t g_st,
    const float *state_in, float *state_out,
    void *o, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int L, int dk, int dv, int chunk,
    const int32_t *cu_seqlens, const int32_t *chunk_offsets, int nseq, int total_chunks,
    void *workspace, size_t workspace_bytes,
    int in_dtype, int out_dtype, void *stream,
    const void *gate, int64_t gt_sb, int64_t gt_st, const void *norm_w, float norm_eps,
    void *y, int64_t y_sb, int64_t y_st) {
  const bool gated = gate != nullptr;
  if (B < 0 || H < 0 || L < 0 || dk <= 0 || dv <= 0 || chunk <= 0)
    return set_error(MOTIF_ERR_INVALID, "gdn_chunk: negative or zero size");
  if (dv % 32 != 0 || dv > 256)
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_chunk: dv must be a multiple of 32 and <= 256");
  if (!state_out) return set_error(MOTIF_ERR_INVALID, "gdn_chunk: state_out is NULL");
  if (in_dtype != out_dtype)
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_chunk: output dtype must equal the input dtype");
  const bool packed = cu_seqlens != nullptr;
  if (packed && (B != 1 || !chunk_offsets || nseq <= 0))
    return set_error(MOTIF_ERR_INVALID, "gdn_chunk: packed sequences need B == 1, chunk_offsets and nseq > 0");
  if (!packed && nseq != B)
    return set_error(MOTIF_ERR_INVALID, "gdn_chunk: nseq must equal B for padded batches");
  const int nper = packed ? 0 : (L + chunk - 1) / chunk;
  if (!packed && total_chunks != B * nper)
    return set_error(MOTIF_ERR_INVALID, "gdn_chunk: total_chunks must be B * ceil(L / chunk)");
  if (nseq == 0 || H == 0) return MOTIF_OK;
  if (total_chunks == 0) {
    // No tokens: the final state is the initial one.
    const size_t n = static_cast<size_t>(nseq) * H * dk * dv * sizeof(float);
    if (!state_in) return zero_async(state_out, n, static_cast<hipStream_t>(stream));
    hipError_t e = hipMemcpyAsync(state_out, state_in, n, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? MOTIF_OK : set_error(MOTIF_ERR_HIP, hipGetErrorString(e));
  }
  if (!q || !k || !v || !beta || !g || (!o && !gated))
    return set_error(MOTIF_ERR_INVALID, "gdn_chunk: NULL input pointer");
  const size_t need = motif_gdn_chunk_workspace_bytes(H, dk, dv, chunk, total_chunks);
  if (!workspace || workspace_bytes < need)
    return set_error(MOTIF_ERR_INVALID, "gdn_chunk: workspace too small (need " + std::to_string(need) + " bytes)");

  GdnArgs a = make_args(q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, v, v_sb, v_sh, v_st,
                        beta, b_sb, b_sh, b_st, g, g_sb, g_sh, g_st, state_in, state_out,
                        o, o_sb, o_sh, o_st, B, H, L, dk, dv);
  if (gated) {
    if (!norm_w || !y) return set_error(MOTIF_ERR_INVALID, "gdn_chunk_gated: NULL norm weight or output");
    // the epilogue lives in the bf16 MFMA output kernel; 8-byte gate / weight / output pieces
    const uintptr_t al = reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(norm_w) |
                         reinterpret_cast<uintptr_t>(y);
    if (!chunk_mfma_eligible(a, chunk, in_dtype, out_dtype) || (al & 7) || ((gt_sb | gt_st | y_sb | y_st) & 3))
      return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_chunk_gated: needs the bf16 MFMA path and 8-byte aligned rows");
    a.gate = gate; a.gt_sb = gt_sb; a.gt_st = gt_st;
    a.nw = norm_w; a.neps = norm_eps;
    a.y = y; a.y_sb = y_sb; a.y_st = y_st;
  }
  ChunkArgs ca;
  ca.cu = cu_seqlens;
  ca.coff = chunk_offsets;
  ca.nseq = nseq;
  ca.nper = nper;
  ca.total_chunks = total_chunks;
  float *ws = static_cast<float *>(workspace);
  const size_t tc = static_cast<size_t>(H) * total_chunks;
  ca.gam = ws;
  ca.W = ca.gam + tc * chunk;
  ca.U = ca.W + tc * chunk * dk;
  ca.attn = ca.U + tc * chunk * dv;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (in_dtype != MOTIF_F32 && in_dtype != MOTIF_BF16)
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_chunk: unsupported dtype");
  // bf16 inputs take the MFMA path (3-pass bf16 products, ~16 mantissa bits);
  // fp32 inputs keep fp32 FMA throughout (the 1e-4 accuracy mode).
  if (chunk_mfma_eligible(a, chunk, in_dtype, out_dtype)) return launch_chunk_mfma(a, ca, workspace, s);
  if (in_dtype == MOTIF_F32) return launch_chunk<float>(a, ca, chunk, s);
  if (in_dtype == MOTIF_BF16) return launch_chunk<bf16_t>(a, ca, chunk, s);
  return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_chunk: unsupported dtype");
}

extern "C" int motif_gdn_chunk_fwd(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    const void *beta, int64_t b_sb, int64_t b_sh, int64_t b_st,
    const void *g, int64_t g_sb, int64_t g_sh, int64_t g_st,
    const float *state_in, float *state_out,
    void *o, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int L, int dk, int dv, int chunk,
    const int32_t *cu_seqlens, const int32_t *chunk_offsets, int nseq, int total_chunks,
    void *workspace, size_t workspace_bytes,
    int in_dtype, int out_dtype, void *stream) {
  return chunk_fwd_impl(q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, v, v_sb, v_sh, v_st,
                        beta, b_sb, b_sh, b_st, g, g_sb, g_sh, g_st, state_in, state_out,
                        o, o_sb, o_sh, o_st, B, H, L, dk, dv, chunk, cu_seqlens, chunk_offsets, nseq,
                        total_chunks, workspace, workspace_bytes, in_dtype, out_dtype, stream,
                        nullptr, 0, 0, nullptr, 0.f, nullptr, 0, 0);
}

extern "C" int motif_gdn_chunk_fwd_gated(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    const void *beta, int64_t b_sb, int64_t b_sh, int64_t b_st,
    const void *g, int64_t g_sb, int64_t g_sh, int64_t g_st,
    const float *state_in, float *state_out,
    void *o, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int L, int dk, int dv, int chunk,
    const int32_t *cu_seqlens, const int32_t *chunk_offsets, int nseq, int total_chunks,
    void *workspace, size_t workspace_bytes,
    const void *gate, int64_t gate_sb, int64_t gate_st, const void *norm_weight, float norm_eps,
    void *y, int64_t y_sb, int64_t y_st,
    int dtype, void *stream) {
  if (!gate) return set_error(MOTIF_ERR_INVALID, "gdn_chunk_gated: NULL gate");
  return chunk_fwd_impl(q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, v, v_sb, v_sh, v_st,
                        beta, b_sb, b_sh, b_st, g, g_sb, g_sh, g_st, state_in, state_out,
                        o, o_sb, o_sh, o_st, B, H, L, dk, dv, chunk, cu_seqlens, chunk_offsets, nseq,
                        total_chunks, workspace, workspace_bytes, dtype, dtype, stream,
                        gate, gate_sb, gate_st, norm_weight, norm_eps, y, y_sb, y_st);
}
