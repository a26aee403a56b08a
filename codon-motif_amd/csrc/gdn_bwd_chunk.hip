// GatedDeltaNet chunk backward, the per-chunk parts (gfx950, fp32 on v_mfma_f32_32x32x2_f32).
//
// The reference differentiates its chunked rule in three pieces (motif/ops/gated_deltanet.py):
// the chunk preparation (`_PrepareChunksFunction.backward`, :180-260, the triangular solve
// differentiated from its saved inverse), the inter-chunk scan (`_FusedScanFunction.backward`,
// :727-765) and the per-chunk output combination (autograd through :830-855).  The two
// sequential scans are gdn_bwd.hip's kernels; everything else is independent per chunk and
// runs here, one workgroup per (batch * head, chunk), in two kernels around the scans:
//
//   gdn_bwd_prep_kernel   gamma = cumsum(g), A = -strict(beta k k^T * D), T = (I - A)^{-1}
//                         (blocked substitution), W = T (beta e^gamma k), U = T (beta v), and
//                         the output's upstream terms dP = (q e^gamma)^T do and
//                         dX = ((q k^T) * D)^T do that feed the reverse scan, and (when
//                         asked) the scans' per-chunk operators A = e^{gamma_C} I - Kd^T W,
//                         H = Kd^T U and G = dP - W^T dX (Kd = k e^{gamma_C - gamma});
//   gdn_bwd_chunk_kernel  from the scans' P, X and dSn: dq, dk, dv, dbeta, dg
//                         (the formulas of ops/gdn_grad.py's GDNChunkFunction.backward).
//
// D[i][j] = e^{gamma_i - gamma_j} for j <= i.  All matrices of a chunk live in LDS as fp32
// rows of odd stride (65 or DV + 1 floats), so the four access patterns of the products
// (row or column of either operand, one float per lane) are free of bank conflicts.  A wave
// owns one 32x32 tile of each 64x64 result (rows 32 (w / 2), columns 32 (w % 2)); row sums
// (dbeta, the decay gradient) are carried per lane and reduced at the end, so every
// product's epilogue works on its accumulator registers directly.
// Shapes: chunk 64, dk 64, dv 64 or 128; inputs zero-padded to whole chunks by the host.
#include "capi_internal.h"
#include "common.h"

namespace motif {

namespace {

constexpr int kC = 64;   // chunk length
constexpr int kDK = 64;  // key head dim
constexpr int kLD = 65;  // LDS row stride of a 64-column matrix (floats)

__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// acc += A(m, k) B(k, n) over k < K for this wave's 32x32 tile: lane l supplies row /
// column l % 32 at k = k0 + l / 32.  fa(m, k) / fb(k, n) take the tile-local m / n.
template <int K, typename FA, typename FB>
__device__ __forceinline__ void mm(f32x16 &acc, FA fa, FB fb) {
  const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
#pragma unroll 8
  for (int k0 = 0; k0 < K; k0 += 2) acc = mfma32(fa(i, k0 + h), fb(k0 + h, i), acc);
}

// Two, three or four independent products over the same K in one loop: their MFMA chains
// interleave, so each waits on its operand reads less (one wave per SIMD here).  Each
// accumulator sums in the same order as mm alone.
template <int K, typename FA1, typename FB1, typename FA2, typename FB2>
__device__ __forceinline__ void mm2(f32x16 &c1, FA1 a1, FB1 b1, f32x16 &c2, FA2 a2, FB2 b2) {
  const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
#pragma unroll 8
  for (int k0 = 0; k0 < K; k0 += 2) {
    c1 = mfma32(a1(i, k0 + h), b1(k0 + h, i), c1);
    c2 = mfma32(a2(i, k0 + h), b2(k0 + h, i), c2);
  }
}
template <int K, typename FA1, typename FB1, typename FA2, typename FB2, typename FA3, typename FB3>
__device__ __forceinline__ void mm3(f32x16 &c1, FA1 a1, FB1 b1, f32x16 &c2, FA2 a2, FB2 b2, f32x16 &c3, FA3 a3,
                                    FB3 b3) {
  const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
#pragma unroll 4
  for (int k0 = 0; k0 < K; k0 += 2) {
    c1 = mfma32(a1(i, k0 + h), b1(k0 + h, i), c1);
    c2 = mfma32(a2(i, k0 + h), b2(k0 + h, i), c2);
    c3 = mfma32(a3(i, k0 + h), b3(k0 + h, i), c3);
  }
}
template <int K, typename FA1, typename FB1, typename FA2, typename FB2, typename FA3, typename FB3, typename FA4,
          typename FB4>
__device__ __forceinline__ void mm4(f32x16 &c1, FA1 a1, FB1 b1, f32x16 &c2, FA2 a2, FB2 b2, f32x16 &c3, FA3 a3,
                                    FB3 b3, f32x16 &c4, FA4 a4, FB4 b4) {
  const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
#pragma unroll 4
  for (int k0 = 0; k0 < K; k0 += 2) {
    c1 = mfma32(a1(i, k0 + h), b1(k0 + h, i), c1);
    c2 = mfma32(a2(i, k0 + h), b2(k0 + h, i), c2);
    c3 = mfma32(a3(i, k0 + h), b3(k0 + h, i), c3);
    c4 = mfma32(a4(i, k0 + h), b4(k0 + h, i), c4);
  }
}

// Row of accumulator register r for lane half h, relative to the tile: 8 (r / 4) + 4 h + r % 4.
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

struct BwdPrepArgs {
  const float *q, *k, *v, *beta, *g, *dout;  // [BH * N][C][dk | dv], [BH * N][C]
  float *W, *U, *gam, *T, *dP, *dX;          // [..][C][dk], [..][C][dv], [..][C], [..][C][C], [..][dk][dv], [..][C][dv]
  float *A, *Hn, *G;                         // optional scan operators [..][dk][dk], [..][dk][dv], [..][dk][dv]
};

struct BwdChunkArgs {
  const float *q, *k, *v, *beta, *gam, *T;  // gam and T from the prep kernel
  const float *P, *X, *dSn;                 // the scans' prefix states, residuals, state gradients
  const float *dout, *dX;                   // do, and the prep kernel's dX
  float *dq, *dk, *dv, *dbeta, *dg;
  const float *W, *U;                       // with X NULL: the residuals X = U - W P formed here
};

// rows [C][cols] of a chunk (global, float4 loads) into LDS rows of stride ld, in two
// halves so that the loads of several matrices can all be in flight before the first
// store: fetch_rows issues a matrix's loads, put_rows writes them (one memory round trip
// for every matrix fetched together).
template <int COLS>
struct Rows {
  static constexpr int q4 = COLS / 4, n = kC * q4 / 256;
  static_assert(kC * q4 % 256 == 0, "whole float4 rounds per thread");
  f32x4 x[n];
};
template <int COLS>
__device__ __forceinline__ Rows<COLS> fetch_rows(const float *src, int64_t src_ld, int col0) {
  using R = Rows<COLS>;
  R rw;
#pragma unroll
  for (int j = 0; j < R::n; ++j) {
    const int e = threadIdx.x + 256 * j, r = e / R::q4, c = 4 * (e - r * R::q4);
    rw.x[j] = *reinterpret_cast<const f32x4 *>(src + r * src_ld + col0 + c);
  }
  return rw;
}
template <int COLS>
__device__ __forceinline__ void put_rows(float *dst, int ld, const Rows<COLS> &rw) {
  using R = Rows<COLS>;
#pragma unroll
  for (int j = 0; j < R::n; ++j) {
    const int e = threadIdx.x + 256 * j, r = e / R::q4, c = 4 * (e - r * R::q4);
#pragma unroll
    for (int t = 0; t < 4; ++t) dst[r * ld + c + t] = rw.x[j][t];
  }
}
template <int COLS>
__device__ __forceinline__ void load_rows(float *dst, int ld, const float *src, int64_t src_ld, int col0) {
  put_rows<COLS>(dst, ld, fetch_rows<COLS>(src, src_ld, col0));
}

template <int DV>
__global__ void __launch_bounds__(256) gdn_bwd_prep_kernel(BwdPrepArgs a) {
  constexpr int C = kC, DK = kDK, LD = kLD, LV = DV + 1;
  extern __shared__ float sm[];
  float *sK = sm, *sQ = sK + C * LD, *sA = sQ + C * LD, *sT = sA + C * LD;
  float *sV = sT + C * LD, *sDo = sV + C * LV;
  float *sGam = sDo + C * LV, *sE = sGam + C, *sB = sE + C, *sXs = sB + C;  // sXs: 3 x 16 x 16

  const int64_t cb = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, i = lane & 31, h = lane >> 5;
  const int r0 = 32 * (w >> 1), c0 = 32 * (w & 1);

  {  // the four matrices' loads in flight together
    const Rows<DK> rk = fetch_rows<DK>(a.k + cb * C * DK, DK, 0), rq = fetch_rows<DK>(a.q + cb * C * DK, DK, 0);
    const Rows<DV> rv = fetch_rows<DV>(a.v + cb * C * DV, DV, 0), rd = fetch_rows<DV>(a.dout + cb * C * DV, DV, 0);
    put_rows<DK>(sK, LD, rk);
    put_rows<DK>(sQ, LD, rq);
    put_rows<DV>(sV, LV, rv);
    put_rows<DV>(sDo, LV, rd);
  }
  if (w == 0) {  // gamma = inclusive cumsum of g over the chunk
    float s = a.g[cb * C + lane];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(s, off, 64);
      if (lane >= off) s += y;
    }
    sGam[lane] = s;
    sE[lane] = __expf(s);
    sB[lane] = a.beta[cb * C + lane];
    a.gam[cb * C + lane] = s;
  }
  __syncthreads();

  // A = -strict(beta k k^T * D)
  {
    f32x16 kk = {};
    mm<DK>(kk, [&](int m, int k) { return sK[(r0 + m) * LD + k]; }, [&](int k, int n) { return sK[(c0 + n) * LD + k]; });
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int R = r0 + acc_row(r, h), Nc = c0 + i;
      sA[R * LD + Nc] = Nc < R ? -sB[R] * kk[r] * __expf(sGam[R] - sGam[Nc]) : 0.f;
    }
  }
  __syncthreads();

  // T = (I - A)^{-1}, unit lower triangular: the 16x16 diagonal blocks by substitution,
  // the 32x32 diagonal blocks' off-diagonal pieces T_{2p+1,2p} = T_{2p+1,2p+1} A_{2p+1,2p}
  // T_{2p,2p} (16-wide products per thread), then the lower left 32x32 block
  // T[32:, :32] = T[32:, 32:] (A[32:, :32] T[:32, :32]) as two 32x32x32 MFMA products.
  if (tid < 64) {
    const int b = tid >> 4, c = tid & 15;
    float x[16];
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) {
      float s = ii == c ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < ii; ++j) s = fmaf(sA[(16 * b + ii) * LD + 16 * b + j], x[j], s);
      x[ii] = s;
    }
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) sT[(16 * b + ii) * LD + 16 * b + c] = x[ii];
  }
  for (int e = tid; e < C * C; e += 256) {
    const int r = e >> 6, c = e & 63;
    if ((c >> 4) > (r >> 4)) sT[r * LD + c] = 0.f;
  }
  __syncthreads();
  for (int e = tid; e < 2 * 256; e += 256) {  // blocks (1, 0) and (3, 2)
    const int bj = 2 * (e >> 8), rr = (e >> 4) & 15, cc = e & 15, bi = bj + 1;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) s = fmaf(sA[(16 * bi + rr) * LD + 16 * bj + k], sT[(16 * bj + k) * LD + 16 * bj + cc], s);
    sXs[e] = s;
  }
  __syncthreads();
  for (int e = tid; e < 2 * 256; e += 256) {
    const int bj = 2 * (e >> 8), rr = (e >> 4) & 15, cc = e & 15, bi = bj + 1;
    float s = 0.f;
    for (int k = 0; k <= rr; ++k) s = fmaf(sT[(16 * bi + rr) * LD + 16 * bi + k], sXs[((e >> 8) << 8) + (k << 4) + cc], s);
    sT[(16 * bi + rr) * LD + 16 * bj + cc] = s;
  }
  __syncthreads();
  if (w == 0) {  // one wave: X = A[32:, :32] T[:32, :32] into A's (zero) upper right block
    f32x16 x = {};
    mm<32>(x, [&](int m, int k) { return sA[(32 + m) * LD + k]; }, [&](int k, int n) { return sT[k * LD + n]; });
#pragma unroll
    for (int r = 0; r < 16; ++r) sA[acc_row(r, h) * LD + 32 + i] = x[r];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // (lgkmcnt 0: the X rows are written before any read)
    __builtin_amdgcn_wave_barrier();
    f32x16 t = {};
    mm<32>(t, [&](int m, int k) { return sT[(32 + m) * LD + 32 + k]; }, [&](int k, int n) { return sA[k * LD + 32 + n]; });
#pragma unroll
    for (int r = 0; r < 16; ++r) sT[(32 + acc_row(r, h)) * LD + i] = t[r];
  }
  __syncthreads();

  // Attn = (q k^T) * D (lower, diagonal included) over the dead A
  {
    f32x16 qk = {};
    mm<DK>(qk, [&](int m, int k) { return sQ[(r0 + m) * LD + k]; }, [&](int k, int n) { return sK[(c0 + n) * LD + k]; });
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int R = r0 + acc_row(r, h), Nc = c0 + i;
      sA[R * LD + Nc] = Nc <= R ? qk[r] * __expf(sGam[R] - sGam[Nc]) : 0.f;
    }
  }
  // W = T (beta e^gamma k)
  f32x16 wreg = {};
  // U = T (beta v), dP = (q e^gamma)^T do: column tiles c0 + 64 j of the dv columns
  f32x16 ureg[DV / 64], dpreg[DV / 64];
#pragma unroll
  for (int j = 0; j < DV / 64; ++j) {
    const int n0 = c0 + 64 * j;
    ureg[j] = f32x16{};
    dpreg[j] = f32x16{};
    auto ta = [&](int m, int k) { return sT[(r0 + m) * LD + k]; };
    auto vb = [&](int k, int n) { return sB[k] * sV[k * LV + n0 + n]; };
    auto qa = [&](int m, int k) { return sQ[k * LD + r0 + m] * sE[k]; };
    auto db = [&](int k, int n) { return sDo[k * LV + n0 + n]; };
    if (j == 0) {  // W with the first column tile's products
      mm3<C>(wreg, ta, [&](int k, int n) { return sB[k] * sE[k] * sK[k * LD + c0 + n]; }, ureg[j], ta, vb, dpreg[j], qa, db);
#pragma unroll
      for (int r = 0; r < 16; ++r) a.W[(cb * C + r0 + acc_row(r, h)) * DK + c0 + i] = wreg[r];
    } else {
      mm2<C>(ureg[j], ta, vb, dpreg[j], qa, db);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int R = r0 + acc_row(r, h);
      a.U[(cb * C + R) * DV + n0 + i] = ureg[j][r];
      if (a.dP) a.dP[(cb * DK + R) * DV + n0 + i] = dpreg[j][r];
    }
  }
  for (int e = tid; e < C * C; e += 256) a.T[cb * C * C + e] = sT[(e >> 6) * LD + (e & 63)];
  __syncthreads();  // Attn complete; the reads of T, V and Q above are done
  // With the scan operators requested: W over the T rows, U over the V rows and the
  // decayed keys Kd = k e^{gamma_C - gamma} over the Q rows (all dead here).
  const bool ops = a.A != nullptr;
  if (ops) {
#pragma unroll
    for (int r = 0; r < 16; ++r) sT[(r0 + acc_row(r, h)) * LD + c0 + i] = wreg[r];
#pragma unroll
    for (int j = 0; j < DV / 64; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) sV[(r0 + acc_row(r, h)) * LV + c0 + 64 * j + i] = ureg[j][r];
    for (int e = tid; e < C * DK; e += 256) {
      const int rr = e / DK, cc = e % DK;
      sQ[rr * LD + cc] = sK[rr * LD + cc] * __expf(sGam[C - 1] - sGam[rr]);
    }
  }
  // dX = Attn^T do (both column tiles in one k loop when dv = 128)
  f32x16 dxreg[DV / 64];
  {
    auto at = [&](int m, int k) { return sA[k * LD + r0 + m]; };
    dxreg[0] = f32x16{};
    if constexpr (DV == 128) {
      dxreg[1] = f32x16{};
      mm2<C>(dxreg[0], at, [&](int k, int n) { return sDo[k * LV + c0 + n]; },
             dxreg[1], at, [&](int k, int n) { return sDo[k * LV + c0 + 64 + n]; });
    } else {
      mm<C>(dxreg[0], at, [&](int k, int n) { return sDo[k * LV + c0 + n]; });
    }
  }
#pragma unroll
  for (int j = 0; j < DV / 64; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) a.dX[(cb * C + r0 + acc_row(r, h)) * DV + c0 + 64 * j + i] = dxreg[j][r];
  if (!ops) return;
  // The per-chunk operators of the operator-form scans (gdn_bwd.hip):
  //   A = e^{gamma_C} I - Kd^T W,  H = Kd^T U,  G = dP - W^T dX,  Kd = k e^{gamma_C - gamma}
  __syncthreads();  // the reads of do are done; W, U and Kd are visible
#pragma unroll
  for (int j = 0; j < DV / 64; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) sDo[(r0 + acc_row(r, h)) * LV + c0 + 64 * j + i] = dxreg[j][r];
  __syncthreads();  // dX over the do rows
  auto kdT = [&](int m, int k) { return sQ[k * LD + r0 + m]; };  // Kd^T
  auto wT = [&](int m, int k) { return sT[k * LD + r0 + m]; };   // W^T
#pragma unroll
  for (int j = 0; j < DV / 64; ++j) {
    const int n0 = c0 + 64 * j;
    f32x16 hacc = {}, gacc = {};
    auto ub = [&](int k, int n) { return sV[k * LV + n0 + n]; };
    auto xb = [&](int k, int n) { return sDo[k * LV + n0 + n]; };
    if (j == 0) {  // A with the first column tile's products
      f32x16 acc = {};
      mm3<C>(acc, kdT, [&](int k, int n) { return sT[k * LD + c0 + n]; }, hacc, kdT, ub, gacc, wT, xb);
      const float ec = sE[C - 1];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int R = r0 + acc_row(r, h), Nc = c0 + i;
        a.A[(cb * DK + R) * DK + Nc] = (R == Nc ? ec : 0.f) - acc[r];
      }
    } else {
      mm2<C>(hacc, kdT, ub, gacc, wT, xb);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int R = r0 + acc_row(r, h);
      a.Hn[(cb * DK + R) * DV + n0 + i] = hacc[r];
      a.G[(cb * DK + R) * DV + n0 + i] = dpreg[j][r] - gacc[r];
    }
  }
}


template <int DV>
__global__ void __launch_bounds__(256) gdn_bwd_chunk_kernel(BwdChunkArgs a) {
  constexpr int C = kC, DK = kDK, LD = kLD;
  extern __shared__ float sm[];
  float *sK = sm, *sT = sK + C * LD;
  float *b0 = sT + C * LD, *b1 = b0 + C * LD, *b2 = b1 + C * LD, *b3 = b2 + C * LD, *b4 = b3 + C * LD,
        *b5 = b4 + C * LD;
  float *sGam = b5 + C * LD, *sE = sGam + C, *sDec = sE + C, *sB = sDec + C;
  float *sRowG = sB + C, *sRowB = sRowG + 2 * C, *sCol = sRowB + 2 * C, *sRed = sCol + 2 * C;

  const int64_t cb = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, i = lane & 31, h = lane >> 5;
  const int tr = w >> 1, tc = w & 1, r0 = 32 * tr, c0 = 32 * tc;

  {
    const Rows<DK> rk = fetch_rows<DK>(a.k + cb * C * DK, DK, 0);
    const Rows<C> rt = fetch_rows<C>(a.T + cb * C * C, C, 0);
    put_rows<DK>(sK, LD, rk);
    put_rows<C>(sT, LD, rt);
  }
  if (tid < 64) {
    const float gm = a.gam[cb * C + tid];
    sGam[tid] = gm;
    sE[tid] = __expf(gm);
    sDec[tid] = __expf(a.gam[cb * C + C - 1] - gm);
    sB[tid] = a.beta[cb * C + tid];
  }

  // ---- phase A, per 64 value columns j: b0 = do, b1 = X, b2 = P, b3 = dSn, b4 = v, b5 = dxt
  f32x16 T1 = {}, T2 = {}, T3 = {}, T4 = {}, T5 = {};  // do X^T, do P^T, X dSn^T, dxt P^T, dxt v^T
  float rowB[16], corr = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) rowB[r] = 0.f;
  for (int j = 0; j < DV / 64; ++j) {
    const int e0 = 64 * j;
    {  // the five matrices' loads in flight together
      const Rows<64> r0_ = fetch_rows<64>(a.dout + cb * C * DV, DV, e0);
      const Rows<64> r1_ = fetch_rows<64>((a.X ? a.X : a.U) + cb * C * DV, DV, e0);
      const Rows<64> r2_ = fetch_rows<64>(a.P + cb * DK * DV, DV, e0);
      const Rows<64> r3_ = fetch_rows<64>(a.dSn + cb * DK * DV, DV, e0);
      const Rows<64> r4_ = fetch_rows<64>(a.v + cb * C * DV, DV, e0);
      put_rows<64>(b0, LD, r0_);
      put_rows<64>(b1, LD, r1_);
      put_rows<64>(b2, LD, r2_);
      put_rows<64>(b3, LD, r3_);
      put_rows<64>(b4, LD, r4_);
    }
    if (!a.X) {  // X = U - W P for these columns: W over b5 (free until dxt), U in b1
      load_rows<DK>(b5, LD, a.W + cb * C * DK, DK, 0);
      __syncthreads();
      f32x16 wp = {};
      mm<DK>(wp, [&](int m, int k) { return b5[(r0 + m) * LD + k]; }, [&](int k, int n) { return b2[k * LD + c0 + n]; });
#pragma unroll
      for (int r = 0; r < 16; ++r) {  // each wave rewrites only its own tile of b1
        const int R = r0 + acc_row(r, h), Nc = c0 + i;
        b1[R * LD + Nc] -= wp[r];
      }
    }
    float dxo[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) dxo[r] = a.dX[(cb * C + r0 + acc_row(r, h)) * DV + e0 + c0 + i];
    __syncthreads();
    f32x16 kds = {};  // k dSn
    static_assert(DK == 64, "the four products below share one k loop");
    mm4<64>(T1, [&](int m, int k) { return b0[(r0 + m) * LD + k]; }, [&](int k, int n) { return b1[(c0 + n) * LD + k]; },
            T2, [&](int m, int k) { return b0[(r0 + m) * LD + k]; }, [&](int k, int n) { return b2[(c0 + n) * LD + k]; },
            T3, [&](int m, int k) { return b1[(r0 + m) * LD + k]; }, [&](int k, int n) { return b3[(c0 + n) * LD + k]; },
            kds, [&](int m, int k) { return sK[(r0 + m) * LD + k]; }, [&](int k, int n) { return b3[k * LD + c0 + n]; });
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int R = r0 + acc_row(r, h), Nc = c0 + i;
      b5[R * LD + Nc] = dxo[r] + kds[r] * sDec[R];  // total dX: upstream + through the state
      corr = fmaf(b3[R * LD + Nc], b2[R * LD + Nc], corr);
    }
    __syncthreads();
    f32x16 dvb = {};  // T^T dxt
    mm3<64>(T4, [&](int m, int k) { return b5[(r0 + m) * LD + k]; }, [&](int k, int n) { return b2[(c0 + n) * LD + k]; },
            T5, [&](int m, int k) { return b5[(r0 + m) * LD + k]; }, [&](int k, int n) { return b4[(c0 + n) * LD + k]; },
            dvb, [&](int m, int k) { return sT[k * LD + r0 + m]; }, [&](int k, int n) { return b5[k * LD + c0 + n]; });
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int R = r0 + acc_row(r, h), Nc = c0 + i;
      a.dv[(cb * C + R) * DV + e0 + Nc] = dvb[r] * sB[R];
      rowB[r] = fmaf(dvb[r], b4[R * LD + Nc], rowB[r]);
    }
    __syncthreads();
  }

  // ---- phase B: b0 = q, b1 = dAttn = (do X^T) * D, b2 = dW = -dxt P^T, b3 = dT, b4 = Y, b5 = dG1
  load_rows<DK>(b0, LD, a.q + cb * C * DK, DK, 0);
  const float bcol = sB[c0 + i], ecol = sE[c0 + i];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int R = r0 + acc_row(r, h), Nc = c0 + i;
    T1[r] = Nc <= R ? T1[r] * __expf(sGam[R] - sGam[Nc]) : 0.f;
    b1[R * LD + Nc] = T1[r];
    b2[R * LD + Nc] = -T4[r];
    T5[r] *= bcol;  // dxt (beta v)^T
  }
  __syncthreads();
  f32x16 qk = {}, kk = {};
  mm2<DK>(qk, [&](int m, int k) { return b0[(r0 + m) * LD + k]; }, [&](int k, int n) { return sK[(c0 + n) * LD + k]; },
          kk, [&](int m, int k) { return sK[(r0 + m) * LD + k]; }, [&](int k, int n) { return sK[(c0 + n) * LD + k]; });
  f32x16 ddec, G1;  // d/dD (times D) and beta k k^T
  float rowG[16], kdk = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    ddec[r] = T1[r] * qk[r];
    G1[r] = sB[r0 + acc_row(r, h)] * kk[r];
  }
  // dq = dqg e^gamma + dAttn k;  dk = dAttn^T q + dKd e^{gamma_C - gamma};
  // dT = dW Z^T + dxt (beta v)^T,  Z = beta e^gamma k  (three independent products)
  f32x16 dq = {}, dk = {}, tdt = {};
  mm3<C>(dq, [&](int m, int k) { return b1[(r0 + m) * LD + k]; }, [&](int k, int n) { return sK[k * LD + c0 + n]; },
         dk, [&](int m, int k) { return b1[k * LD + r0 + m]; }, [&](int k, int n) { return b0[k * LD + c0 + n]; },
         tdt, [&](int m, int k) { return b2[(r0 + m) * LD + k]; }, [&](int k, int n) { return sK[(c0 + n) * LD + k]; });
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int R = r0 + acc_row(r, h), Nc = c0 + i;
    a.dq[(cb * C + R) * DK + Nc] = fmaf(T2[r], sE[R], dq[r]);
    rowG[r] = T2[r] * b0[R * LD + Nc] * sE[R];
    const float t = T3[r] * sDec[R];
    dk[r] += t;
    const float kd = t * sK[R * LD + Nc];
    rowG[r] -= kd;
    kdk += kd;
    b3[R * LD + Nc] = fmaf(tdt[r], bcol * ecol, T5[r]);
  }
  __syncthreads();
  f32x16 dkb = {};
  {  // dZ = T^T dW: dkb = dZ e^gamma, d gamma += dZ . Z;  Y = dT T^T
    f32x16 dZ = {}, y = {};
    mm2<C>(dZ, [&](int m, int k) { return sT[k * LD + r0 + m]; }, [&](int k, int n) { return b2[k * LD + c0 + n]; },
           y, [&](int m, int k) { return b3[(r0 + m) * LD + k]; }, [&](int k, int n) { return sT[(c0 + n) * LD + k]; });
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int R = r0 + acc_row(r, h), Nc = c0 + i;
      dkb[r] = dZ[r] * sE[R];
      rowG[r] = fmaf(dkb[r] * sB[R], sK[R * LD + Nc], rowG[r]);
      b4[R * LD + Nc] = y[r];
    }
  }
  __syncthreads();
  float colG = 0.f;
  {  // dA = strict(T^T Y), dG1 = -dA * D, ddec -= dA * G1 * D
    f32x16 dA = {};
    mm<C>(dA, [&](int m, int k) { return sT[k * LD + r0 + m]; }, [&](int k, int n) { return b4[k * LD + c0 + n]; });
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int R = r0 + acc_row(r, h), Nc = c0 + i;
      const float D = Nc < R ? __expf(sGam[R] - sGam[Nc]) : 0.f;
      const float da = Nc < R ? dA[r] : 0.f;
      b5[R * LD + Nc] = -da * D;
      ddec[r] -= da * G1[r] * D;
      rowG[r] += ddec[r];
      colG += ddec[r];
    }
  }
  __syncthreads();
  // dkb += dG1 k;  dk += dG1^T (beta k) + dkb beta;  dbeta += dkb . k
  mm2<C>(dkb, [&](int m, int k) { return b5[(r0 + m) * LD + k]; }, [&](int k, int n) { return sK[k * LD + c0 + n]; },
         dk, [&](int m, int k) { return b5[k * LD + r0 + m] * sB[k]; }, [&](int k, int n) { return sK[k * LD + c0 + n]; });
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int R = r0 + acc_row(r, h), Nc = c0 + i;
    rowB[r] = fmaf(dkb[r], sK[R * LD + Nc], rowB[r]);
    a.dk[(cb * C + R) * DK + Nc] = fmaf(dkb[r], sB[R], dk[r]);
  }

  // ---- reductions: row sums over the 32 lanes of a half and the two column waves, column
  // sums of ddec over the two lane halves and the two row waves, block sums of kdk and corr
#pragma unroll
  for (int r = 0; r < 16; ++r) {
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) {
      rowG[r] += __shfl_xor(rowG[r], off, 64);
      rowB[r] += __shfl_xor(rowB[r], off, 64);
    }
  }
  if (i == 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sRowG[tc * C + r0 + acc_row(r, h)] = rowG[r];
      sRowB[tc * C + r0 + acc_row(r, h)] = rowB[r];
    }
  }
  colG += __shfl_xor(colG, 32, 64);
  if (h == 0) sCol[tr * C + c0 + i] = colG;
  kdk = wave_sum(kdk);
  corr = wave_sum(corr);
  if (lane == 0) {
    sRed[w] = kdk;
    sRed[4 + w] = corr;
  }
  __syncthreads();
  if (w == 0) {
    const int c = lane;
    float dgam = sRowG[c] + sRowG[C + c] - sCol[c] - sCol[C + c];
    if (c == C - 1)
      dgam += (sRed[0] + sRed[1] + sRed[2] + sRed[3]) + sE[C - 1] * (sRed[4] + sRed[5] + sRed[6] + sRed[7]);
    // dg = reverse cumulative sum of d gamma (gamma = cumsum g)
    float s = dgam;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_down(s, off, 64);
      if (c + off < 64) s += y;
    }
    a.dg[cb * C + c] = s;
    a.dbeta[cb * C + c] = sRowB[c] + sRowB[C + c];
  }
}

constexpr size_t prep_smem(int dv) { return sizeof(float) * (4 * kC * kLD + 2 * kC * (dv + 1) + 3 * kC + 3 * 256); }
constexpr size_t chunk_smem() { return sizeof(float) * (8 * kC * kLD + 4 * kC + 6 * kC + 8); }

// kernels above 64 KB of dynamic LDS need the limit raised first
template <typename K>
int set_smem(K kern, size_t smem, const char *what) {
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(smem));
  if (e != hipSuccess) return set_error(MOTIF_ERR_HIP, std::string(what) + " smem: " + hipGetErrorString(e));
  return MOTIF_OK;
}

int check_bwd_sizes(int BH, int N, int C, int Dk, int Dv, const char *who) {
  if (BH < 0 || N < 0 || C <= 0 || Dk <= 0 || Dv <= 0) return set_error(MOTIF_ERR_INVALID, std::string(who) + ": bad sizes");
  if (C != kC || Dk != kDK || (Dv != 64 && Dv != 128))
    return set_error(MOTIF_ERR_UNSUPPORTED, std::string(who) + ": needs C == 64, Dk == 64 and Dv in {64, 128}");
  if (static_cast<int64_t>(BH) * N >= (int64_t(1) << 31))
    return set_error(MOTIF_ERR_UNSUPPORTED, std::string(who) + ": too many chunks");
  return MOTIF_OK;
}

bool aligned16(std::initializer_list<const void *> ps) {
  uintptr_t u = 0;
  for (const void *p : ps) u |= reinterpret_cast<uintptr_t>(p);
  return (u & 15) == 0;
}

}  // namespace

}  // namespace motif

extern "C" int motif_gdn_bwd_prep_f32(const float *q, const float *k, const float *v, const float *beta,
                                      const float *g, const float *dout, float *W, float *U, float *gam, float *T,
                                      float *dP, float *dX, float *A, float *Hn, float *G, int BH, int N, int C,
                                      int Dk, int Dv, void *stream) {
  using namespace motif;
  if (int rc = check_bwd_sizes(BH, N, C, Dk, Dv, "gdn_bwd_prep_f32")) return rc;
  const int64_t blocks = static_cast<int64_t>(BH) * N;
  if (blocks == 0) return MOTIF_OK;
  if (!q || !k || !v || !beta || !g || !dout || !W || !U || !gam || !T || !dX || (!dP && !A) ||
      (A && (!Hn || !G)))
    return set_error(MOTIF_ERR_INVALID, "gdn_bwd_prep_f32: NULL pointer");
  if (!aligned16({q, k, v, dout}))
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_bwd_prep_f32: q, k, v and dout need 16-byte alignment");
  BwdPrepArgs a{q, k, v, beta, g, dout, W, U, gam, T, dP, dX, A, Hn, G};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t smem = prep_smem(Dv);
  if (Dv == 64) {
    if (int rc = set_smem(gdn_bwd_prep_kernel<64>, smem, "gdn_bwd_prep_kernel")) return rc;
    gdn_bwd_prep_kernel<64><<<dim3(static_cast<unsigned>(blocks)), dim3(256), smem, s>>>(a);
  } else {
    if (int rc = set_smem(gdn_bwd_prep_kernel<128>, smem, "gdn_bwd_prep_kernel")) return rc;
    gdn_bwd_prep_kernel<128><<<dim3(static_cast<unsigned>(blocks)), dim3(256), smem, s>>>(a);
  }
  return check_launch("gdn_bwd_prep_kernel");
}

extern "C" int motif_gdn_bwd_chunk_f32(const float *q, const float *k, const float *v, const float *beta,
                                       const float *gam, const float *T, const float *P, const float *X,
                                       const float *dSn, const float *dout, const float *dX, float *dq, float *dk,
                                       float *dv, float *dbeta, float *dg, const float *W, const float *U, int BH,
                                       int N, int C, int Dk, int Dv, void *stream) {
  using namespace motif;
  if (int rc = check_bwd_sizes(BH, N, C, Dk, Dv, "gdn_bwd_chunk_f32")) return rc;
  const int64_t blocks = static_cast<int64_t>(BH) * N;
  if (blocks == 0) return MOTIF_OK;
  if (!q || !k || !v || !beta || !gam || !T || !P || !dSn || !dout || !dX || !dq || !dk || !dv || !dbeta || !dg ||
      (!X && (!W || !U)))
    return set_error(MOTIF_ERR_INVALID, "gdn_bwd_chunk_f32: NULL pointer");
  if (!aligned16({q, k, v, T, P, X, dSn, dout, W, U}))
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_bwd_chunk_f32: the row operands need 16-byte alignment");
  BwdChunkArgs a{q, k, v, beta, gam, T, P, X, dSn, dout, dX, dq, dk, dv, dbeta, dg, X ? nullptr : W, X ? nullptr : U};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t smem = chunk_smem();
  if (Dv == 64) {
    if (int rc = set_smem(gdn_bwd_chunk_kernel<64>, smem, "gdn_bwd_chunk_kernel")) return rc;
    gdn_bwd_chunk_kernel<64><<<dim3(static_cast<unsigned>(blocks)), dim3(256), smem, s>>>(a);
  } else {
    if (int rc = set_smem(gdn_bwd_chunk_kernel<128>, smem, "gdn_bwd_chunk_kernel")) return rc;
    gdn_bwd_chunk_kernel<128><<<dim3(static_cast<unsigned>(blocks)), dim3(256), smem, s>>>(a);
  }
  return check_launch("gdn_bwd_chunk_kernel");
}
