// GatedDeltaNet chunk scans in fp32 for the backward pass (gfx950), on 16x16x4 fp32 MFMAs.
//
// Forward re-scan (the reference's _gdn_fused_scan_kernel, motif/ops/gated_deltanet.py:327-408):
//   per chunk n of C tokens, with gamma the within-chunk cumulative log decay,
//     P_n = S;  X_n = U_n - W_n S;  S <- e^{gamma_C} S + Kd_n^T X_n,
//     Kd_n[c] = k_n[c] e^{gamma_C - gamma_c}.
// Reverse scan (the reference's _gdn_bwd_scan_kernel, :428-520), from gS = dS_final:
//   for n = N-1 .. 0:  dSn_n = gS;  dx = Kd_n gS + dX_n;  gS <- e^{gamma_C} gS - W_n^T dx + dP_n,
//   dS0 = gS.
// The columns of the state are independent, so a workgroup owns 16 of them for one
// (batch, head) and walks the chunks; 4 waves split the 16-row tiles of X (C rows) and of
// the state (Dk rows).  W and the decayed keys of a chunk sit in LDS (rows padded so the
// operand reads of both the matrix and its transpose are free of bank conflicts), the
// next chunk's rows are prefetched in registers.  fp32 throughout: the reference runs
// this path in fp32 (tf32x3 products).
#include "capi_internal.h"
#include "common.h"

namespace motif {

namespace {

constexpr int kCols = 16;  // state columns per workgroup
constexpr int kPadRow = 4;   // stride Dk + 4: rows of a 16-row A tile in distinct banks
constexpr int kPadCol = 16;  // stride Dk + 16: the 4 k-rows of a transposed A tile apart

__device__ __forceinline__ f32x4 mma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

struct ScanArgs {
  const float *k, *w, *u, *g;    // [BH][N][C][Dk], [BH][N][C][Dk], [BH][N][C][Dv], [BH][N][C]
  const float *s0;               // [BH][Dk][Dv] (forward) or dS_final (reverse)
  const float *dx, *dp;          // reverse: [BH][N][C][Dv], [BH][N][Dk][Dv] or null
  float *p, *x, *s_out;          // forward: P, X, S_out;  reverse: dSn, -, dS0
  int N, C, Dk, Dv;
};

// What a chunk reads from global memory, loaded one chunk ahead: the rows [C][Dk] of W
// and k (256 threads, a float4 of each per 256 elements: C * Dk <= 8192) with the
// cumulative log decay of each row, the chunk's last decay, and per wave its tile of U
// (forward) or dX (reverse) and, reverse only, its tiles of dP.
template <int NP>
struct Pre {
  f32x4 w[NP], k[NP];
  float grow[NP];
  float gl;
  f32x4 xin, pin[2];
};

// ------------------------------------------------------------------ the scans
// REV = false: forward re-scan (A operands: W rows, Kd^T); REV = true: reverse scan
// (Kd rows, W^T).  The matrix read row-wise has row stride Dk + 4, the transposed one
// Dk + 16.
// Order of global traffic per chunk: once chunk i's products are done, all loads for
// chunk i + 1 are issued together and then written to LDS (one memory round trip per
// chunk); chunk i's stores (P or dSn, X) follow, so a wait for a load never waits on
// stores of the same chunk (the memory counter is in order across loads and stores).
template <bool REV, int C, int DK>
__global__ void __launch_bounds__(256) gdn_scan_f32_kernel(ScanArgs a) {
  const int v0 = blockIdx.x * kCols;
  const int64_t bh = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int lr = lane & 15, lq = lane >> 4;  // A row / B column, k quad
  const int sw_st = DK + (REV ? kPadCol : kPadRow), kd_st = DK + (REV ? kPadRow : kPadCol);
  __shared__ __attribute__((aligned(16))) float sW[C * (DK + kPadCol)];
  __shared__ __attribute__((aligned(16))) float sKd[C * (DK + kPadCol)];
  __shared__ float sS[DK * kCols];
  __shared__ float sX[C * kCols];
  __shared__ float sXin[C * kCols];   // the chunk's U (forward) or dX (reverse) columns
  __shared__ float sPin[DK * kCols];  // reverse: the chunk's dP columns
  __shared__ float sGl;                   // the chunk's last cumulative log decay
  constexpr int xt = C / 16, st = DK / 16;  // row tiles of X and of the state (st <= 8)
  constexpr int nv = C * DK / 4, q4 = DK / 4;
  constexpr int NP = (nv + 255) / 256;  // float4 rows of W (and of k) per thread

  auto load = [&](int n, Pre<NP> &p) {
    const int64_t cb = bh * a.N + n;
    const f32x4 *wp = reinterpret_cast<const f32x4 *>(a.w + cb * C * DK);
    const f32x4 *kp = reinterpret_cast<const f32x4 *>(a.k + cb * C * DK);
    const float *gp = a.g + cb * C;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int e = threadIdx.x + 256 * i;
      if (nv % 256 == 0 || e < nv) {
        p.w[i] = wp[e];
        p.k[i] = kp[e];
        p.grow[i] = gp[e / q4];
      }
    }
    p.gl = gp[C - 1];
    p.xin = f32x4{0.f, 0.f, 0.f, 0.f};
    const float *xs = REV ? a.dx : a.u;
    if (w < xt && xs)
#pragma unroll
      for (int r = 0; r < 4; ++r) p.xin[r] = xs[(cb * C + 16 * w + 4 * lq + r) * a.Dv + v0 + lr];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = w + 4 * j;
      p.pin[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (REV && a.dp && m < st)
#pragma unroll
        for (int r = 0; r < 4; ++r) p.pin[j][r] = a.dp[(cb * DK + 16 * m + 4 * lq + r) * a.Dv + v0 + lr];
    }
  };
  // everything the chunk needs into LDS: W, Kd = k e^{gamma_C - gamma_c}, the U / dX and
  // dP columns, the last decay
  auto store = [&](const Pre<NP> &p) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int e = threadIdx.x + 256 * i;
      if (nv % 256 == 0 || e < nv) {
        const int row = e / q4, c0 = 4 * (e - row * q4);
        const float dec = __expf(p.gl - p.grow[i]);
        *reinterpret_cast<f32x4 *>(sW + row * sw_st + c0) = p.w[i];
        *reinterpret_cast<f32x4 *>(sKd + row * kd_st + c0) = p.k[i] * dec;
      }
    }
    if (w < xt)
#pragma unroll
      for (int r = 0; r < 4; ++r) sXin[(16 * w + 4 * lq + r) * kCols + lr] = p.xin[r];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = w + 4 * j;
      if (REV && m < st)
#pragma unroll
        for (int r = 0; r < 4; ++r) sPin[(16 * m + 4 * lq + r) * kCols + lr] = p.pin[j][r];
    }
    if (threadIdx.x == 0) sGl = p.gl;
  };

  // the state's tiles this wave owns (tiles w and w + 4), in registers and LDS
  f32x4 sreg[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = w + 4 * j;
    sreg[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (m < st)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * m + 4 * lq + r;
        sreg[j][r] = a.s0 ? a.s0[(bh * DK + row) * a.Dv + v0 + lr] : 0.f;
        sS[row * kCols + lr] = sreg[j][r];
      }
  }
  auto chunk_of = [&](int i) { return REV ? a.N - 1 - i : i; };
  Pre<NP> pre;
  if (a.N > 0) {
    load(chunk_of(0), pre);
    store(pre);
  }
  __syncthreads();

  for (int i = 0; i < a.N; ++i) {
    const int64_t cb = bh * a.N + chunk_of(i);
    if (i + 1 < a.N) load(chunk_of(i + 1), pre);  // in flight during this chunk's products
    const float egl = __expf(sGl);
    const f32x4 sold[2] = {sreg[0], sreg[1]};  // forward: P_n; reverse: dSn_n
    // forward: X = U - W S;  reverse: dx = Kd gS + dX   (four independent product chains)
    f32x4 xv = {0.f, 0.f, 0.f, 0.f};
    if (w < xt) {
      const float *am = REV ? sKd : sW;
      const int ast = REV ? kd_st : sw_st;
      f32x4 acc[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
      for (int s = 0; s < DK / 4; s += 4)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          acc[t] = mma4(am[(16 * w + lr) * ast + 4 * (s + t) + lq], sS[(4 * (s + t) + lq) * kCols + lr], acc[t]);
      const f32x4 prod = (acc[0] + acc[1]) + (acc[2] + acc[3]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * w + 4 * lq + r;
        const float xin = sXin[row * kCols + lr];
        xv[r] = REV ? xin + prod[r] : xin - prod[r];
        sX[row * kCols + lr] = xv[r];
      }
    }
    __syncthreads();  // X complete
    // forward: S <- e^{gamma_C} S + Kd^T X;  reverse: gS <- e^{gamma_C} gS - W^T dx + dP
    {
      const float *am = REV ? sW : sKd;
      const int ast = REV ? sw_st : kd_st;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int m = w + 4 * j;
        if (m < st) {
          f32x4 acc[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
          for (int s = 0; s < C / 4; s += 4)
#pragma unroll
            for (int t = 0; t < 4; ++t)
              acc[t] = mma4(am[(4 * (s + t) + lq) * ast + 16 * m + lr], sX[(4 * (s + t) + lq) * kCols + lr], acc[t]);
          const f32x4 prod = (acc[0] + acc[1]) + (acc[2] + acc[3]);
          f32x4 nv4 = sreg[j] * egl;
          if (REV) {
#pragma unroll
            for (int r = 0; r < 4; ++r) nv4[r] += sPin[(16 * m + 4 * lq + r) * kCols + lr] - prod[r];
          } else {
            nv4 += prod;
          }
          sreg[j] = nv4;
#pragma unroll
          for (int r = 0; r < 4; ++r) sS[(16 * m + 4 * lq + r) * kCols + lr] = nv4[r];
        }
      }
    }
    __syncthreads();  // the chunk's reads of W, Kd, X and the inputs are done
    if (i + 1 < a.N) store(pre);
    // the chunk's stores, after the waits for the loads above
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = w + 4 * j;
      if (m < st)
#pragma unroll
        for (int r = 0; r < 4; ++r) a.p[(cb * DK + 16 * m + 4 * lq + r) * a.Dv + v0 + lr] = sold[j][r];
    }
    if (!REV && w < xt)
#pragma unroll
      for (int r = 0; r < 4; ++r) a.x[(cb * C + 16 * w + 4 * lq + r) * a.Dv + v0 + lr] = xv[r];
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = w + 4 * j;
    if (m < st)
#pragma unroll
      for (int r = 0; r < 4; ++r) a.s_out[(bh * DK + 16 * m + 4 * lq + r) * a.Dv + v0 + lr] = sreg[j][r];
  }
}

template <bool REV>
int launch_scan(const ScanArgs &a, int BH, hipStream_t stream) {
  const dim3 grid(a.Dv / kCols, BH), block(256);
#define MOTIF_SCAN_CASE(CC, DD)                                        \
  if (a.C == CC && a.Dk == DD) {                                      \
    gdn_scan_f32_kernel<REV, CC, DD><<<grid, block, 0, stream>>>(a); \
    return check_launch("gdn_scan_f32_kernel");                       \
  }
#define MOTIF_SCAN_DK(CC) MOTIF_SCAN_CASE(CC, 16) MOTIF_SCAN_CASE(CC, 32) MOTIF_SCAN_CASE(CC, 64) MOTIF_SCAN_CASE(CC, 128)
  MOTIF_SCAN_DK(16)
  MOTIF_SCAN_DK(32)
  MOTIF_SCAN_DK(64)
#undef MOTIF_SCAN_DK
#undef MOTIF_SCAN_CASE
  return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_scan_f32: C in {16, 32, 64} and Dk in {16, 32, 64, 128}");
}

// ------------------------------------------------------------------ operator-form scan
// The same two recurrences with each chunk's step folded into one affine operator, formed
// in parallel before the scan (all chunks at once):
//   forward   S_{n+1} = A_n S_n + H_n,     A_n = e^{gamma_C} I - Kd_n^T W_n,  H_n = Kd_n^T U_n
//   reverse   gS_n    = A_n^T gS_{n+1} + G_n,                 G_n = dP_n - W_n^T dX_n
// (expanding the loops above: X_n = U_n - W_n S_n and dx = Kd_n gS + dX_n substituted),
// so a chunk costs one Dk x Dk x 16 product per workgroup and one barrier instead of two
// products and three barriers; X_n = U_n - W_n P_n is then formed outside the scan, for
// all chunks in parallel.  The kernel walks S <- M_n S + Q_n over the chunks in order
// (REV: last to first) and records S before each step: P_n (forward) or dSn_n (reverse),
// with M = A (forward) or A^T (reverse) handed in row-major.
// Workgroup = (16 state columns, batch.head), 4 waves; wave w owns state row tiles
// w, w + 4, ...  M_n goes through LDS (double buffered, filled from registers loaded
// kOpDepth chunks ahead), S^T through LDS (double buffered) for the B operands; the k-sum
// of each tile is split over four accumulators (independent MFMA chains).  TRANS reads
// M_n transposed (the reverse scan takes A_n as the forward scan does).  Workgroups go
// to the 8 XCDs round-robin by linear id: the column groups of one batch.head are
// placed on one XCD, so each M_n comes from HBM once and from that XCD's L2 after.
constexpr int kOpDepth = 4;
constexpr int kXcds = 8;

template <int DK>
struct OpPre {
  static constexpr int kMv = DK * DK / 4 / 256 > 0 ? DK * DK / 4 / 256 : 1;  // float4 of M per thread
  static constexpr int kJt = (DK / 16 + 3) / 4;                             // row tiles per wave
  f32x4 m[kMv];
  f32x4 q[kJt];
};

struct OpScanArgs {
  const float *M, *Q, *s0;  // [BH][N][DK][DK], [BH][N][DK][Dv], [BH][DK][Dv] or null
  float *rec, *s_out;       // [BH][N][DK][Dv], [BH][DK][Dv]
  int N, Dv, BH, rev;
};
template <int DK> constexpr int opscan_ms() { return DK + 4; }  // LDS row stride (floats) of M and S^T
// workgroups of one scan: whole groups of column-group workgroups per XCD
inline int opscan_blocks(int BH, int Dv) { return (BH + kXcds - 1) / kXcds * kXcds * (Dv / kCols); }

// One scan on workgroup `id` of its launch range, with the caller's LDS: sM [2][DK * MS]
// and sS [2][16 * MS] floats.
template <int DK, bool TRANS>
__device__ __forceinline__ void opscan_body(const OpScanArgs &oa, int id, float (*sM)[DK * opscan_ms<DK>()],
                                            float (*sS)[kCols * opscan_ms<DK>()]) {
  constexpr int TT = DK / 16, MS = opscan_ms<DK>();  // row tiles; LDS row stride
  using PR = OpPre<DK>;
  const float *__restrict__ M = oa.M, *__restrict__ Q = oa.Q, *__restrict__ s0 = oa.s0;
  float *__restrict__ rec = oa.rec, *__restrict__ s_out = oa.s_out;
  const int N = oa.N, Dv = oa.Dv, BH = oa.BH, rev = oa.rev;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lr = lane & 15, lq = lane >> 4;
  // linear id L on XCD L % 8: slot L / 8 of that XCD holds column group slot % ncg of
  // batch.head 8 (slot / ncg) + L % 8 (the grid is padded to whole groups per XCD)
  const int ncg = Dv / kCols, slot = id / kXcds;
  const int bh = (slot / ncg) * kXcds + id % kXcds, v0 = (slot % ncg) * kCols;
  if (bh >= BH) return;
  const size_t mstride = static_cast<size_t>(DK) * DK, qstride = static_cast<size_t>(DK) * Dv;
  const float *Mb = M + static_cast<size_t>(bh) * N * mstride;
  const float *Qb = Q + static_cast<size_t>(bh) * N * qstride;
  float *recb = rec + static_cast<size_t>(bh) * N * qstride;
  auto order = [&](int i) { return rev ? N - 1 - i : i; };

  // element (row, col) of a state-shaped [DK][Dv] matrix held by this lane for tile m, r
  auto qoff = [&](int m, int r) { return static_cast<size_t>(16 * m + 4 * lq + r) * Dv + v0 + lr; };
  auto load = [&](PR &pr, int n) {
    const float *mp = Mb + static_cast<size_t>(n) * mstride;
#pragma unroll
    for (int e = 0; e < PR::kMv; ++e) {
      const int idx = tid + 256 * e;  // float4 index
      if (idx < DK * DK / 4) pr.m[e] = *reinterpret_cast<const f32x4 *>(mp + 4 * idx);
    }
    const float *qp = Qb + static_cast<size_t>(n) * qstride;
#pragma unroll
    for (int j = 0; j < PR::kJt; ++j) {
      const int m = w + 4 * j;
      if (m < TT)
#pragma unroll
        for (int r = 0; r < 4; ++r) pr.q[j][r] = qp[qoff(m, r)];
    }
  };
  auto put_m = [&](const PR &pr, int buf) {
#pragma unroll
    for (int e = 0; e < PR::kMv; ++e) {
      const int idx = tid + 256 * e;
      if (idx < DK * DK / 4) {
        const int row = (4 * idx) / DK, col = (4 * idx) % DK;
        *reinterpret_cast<f32x4 *>(&sM[buf][row * MS + col]) = pr.m[e];
      }
    }
  };

  f32x4 sreg[PR::kJt];
#pragma unroll
  for (int j = 0; j < PR::kJt; ++j) {
    const int m = w + 4 * j;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sreg[j][r] = (s0 && m < TT) ? s0[static_cast<size_t>(bh) * qstride + qoff(m, r)] : 0.f;
    if (m < TT) *reinterpret_cast<f32x4 *>(&sS[0][lr * MS + 16 * m + 4 * lq]) = sreg[j];
  }
  PR pre[kOpDepth];
#pragma unroll
  for (int d = 0; d < kOpDepth; ++d)
    if (d < N) load(pre[d], order(d));
  if (N > 0) put_m(pre[0], 0);
  __syncthreads();

  // step i with the register stages of chunk i (cur) and of chunk i + 1 (nxt); the loop
  // below is unrolled by kOpDepth so the stage indices are compile-time constants
  auto step = [&](int i, PR &cur, const PR &nxt) {
    const int n = order(i), buf = i & 1;
    float *rp = recb + static_cast<size_t>(n) * qstride;
#pragma unroll
    for (int j = 0; j < PR::kJt; ++j) {
      const int m = w + 4 * j;
      if (m < TT) {
#pragma unroll
        for (int r = 0; r < 4; ++r) rp[qoff(m, r)] = sreg[j][r];
        f32x4 acc[4] = {cur.q[j], {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        const float *mrow = TRANS ? &sM[buf][4 * lq * MS + 16 * m + lr] : &sM[buf][(16 * m + lr) * MS + 4 * lq];
        const float *srow = &sS[buf][lr * MS + 4 * lq];
#pragma unroll
        for (int b = 0; b < TT; ++b) {
          f32x4 a4;
          if (TRANS) {  // M^T[16 m + lr][16 b + 4 lq + t] = M[16 b + 4 lq + t][16 m + lr]
#pragma unroll
            for (int t = 0; t < 4; ++t) a4[t] = mrow[(16 * b + t) * MS];
          } else {
            a4 = *reinterpret_cast<const f32x4 *>(mrow + 16 * b);
          }
          const f32x4 s4 = *reinterpret_cast<const f32x4 *>(srow + 16 * b);
#pragma unroll
          for (int t = 0; t < 4; ++t) acc[t] = mma4(a4[t], s4[t], acc[t]);
        }
        sreg[j] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        *reinterpret_cast<f32x4 *>(&sS[buf ^ 1][lr * MS + 16 * m + 4 * lq]) = sreg[j];
      }
    }
    if (i + 1 < N) put_m(nxt, buf ^ 1);
    if (i + kOpDepth < N) load(cur, order(i + kOpDepth));
    __syncthreads();
  };
  int i = 0;
  for (; i + kOpDepth <= N; i += kOpDepth) {
#pragma unroll
    for (int j = 0; j < kOpDepth; ++j) step(i + j, pre[j], pre[(j + 1) % kOpDepth]);
  }
#pragma unroll
  for (int j = 0; j < kOpDepth - 1; ++j)
    if (i + j < N) step(i + j, pre[j], pre[(j + 1) % kOpDepth]);
#pragma unroll
  for (int j = 0; j < PR::kJt; ++j) {
    const int m = w + 4 * j;
    if (m < TT)
#pragma unroll
      for (int r = 0; r < 4; ++r) s_out[static_cast<size_t>(bh) * qstride + qoff(m, r)] = sreg[j][r];
  }
}

template <int DK, bool TRANS>
__global__ void __launch_bounds__(256) gdn_opscan_f32_kernel(OpScanArgs oa) {
  __shared__ __attribute__((aligned(16))) float sM[2][DK * opscan_ms<DK>()];
  __shared__ __attribute__((aligned(16))) float sS[2][kCols * opscan_ms<DK>()];
  opscan_body<DK, TRANS>(oa, blockIdx.x, sM, sS);
}

// Both scans of the backward in one launch (they are independent: the reverse scan needs
// only A and G): workgroups [0, g1) walk the forward scan, the rest the reverse one (A
// read transposed), so the two serial chains run side by side.
template <int DK>
__global__ void __launch_bounds__(256) gdn_opscan_pair_f32_kernel(OpScanArgs fwd, OpScanArgs rev, int g1) {
  __shared__ __attribute__((aligned(16))) float sM[2][DK * opscan_ms<DK>()];
  __shared__ __attribute__((aligned(16))) float sS[2][kCols * opscan_ms<DK>()];
  const int id = blockIdx.x;
  if (id < g1) opscan_body<DK, false>(fwd, id, sM, sS);
  else opscan_body<DK, true>(rev, id - g1, sM, sS);
}

int check_scan_sizes(int BH, int N, int C, int Dk, int Dv, const char *who) {
  if (BH < 0 || N < 0 || C <= 0 || Dk <= 0 || Dv <= 0) return set_error(MOTIF_ERR_INVALID, std::string(who) + ": bad sizes");
  if ((C != 16 && C != 32 && C != 64) || (Dk != 16 && Dk != 32 && Dk != 64 && Dk != 128) || Dv % kCols)
    return set_error(MOTIF_ERR_UNSUPPORTED,
                     std::string(who) + ": needs C in {16, 32, 64}, Dk in {16, 32, 64, 128} and Dv a multiple of 16");
  return MOTIF_OK;
}

}  // namespace

}  // namespace motif

extern "C" int motif_gdn_scan_fwd_f32(const float *k, const float *W, const float *U, const float *g, const float *S0,
                                      float *P, float *X, float *S_out, int BH, int N, int C, int Dk, int Dv,
                                      void *stream) {
  using namespace motif;
  if (int rc = check_scan_sizes(BH, N, C, Dk, Dv, "gdn_scan_fwd_f32")) return rc;
  if (BH == 0) return MOTIF_OK;
  if ((N > 0 && (!k || !W || !U || !g || !P || !X)) || !S_out)
    return set_error(MOTIF_ERR_INVALID, "gdn_scan_fwd_f32: NULL pointer");
  if ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(W)) & 15)
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_scan_fwd_f32: k and W need 16-byte alignment");
  ScanArgs a{k, W, U, g, S0, nullptr, nullptr, P, X, S_out, N, C, Dk, Dv};
  return launch_scan<false>(a, BH, static_cast<hipStream_t>(stream));
}

extern "C" int motif_gdn_scan_bwd_f32(const float *k, const float *W, const float *g, const float *dX, const float *dP,
                                      const float *dS_final, float *dSn, float *dS0, int BH, int N, int C, int Dk,
                                      int Dv, void *stream) {
  using namespace motif;
  if (int rc = check_scan_sizes(BH, N, C, Dk, Dv, "gdn_scan_bwd_f32")) return rc;
  if (BH == 0) return MOTIF_OK;
  if ((N > 0 && (!k || !W || !g || !dSn)) || !dS0)
    return set_error(MOTIF_ERR_INVALID, "gdn_scan_bwd_f32: NULL pointer");
  if ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(W)) & 15)
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_scan_bwd_f32: k and W need 16-byte alignment");
  ScanArgs a{k, W, nullptr, g, dS_final, dX, dP, dSn, nullptr, dS0, N, C, Dk, Dv};
  return launch_scan<true>(a, BH, static_cast<hipStream_t>(stream));
}

extern "C" int motif_gdn_opscan_f32(const float *M, const float *Q, const float *S0, float *rec, float *S_out, int BH,
                                    int N, int Dk, int Dv, int reverse, int transpose, void *stream) {
  using namespace motif;
  if (BH < 0 || N < 0 || Dk <= 0 || Dv <= 0) return set_error(MOTIF_ERR_INVALID, "gdn_opscan_f32: bad sizes");
  if ((Dk != 16 && Dk != 32 && Dk != 64) || Dv % kCols)
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_opscan_f32: needs Dk in {16, 32, 64} and Dv a multiple of 16");
  if (BH == 0) return MOTIF_OK;
  if ((N > 0 && (!M || !Q || !rec)) || !S_out) return set_error(MOTIF_ERR_INVALID, "gdn_opscan_f32: NULL pointer");
  if (reinterpret_cast<uintptr_t>(M) & 15) return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_opscan_f32: M needs 16-byte alignment");
  const dim3 grid(opscan_blocks(BH, Dv)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const OpScanArgs oa{M, Q, S0, rec, S_out, N, Dv, BH, reverse};
#define MOTIF_OPSCAN(D, T) gdn_opscan_f32_kernel<D, T><<<grid, block, 0, s>>>(oa)
  if (Dk == 16) { if (transpose) MOTIF_OPSCAN(16, true); else MOTIF_OPSCAN(16, false); }
  else if (Dk == 32) { if (transpose) MOTIF_OPSCAN(32, true); else MOTIF_OPSCAN(32, false); }
  else { if (transpose) MOTIF_OPSCAN(64, true); else MOTIF_OPSCAN(64, false); }
#undef MOTIF_OPSCAN
  return check_launch("gdn_opscan_f32_kernel");
}

extern "C" int motif_gdn_opscan_pair_f32(const float *A, const float *Hn, const float *S0, float *P, float *S_out,
                                         const float *G, const float *dS_final, float *dSn, float *dS0, int BH, int N,
                                         int Dk, int Dv, void *stream) {
  using namespace motif;
  if (BH < 0 || N < 0 || Dk <= 0 || Dv <= 0) return set_error(MOTIF_ERR_INVALID, "gdn_opscan_pair_f32: bad sizes");
  if ((Dk != 16 && Dk != 32 && Dk != 64) || Dv % kCols)
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_opscan_pair_f32: needs Dk in {16, 32, 64} and Dv a multiple of 16");
  if (BH == 0) return MOTIF_OK;
  if ((N > 0 && (!A || !Hn || !P || !G || !dSn)) || !S_out || !dS0)
    return set_error(MOTIF_ERR_INVALID, "gdn_opscan_pair_f32: NULL pointer");
  if (reinterpret_cast<uintptr_t>(A) & 15)
    return set_error(MOTIF_ERR_UNSUPPORTED, "gdn_opscan_pair_f32: A needs 16-byte alignment");
  const int g1 = opscan_blocks(BH, Dv);
  const dim3 grid(2 * g1), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const OpScanArgs fwd{A, Hn, S0, P, S_out, N, Dv, BH, 0}, rev{A, G, dS_final, dSn, dS0, N, Dv, BH, 1};
  if (Dk == 16) gdn_opscan_pair_f32_kernel<16><<<grid, block, 0, s>>>(fwd, rev, g1);
  else if (Dk == 32) gdn_opscan_pair_f32_kernel<32><<<grid, block, 0, s>>>(fwd, rev, g1);
  else gdn_opscan_pair_f32_kernel<64><<<grid, block, 0, s>>>(fwd, rev, g1);
  return check_launch("gdn_opscan_pair_f32_kernel");
}
