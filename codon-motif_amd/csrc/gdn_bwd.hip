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
