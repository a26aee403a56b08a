// y = x W^T for a few activation rows (M <= 64 per launch row-block): the
// projections of a decode step (nn.Linear with the weight W [N, K] row-major, bf16,
// fp32 accumulation), with the elementwise op that follows each of them fused in:
//   EPI_NONE    y = x W^T
//   EPI_GATE    y = (x W^T) * sigmoid(aux)          Chord: o_proj(out) * sigmoid(g_proj h)
//                                                   (motif/block/attention/chord_attn.py:117, :312)
//   EPI_RESID   y = (x W^T) + aux, y2 = aux2 + y    decoder: f_h = attn + mlp, then the block's
//                                                   running sum (motif/block/decoder.py:205-210,
//                                                   motif/model/cache.py:264-266 in this package)
//   EPI_SWIGLU  y = (x W_a^T) * SiLU(x W_b^T)       SwiGLU MLP (motif/block/mlp.py:42-63 with
//                                                   motif/ops/swiglu.py:252-253), W = [W_a; W_b]
// Every intermediate is rounded to bf16 where the reference's separate ops round
// (GEMM output, sigmoid / SiLU output, product / sum).
//
// At M = 64 the weight is the only large operand: N * K * 2 bytes streamed once from
// HBM.  A workgroup computes an (16 MT) x (16 NT) output tile over the whole of K; its
// 8 waves split K, and each wave issues the loads of its whole share (up to 8 k-steps
// of 32) at once, so a launch costs one memory round trip rather than one per k-step.
// The v_mfma_f32_16x16x32_bf16 partial sums meet in LDS for the epilogue.  What bounds
// a workgroup is the bytes through its CU, (16 MT + 16 NT) * K * 2, so the host picks
// the largest tile whose grid still has 100 workgroups or more (200 for SWIGLU, below);
// the workgroups that share a
// weight tile are placed on one XCD (workgroups go to XCDs round-robin), so the tile
// comes from HBM once and from that XCD's L2 after.
#include "capi_internal.h"
#include "common.h"

namespace motif {

namespace {

enum { EPI_NONE = 0, EPI_GATE = 1, EPI_RESID = 2, EPI_SWIGLU = 3 };

struct LinArgs {
  const bf16_t *x; int64_t x_rs;     // [M, K]
  const bf16_t *w; int64_t w_rs;     // [N, K]
  bf16_t *y; int64_t y_rs;           // [M, Nout]
  const bf16_t *aux; int64_t aux_rs; // GATE: gate pre-activation; RESID: residual  [M, Nout]
  const bf16_t *aux2; int64_t aux2_rs;
  bf16_t *y2; int64_t y2_rs;         // RESID: y2 = aux2 + y (skipped when y2 is NULL)
  int M, N, K;                       // N = rows of W (SWIGLU: 2 * Nout)
  int mblocks, ntiles;               // output tiles along M and along the columns
  int grid;                          // workgroups of this problem
};

constexpr int kWaves = 8;
constexpr int kMaxSteps = 8;  // k-steps (of 32) per wave per round trip
constexpr int kXcds = 8;

__device__ __forceinline__ f32x4 mma(const bf16x8 &a, const bf16x8 &b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 ld8(buf_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
// A weight piece read by this workgroup alone (whole-row tiles: no other workgroup of the
// launch reads it): a nontemporal load (cache policy 2), so the stream does not evict
// the activation rows every workgroup re-reads.
template <bool STREAM>
__device__ __forceinline__ bf16x8 ldw(buf_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, STREAM ? 2 : 0));
}

__device__ __forceinline__ float rb(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// Output column of W tile t, column c of a workgroup whose first output column is n0.
// SWIGLU pairs value tile t with gate tile t (W rows nout + ...), so a workgroup of NT
// W tiles covers 16 NT / 2 output columns there.
template <int NT, int EPI>
__device__ __forceinline__ int w_row(int n0, int t, int c, int nout) {
  if (EPI == EPI_SWIGLU) return (t < NT / 2 ? 0 : nout) + n0 + 16 * (t % (NT / 2)) + c;
  return n0 + 16 * t + c;
}

// Per k-step a lane holds P 16-byte pieces of its row: P = 2 covers 64 k per step with
// the lane's two pieces adjacent (k = 16 kq .. 16 kq + 15 of the step), so one load
// instruction spans whole 128-byte lines (every 32-byte sector of a row's line) and the
// L1 asks L2 for full lines -- half the requests of P = 1 (16 rows x 64 bytes per
// instruction).  MFMA j of the step sums k = 16 kq + 8 j .. +7 over the lane groups
// kq, the same set in A and B, so the products are unchanged.
// The activation rows of a wave's k-steps go through LDS when they fit (P == 2, at most
// 8 row tiles x k-steps): direct buffer-to-LDS loads of whole 128-byte row segments, 8 rows
// per instruction (a load instruction spanning 16 rows x 64 bytes, the MFMA operand
// layout, keeps twice the lines in flight per byte and measured slower), then 16-byte LDS
// reads in operand order.  Each wave stages its rows in its own LDS region, which then
// takes its partial sums for the cross-wave sum; a row's 16-byte chunks are XOR-swizzled
// by row so the operand reads of 16 rows spread over the banks.
template <int MT, int KS, int P>
constexpr bool x_staged() { return P == 2 && MT * KS <= 8; }
// LDS per wave: partials [MT * NT][64] f32x4 or the staged rows [KS][16 MT][128 B]
template <int MT, int NT, int KS, int P>
constexpr int wave_lds() {
  return MT * NT * 1024 > (x_staged<MT, KS, P>() ? KS * MT * 2048 : 0) ? MT * NT * 1024 : KS * MT * 2048;
}
template <int MT, int NT, int KS, int P>
constexpr int tile_lds() { return kWaves * wave_lds<MT, NT, KS, P>(); }

// 16 bytes per lane of rows [8 g, 8 g + 8) x one 128-byte k-step of the staged rows
// (lane l: row 8 g + l / 8, physical chunk l % 8 holding logical chunk (l % 8) ^ (row % 8)),
// into dst + 16 l
__device__ __forceinline__ void x_stage(buf_t xb, char *dst, uint32_t voff, uint32_t soff) {
  buf_ld16_lds(xb, dst, voff, soff);
}

// One workgroup's output tile; `id` is its index among the launch's workgroups for this
// problem, `red` the LDS for the cross-wave sum.
template <int MT, int NT, int KS, int EPI, int P>
__device__ __forceinline__ void rows_tile(const LinArgs &a, const int id, char *lds) {
  constexpr bool XS = x_staged<MT, KS, P>();
  constexpr int WL = wave_lds<MT, NT, KS, P>();
  // The wave index in an SGPR: the k-range below is then wave-uniform to the compiler
  // (scalar branches, step offsets in the loads' scalar offset operand).
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  constexpr int kCols = EPI == EPI_SWIGLU ? 8 * NT : 16 * NT;  // output columns per tile
  const int nout = EPI == EPI_SWIGLU ? a.N / 2 : a.N;

  // XCD-aware tile order: the mblocks workgroups of one column tile sit kXcds ids apart.
  const int group = id / (kXcds * a.mblocks), r = id % (kXcds * a.mblocks);
  const int nt = group * kXcds + r % kXcds, mb = r / kXcds;
  if (nt >= a.ntiles) return;
  const int n0 = nt * kCols, m0 = mb * 16 * MT;
  const int rows = min(a.M - m0, 16 * MT);

  // Output row r depends only on x row r and output column c only on W row c, so
  // tiles past M or N read a clamped (valid) row and their outputs are not stored.
  const bf16_t *xbase = a.x + static_cast<int64_t>(m0) * a.x_rs;
  const buf_t xb = make_buf(xbase, static_cast<uint32_t>(((rows - 1) * a.x_rs + a.K) * 2));
  const buf_t wb = make_buf(a.w, static_cast<uint32_t>(((a.N - 1) * a.w_rs + a.K) * 2));
  uint32_t xo[MT], wo[NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xo[mt] = static_cast<uint32_t>((min(mt * 16 + r16, rows - 1) * a.x_rs + kq * 8 * P) * 2);
#pragma unroll
  for (int t = 0; t < NT; ++t)
    wo[t] = static_cast<uint32_t>((min(w_row<NT, EPI>(n0, t, r16, nout), a.N - 1) * a.w_rs + kq * 8 * P) * 2);

  const int nsteps = a.K / (32 * P);
  const int s0 = wv * nsteps / kWaves, s1 = (wv + 1) * nsteps / kWaves;
  char *wlds = lds + wv * WL;  // this wave's LDS region
  uint32_t xso[XS ? 2 * MT : 1];
  if constexpr (XS) {
#pragma unroll
    for (int g8 = 0; g8 < 2 * MT; ++g8) {
      const int rl = 8 * g8 + (lane >> 3);
      xso[g8] = static_cast<uint32_t>((min(rl, rows - 1) * a.x_rs + 8 * ((lane & 7) ^ (rl & 7))) * 2);
    }
  }

  f32x4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // KS k-steps per round trip (longer K loops).  Steps past the wave's range
  // read at an offset of 2^31 or more, which the range check turns into zeros (every
  // operand offset is below 2^31), so every MFMA runs unconditionally: a guard around
  // the MFMAs would let the compiler sink each step's loads into it and pay one
  // memory round trip per step.
  for (int s = s0; s < s1; s += KS) {
    bf16x8 A[KS][P][MT], B[KS][P][NT];
#pragma unroll
    for (int c = 0; c < KS; ++c) {
      const uint32_t soff = s + c < s1 ? static_cast<uint32_t>(s + c) * (64u * P) : 0x80000000u;
      if constexpr (XS) {
#pragma unroll
        for (int g8 = 0; g8 < 2 * MT; ++g8) x_stage(xb, wlds + (c * MT * 16 + 8 * g8) * 128, xso[g8], soff);
      }
#pragma unroll
      for (int j = 0; j < P; ++j) {
        if constexpr (!XS) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) A[c][j][mt] = ld8(xb, xo[mt] + 16 * j, soff);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) B[c][j][t] = ldw<MT == 4>(wb, wo[t] + 16 * j, soff);
      }
    }
    // keep the whole batch of loads ahead of the MFMAs (the scheduler would otherwise
    // interleave them to save registers, serialising the round trips)
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XS) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the staged rows have landed
#pragma unroll
      for (int c = 0; c < KS; ++c)
#pragma unroll
        for (int j = 0; j < P; ++j)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            A[c][j][mt] = *reinterpret_cast<const bf16x8 *>(wlds + (c * MT * 16 + 16 * mt + r16) * 128 +
                                                            ((2 * kq + j) ^ (r16 & 7)) * 16);
    }
#pragma unroll
    for (int c = 0; c < KS; ++c)
#pragma unroll
      for (int j = 0; j < P; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int t = 0; t < NT; ++t) acc[mt][t] = mma(A[c][j][mt], B[c][j][t], acc[mt][t]);
  }

  // Cross-wave sum in LDS: wave w's partials at lds + w * WL, [tile][lane] (16 bytes per
  // lane), over its own staged rows (its reads of them are done: LDS operations of a wave
  // complete in order).
  auto red = [&](int w, int tile, int l) -> f32x4 & {
    return reinterpret_cast<f32x4 *>(lds + w * WL)[tile * 64 + l];
  };
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t) red(wv, mt * NT + t, lane) = acc[mt][t];
  __syncthreads();

  // Thread p (p, p + 512, ...) finishes (row tile mt, value tile tv, lane l): one C tile
  // (two for SWIGLU, the value tile and its gate tile).
  constexpr int kOut = EPI == EPI_SWIGLU ? NT / 2 : NT;  // output tiles per row tile
  for (int p = threadIdx.x; p < MT * kOut * 64; p += 64 * kWaves) {
  const int l = p & 63, tv = (p >> 6) % kOut, mt = (p >> 6) / kOut;
  f32x4 v = red(0, mt * NT + tv, l), g = f32x4{0.f, 0.f, 0.f, 0.f};
  if (EPI == EPI_SWIGLU) g = red(0, mt * NT + tv + kOut, l);
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    v += red(w, mt * NT + tv, l);
    if (EPI == EPI_SWIGLU) g += red(w, mt * NT + tv + kOut, l);
  }
  const int col = n0 + 16 * tv + (l & 15);
  if (col >= nout) continue;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int rr = mt * 16 + 4 * (l >> 4) + j;
    if (rr >= rows) continue;
    const int64_t m = m0 + rr;
    float val = rb(v[j]);
    if (EPI == EPI_SWIGLU) {
      val = val * rb(silu_fast(rb(g[j])));
    } else if (EPI == EPI_GATE) {
      const float gp = bf16_to_f32(a.aux[m * a.aux_rs + col]);
      val = val * rb(rcp_fast(1.f + __builtin_amdgcn_exp2f(-gp * kLog2e)));
    } else if (EPI == EPI_RESID) {
      val = rb(val + bf16_to_f32(a.aux[m * a.aux_rs + col]));
      if (a.y2) a.y2[m * a.y2_rs + col] = f32_to_bf16(bf16_to_f32(a.aux2[m * a.aux2_rs + col]) + val);
    }
    a.y[m * a.y_rs + col] = f32_to_bf16(val);
  }
  }
}

template <int MT, int NT, int KS, int EPI, int P>
__global__ void __launch_bounds__(512) linear_rows_kernel(LinArgs a) {
  __shared__ f32x4 lds[tile_lds<MT, NT, KS, P>() / 16];
  rows_tile<MT, NT, KS, EPI, P>(a, blockIdx.x, reinterpret_cast<char *>(lds));
}

// Two independent projections in one launch (the decoder's attention input projection
// and its MLP gate/up projection, whose inputs are ready together): workgroups
// [0, a1.grid) take problem 1, the rest problem 2.  Each keeps its own tile shape.
template <int MT1, int NT1, int KS1, int EPI1, int MT2, int NT2, int KS2, int EPI2, int P>
__global__ void __launch_bounds__(512) linear_rows_pair_kernel(LinArgs a1, LinArgs a2) {
  constexpr int b1 = tile_lds<MT1, NT1, KS1, P>(), b2 = tile_lds<MT2, NT2, KS2, P>();
  __shared__ f32x4 lds[(b1 > b2 ? b1 : b2) / 16];
  const int id = blockIdx.x;
  if (id < a1.grid) rows_tile<MT1, NT1, KS1, EPI1, P>(a1, id, reinterpret_cast<char *>(lds));
  else rows_tile<MT2, NT2, KS2, EPI2, P>(a2, id - a1.grid, reinterpret_cast<char *>(lds));
}

// The decoder's two output projections into one output tile (no reference
// counterpart as one op; motif/block/decoder.py:205-213 with the o_proj of the attention
// layer and the MLP's down projection):
//   u = T(x1 W1^T)            the attention output (o_proj), GATE: u = T(u * T(sigmoid(gate)))
//   m = T(x2 W2^T)            the MLP output (down_proj)
//   y = T(u + m)              f_h;   y2 = T(aux2 + y) when y2 != NULL (the block's running sum)
// Rounded where the reference's separate ops round.  Each wave runs its share of both
// products' k-steps back to back; each product keeps its own accumulator.
struct DualArgs {
  const bf16_t *x1; int64_t x1_rs; const bf16_t *w1; int64_t w1_rs; int K1;
  const bf16_t *x2; int64_t x2_rs; const bf16_t *w2; int64_t w2_rs; int K2;
  const bf16_t *gate; int64_t gate_rs;
  const bf16_t *aux2; int64_t aux2_rs;
  bf16_t *y; int64_t y_rs; bf16_t *y2; int64_t y2_rs;
  int M, N;
  int mblocks, ntiles;
};

template <int MT, int NT, int KS, bool GATE, int P>
__global__ void __launch_bounds__(512) linear_rows_dual_kernel(DualArgs a) {
  // per wave: both products' partials [2][MT * NT][64] f32x4, or before them the staged rows
  constexpr bool XS = x_staged<MT, KS, P>();
  constexpr int WL = 2 * MT * NT * 1024 > (XS ? KS * MT * 2048 : 0) ? 2 * MT * NT * 1024 : KS * MT * 2048;
  __shared__ f32x4 lds_[kWaves * WL / 16];
  char *lds = reinterpret_cast<char *>(lds_);
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, kq = lane >> 4;
  constexpr int kCols = 16 * NT;
  const int id = blockIdx.x;
  const int group = id / (kXcds * a.mblocks), r = id % (kXcds * a.mblocks);
  const int nt = group * kXcds + r % kXcds, mb = r / kXcds;
  if (nt >= a.ntiles) return;
  const int n0 = nt * kCols, m0 = mb * 16 * MT;
  const int rows = min(a.M - m0, 16 * MT);

  const buf_t xb1 = make_buf(a.x1 + static_cast<int64_t>(m0) * a.x1_rs,
                             static_cast<uint32_t>(((rows - 1) * a.x1_rs + a.K1) * 2));
  const buf_t xb2 = make_buf(a.x2 + static_cast<int64_t>(m0) * a.x2_rs,
                             static_cast<uint32_t>(((rows - 1) * a.x2_rs + a.K2) * 2));
  const buf_t wb1 = make_buf(a.w1, static_cast<uint32_t>(((a.N - 1) * a.w1_rs + a.K1) * 2));
  const buf_t wb2 = make_buf(a.w2, static_cast<uint32_t>(((a.N - 1) * a.w2_rs + a.K2) * 2));
  uint32_t xo1[MT], xo2[MT], wo1[NT], wo2[NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = min(mt * 16 + r16, rows - 1);
    xo1[mt] = static_cast<uint32_t>((row * a.x1_rs + kq * 8 * P) * 2);
    xo2[mt] = static_cast<uint32_t>((row * a.x2_rs + kq * 8 * P) * 2);
  }
  char *wlds = lds + wv * WL;  // this wave's LDS region
  uint32_t xso1[XS ? 2 * MT : 1], xso2[XS ? 2 * MT : 1];
  if constexpr (XS) {
#pragma unroll
    for (int g8 = 0; g8 < 2 * MT; ++g8) {
      const int rl = 8 * g8 + (lane >> 3), row = min(rl, rows - 1), ch = 8 * ((lane & 7) ^ (rl & 7));
      xso1[g8] = static_cast<uint32_t>((row * a.x1_rs + ch) * 2);
      xso2[g8] = static_cast<uint32_t>((row * a.x2_rs + ch) * 2);
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = min(n0 + 16 * t + r16, a.N - 1);
    wo1[t] = static_cast<uint32_t>((n * a.w1_rs + kq * 8 * P) * 2);
    wo2[t] = static_cast<uint32_t>((n * a.w2_rs + kq * 8 * P) * 2);
  }
  // The epilogue's gate and running-sum inputs, loaded first: they arrive during the
  // product loads instead of costing a round trip after the reduction.
  const int ep_l = threadIdx.x & 63, ep_tv = (threadIdx.x >> 6) % NT, ep_mt = (threadIdx.x >> 6) / NT;
  const int ep_col = n0 + 16 * ep_tv + (ep_l & 15);
  const bool ep_on = static_cast<int>(threadIdx.x) < MT * NT * 64 && ep_col < a.N;
  // (kept as raw bf16 until the epilogue: a conversion here would wait for each load)
  uint32_t gpre[4] = {0u, 0u, 0u, 0u}, apre[4] = {0u, 0u, 0u, 0u};
  if (ep_on) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rr = min(ep_mt * 16 + 4 * (ep_l >> 4) + j, rows - 1);
      const int64_t m = m0 + rr;
      if (GATE) gpre[j] = static_cast<uint32_t>(a.gate[m * a.gate_rs + ep_col]);
      if (a.y2) apre[j] = static_cast<uint32_t>(a.aux2[m * a.aux2_rs + ep_col]);
    }
  }
  // Wave w takes the same k-steps of each product as the single-product kernel gives
  // it (w n / kWaves .. (w + 1) n / kWaves), so both sums are formed in the same order
  // as two separate launches would form them: the result is identical to them.
  const int n1 = a.K1 / (32 * P), n2 = a.K2 / (32 * P);
  const int a0 = wv * n1 / kWaves, c1 = (wv + 1) * n1 / kWaves - a0;
  const int b0 = wv * n2 / kWaves, c2 = (wv + 1) * n2 / kWaves - b0;
  const int nv = c1 + c2;  // the wave's steps: c1 of product 1, then c2 of product 2

  f32x4 acc[2][MT][NT];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[u][mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s = 0; s < nv; s += KS) {
    bf16x8 A[KS][P][MT], B[KS][P][NT];
#pragma unroll
    for (int c = 0; c < KS; ++c) {
      const int v = s + c;
      const bool first = v < c1;  // wave-uniform
      // steps past the wave's range read zeros (offset >= 2^31 fails the range check)
      const uint32_t soff = v < nv ? static_cast<uint32_t>(first ? a0 + v : b0 + v - c1) * (64u * P) : 0x80000000u;
      // pick the operand, then load once (a select between two loads would issue both)
      const buf_t xb = first ? xb1 : xb2, wb = first ? wb1 : wb2;
      if constexpr (XS) {
#pragma unroll
        for (int g8 = 0; g8 < 2 * MT; ++g8)
          x_stage(xb, wlds + (c * MT * 16 + 8 * g8) * 128, first ? xso1[g8] : xso2[g8], soff);
      }
#pragma unroll
      for (int j = 0; j < P; ++j) {
        if constexpr (!XS) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) A[c][j][mt] = ld8(xb, (first ? xo1[mt] : xo2[mt]) + 16 * j, soff);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) B[c][j][t] = ld8(wb, (first ? wo1[t] : wo2[t]) + 16 * j, soff);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XS) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the staged rows have landed
#pragma unroll
      for (int c = 0; c < KS; ++c)
#pragma unroll
        for (int j = 0; j < P; ++j)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            A[c][j][mt] = *reinterpret_cast<const bf16x8 *>(wlds + (c * MT * 16 + 16 * mt + r16) * 128 +
                                                            ((2 * kq + j) ^ (r16 & 7)) * 16);
    }
#pragma unroll
    for (int c = 0; c < KS; ++c) {
      // steps past the range add zeros to product 2, which changes nothing
      const int u = __builtin_amdgcn_readfirstlane(s + c < c1 ? 0 : 1);
#pragma unroll
      for (int j = 0; j < P; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            if (u == 0) acc[0][mt][t] = mma(A[c][j][mt], B[c][j][t], acc[0][mt][t]);
            else acc[1][mt][t] = mma(A[c][j][mt], B[c][j][t], acc[1][mt][t]);
          }
    }
  }

  // partials of wave w, product u at lds + w * WL: [u][tile][lane] (over the wave's own
  // staged rows, whose reads are done)
  auto red = [&](int w, int u, int tile, int l) -> f32x4 & {
    return reinterpret_cast<f32x4 *>(lds + w * WL)[(u * MT * NT + tile) * 64 + l];
  };
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t) red(wv, u, mt * NT + t, lane) = acc[u][mt][t];
  __syncthreads();
  const int p = threadIdx.x;
  if (p >= MT * NT * 64) return;
  const int l = p & 63, tv = (p >> 6) % NT, mt = (p >> 6) / NT;
  f32x4 v1 = red(0, 0, mt * NT + tv, l), v2 = red(0, 1, mt * NT + tv, l);
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    v1 += red(w, 0, mt * NT + tv, l);
    v2 += red(w, 1, mt * NT + tv, l);
  }
  const int col = n0 + 16 * tv + (l & 15);
  if (col >= a.N) return;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int rr = mt * 16 + 4 * (l >> 4) + j;
    if (rr >= rows) continue;
    const int64_t m = m0 + rr;
    // (the empty asm keeps the compiler from hoisting the conversions, and with them
    // the waits for these loads, to the top of the kernel)
    uint32_t graw = gpre[j], araw = apre[j];
    asm volatile("" : "+v"(graw), "+v"(araw));
    float u = rb(v1[j]);
    if (GATE) u = rb(u * rb(rcp_fast(1.f + __builtin_amdgcn_exp2f(-bf16_to_f32(static_cast<bf16_t>(graw)) * kLog2e))));
    const float f = rb(u + rb(v2[j]));
    a.y[m * a.y_rs + col] = f32_to_bf16(f);
    if (a.y2) a.y2[m * a.y2_rs + col] = f32_to_bf16(bf16_to_f32(static_cast<bf16_t>(araw)) + f);
  }
}

template <int MT, int NT, int EPI, int P>
int launch_tile_p(const LinArgs &a, const dim3 &grid, hipStream_t s) {
  const dim3 block(64 * kWaves);
  const int per_wave = (a.K / (32 * P) + kWaves - 1) / kWaves;
  if (per_wave <= 1) linear_rows_kernel<MT, NT, 1, EPI, P><<<grid, block, 0, s>>>(a);
  else if (per_wave <= 2) linear_rows_kernel<MT, NT, 2, EPI, P><<<grid, block, 0, s>>>(a);
  else if constexpr (P == 2) {
    linear_rows_kernel<MT, NT, 4, EPI, P><<<grid, block, 0, s>>>(a);  // 64-k steps: 4 per round trip
  } else {
    if (per_wave <= 4) linear_rows_kernel<MT, NT, 4, EPI, P><<<grid, block, 0, s>>>(a);
    else if (per_wave <= 6) linear_rows_kernel<MT, NT, 6, EPI, P><<<grid, block, 0, s>>>(a);
    else linear_rows_kernel<MT, NT, kMaxSteps, EPI, P><<<grid, block, 0, s>>>(a);
  }
  return check_launch("linear_rows_kernel");
}

template <int MT, int NT, int EPI>
int launch_tile(LinArgs a, hipStream_t s) {
  constexpr int kCols = EPI == EPI_SWIGLU ? 8 * NT : 16 * NT;
  const int nout = EPI == EPI_SWIGLU ? a.N / 2 : a.N;
  a.ntiles = (nout + kCols - 1) / kCols;
  a.mblocks = (a.M + 16 * MT - 1) / (16 * MT);
  const int groups = (a.ntiles + kXcds - 1) / kXcds;
  const dim3 grid(groups * kXcds * a.mblocks);
  // 64-k steps with full-line loads when K allows it
  return a.K % 64 == 0 ? launch_tile_p<MT, NT, EPI, 2>(a, grid, s) : launch_tile_p<MT, NT, EPI, 1>(a, grid, s);
}

// Tile choice: rows per tile 16 MT (MT = 4, 2, 1) and W tiles NT (2, or 1 when the
// epilogue allows it), the largest tile whose grid still has enough workgroups: 100
// (200 for SWIGLU, whose tiles carry a value and a gate half).  Measured at M = 64,
// K = 768: N = 4632 7.0 us with 145 whole-row tiles vs 8.1 us with 290 half-row tiles,
// N = 2304 5.1 vs 6.4 us; SWIGLU N = 4096 5.5 us with 256 half-row tiles vs 7.0 with 128.
template <int EPI>
int launch_epi(const LinArgs &a, hipStream_t s) {
  const int nout = EPI == EPI_SWIGLU ? a.N / 2 : a.N;
  const int cols2 = EPI == EPI_SWIGLU ? 16 : 32;  // output columns of an NT = 2 tile
  const int enough = EPI == EPI_SWIGLU ? 200 : 100;
  auto wgs = [&](int mt, int cols) { return ((a.M + 16 * mt - 1) / (16 * mt)) * ((nout + cols - 1) / cols); };
  const int mtmax = a.M > 32 ? 4 : (a.M > 16 ? 2 : 1);
  if (mtmax >= 4 && wgs(4, cols2) >= enough) return launch_tile<4, 2, EPI>(a, s);
  if (mtmax >= 2 && wgs(2, cols2) >= enough) return launch_tile<2, 2, EPI>(a, s);
  if constexpr (EPI == EPI_SWIGLU) {
    return launch_tile<1, 2, EPI>(a, s);  // a value tile and its gate tile
  } else {
    if (wgs(1, cols2) >= enough) return launch_tile<1, 2, EPI>(a, s);
    return launch_tile<1, 1, EPI>(a, s);
  }
}

// Paired launch: problem 1 (none or SwiGLU epilogue) with tile (MT1, NT1), problem 2 a
// SwiGLU projection with tile (MT2, 2); both with the same K.  With 64 rows and short K
// both take whole-row tiles and problem 1 four W tiles (64 columns): about 200
// workgroups, one per CU, so the launch is a single round of workgroups.  Measured at
// M = 64, K = 768 with the 16 decoders' weights cycled (cold): 9.2 us per pair against
// 11.4 with (4, 2) / (2, 2) tiles (400 workgroups, two rounds at one per CU).
template <int MT1, int NT1, int MT2, int EPI1, int KS>
int launch_pair_k(LinArgs a1, LinArgs a2, hipStream_t s) {
  auto prep = [](LinArgs &a, int MT, int NT, int EPI) {
    const int cols = EPI == EPI_SWIGLU ? 8 * NT : 16 * NT;
    const int nout = EPI == EPI_SWIGLU ? a.N / 2 : a.N;
    a.ntiles = (nout + cols - 1) / cols;
    a.mblocks = (a.M + 16 * MT - 1) / (16 * MT);
    a.grid = (a.ntiles + kXcds - 1) / kXcds * kXcds * a.mblocks;
  };
  prep(a1, MT1, NT1, EPI1);
  prep(a2, MT2, 2, EPI_SWIGLU);
  linear_rows_pair_kernel<MT1, NT1, KS, EPI1, MT2, 2, KS, EPI_SWIGLU, 2><<<dim3(a1.grid + a2.grid), dim3(64 * kWaves), 0, s>>>(a1, a2);
  return check_launch("linear_rows_pair_kernel");
}

template <int MT1, int EPI1>
int launch_pair(const LinArgs &a1, const LinArgs &a2, hipStream_t s) {
  const int per_wave = (a1.K / 64 + kWaves - 1) / kWaves;
  if (MT1 == 4 && per_wave <= 2) {
    if (per_wave <= 1) return launch_pair_k<4, 4, 4, EPI1, 1>(a1, a2, s);
    return launch_pair_k<4, 4, 4, EPI1, 2>(a1, a2, s);
  }
  if (per_wave <= 1) return launch_pair_k<MT1, 2, 2, EPI1, 1>(a1, a2, s);
  if (per_wave <= 2) return launch_pair_k<MT1, 2, 2, EPI1, 2>(a1, a2, s);
  return launch_pair_k<MT1, 2, 2, EPI1, 4>(a1, a2, s);
}

template <bool GATE, int KS>
int launch_dual_k(DualArgs a, hipStream_t s) {
  a.ntiles = (a.N + 15) / 16;
  a.mblocks = (a.M + 15) / 16;
  const int grid = (a.ntiles + kXcds - 1) / kXcds * kXcds * a.mblocks;
  linear_rows_dual_kernel<1, 1, KS, GATE, 2><<<dim3(grid), dim3(64 * kWaves), 0, s>>>(a);
  return check_launch("linear_rows_dual_kernel");
}

template <bool GATE>
int launch_dual(const DualArgs &a, hipStream_t s) {
  const int per_wave = (a.K1 / 64 + kWaves - 1) / kWaves + (a.K2 / 64 + kWaves - 1) / kWaves;
  if (per_wave <= 2) return launch_dual_k<GATE, 2>(a, s);
  if (per_wave <= 4) return launch_dual_k<GATE, 4>(a, s);
  return launch_dual_k<GATE, 8>(a, s);
}

bool rows_ok(const void *x, int64_t x_rs, const void *w, int64_t w_rs, int N, int K) {
  if (!x || !w || N <= 0 || K <= 0 || K % 64) return false;
  if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15) || (x_rs % 8) || (w_rs % 8)) return false;
  if (x_rs < K || w_rs < K) return false;
  return (static_cast<int64_t>(N - 1) * w_rs + K) * 2 < (int64_t(1) << 31) &&
         (static_cast<int64_t>(63) * x_rs + K) * 2 < (int64_t(1) << 31);
}

}  // namespace

}  // namespace motif

extern "C" int motif_linear_rows(const void *x, int64_t x_rs, const void *w, int64_t w_rs, void *y, int64_t y_rs,
                                 int M, int N, int K, int epilogue, const void *aux, int64_t aux_rs,
                                 const void *aux2, int64_t aux2_rs, void *y2, int64_t y2_rs, void *stream) {
  using namespace motif;
  if (M < 0 || N <= 0 || K <= 0) return set_error(MOTIF_ERR_INVALID, "linear_rows: bad size");
  if (!x || !w || !y) return set_error(MOTIF_ERR_INVALID, "linear_rows: NULL pointer");
  if (epilogue < EPI_NONE || epilogue > EPI_SWIGLU) return set_error(MOTIF_ERR_INVALID, "linear_rows: epilogue");
  if ((epilogue == EPI_GATE || epilogue == EPI_RESID) && !aux)
    return set_error(MOTIF_ERR_INVALID, "linear_rows: epilogue needs aux");
  if (epilogue == EPI_RESID && y2 && !aux2) return set_error(MOTIF_ERR_INVALID, "linear_rows: y2 needs aux2");
  if (epilogue == EPI_SWIGLU && (N & 1)) return set_error(MOTIF_ERR_INVALID, "linear_rows: SwiGLU needs even N");
  if (K % 32) return set_error(MOTIF_ERR_UNSUPPORTED, "linear_rows: K must be a multiple of 32");
  if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15) || (x_rs % 8) || (w_rs % 8))
    return set_error(MOTIF_ERR_UNSUPPORTED, "linear_rows: x / W rows must be 16-byte aligned");
  if (x_rs < K || w_rs < K) return set_error(MOTIF_ERR_INVALID, "linear_rows: row stride below K");
  if ((static_cast<int64_t>(N - 1) * w_rs + K) * 2 >= (int64_t(1) << 31) ||
      (static_cast<int64_t>(63) * x_rs + K) * 2 >= (int64_t(1) << 31))
    return set_error(MOTIF_ERR_UNSUPPORTED, "linear_rows: operand above 2 GiB");
  if (M == 0) return MOTIF_OK;
  LinArgs a;
  a.x = static_cast<const bf16_t *>(x); a.x_rs = x_rs;
  a.w = static_cast<const bf16_t *>(w); a.w_rs = w_rs;
  a.y = static_cast<bf16_t *>(y); a.y_rs = y_rs;
  a.aux = static_cast<const bf16_t *>(aux); a.aux_rs = aux_rs;
  a.aux2 = static_cast<const bf16_t *>(aux2); a.aux2_rs = aux2_rs;
  a.y2 = static_cast<bf16_t *>(y2); a.y2_rs = y2_rs;
  a.M = M; a.N = N; a.K = K;
  a.mblocks = a.ntiles = 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (epilogue) {
    case EPI_GATE: return launch_epi<EPI_GATE>(a, s);
    case EPI_RESID: return launch_epi<EPI_RESID>(a, s);
    case EPI_SWIGLU: return launch_epi<EPI_SWIGLU>(a, s);
    default: return launch_epi<EPI_NONE>(a, s);
  }
}

extern "C" int motif_linear_rows_pair(const void *x1, int64_t x1_rs, const void *w1, int64_t w1_rs, void *y1,
                                      int64_t y1_rs, int N1, int K1, int epilogue1, const void *x2, int64_t x2_rs,
                                      const void *w2, int64_t w2_rs, void *y2, int64_t y2_rs, int N2, int K2,
                                      int M, void *stream) {
  using namespace motif;
  if (M < 0 || M > 64) return set_error(MOTIF_ERR_UNSUPPORTED, "linear_rows_pair: 1 .. 64 rows");
  if (epilogue1 != EPI_NONE && epilogue1 != EPI_SWIGLU)
    return set_error(MOTIF_ERR_UNSUPPORTED, "linear_rows_pair: problem 1 takes no epilogue or SwiGLU");
  if (K1 != K2 || !rows_ok(x1, x1_rs, w1, w1_rs, N1, K1) || !rows_ok(x2, x2_rs, w2, w2_rs, N2, K2) || !y1 || !y2 ||
      (N2 & 1) || (epilogue1 == EPI_SWIGLU && (N1 & 1)))
    return set_error(MOTIF_ERR_UNSUPPORTED, "linear_rows_pair: unsupported shapes or alignment");
  if (M == 0) return MOTIF_OK;
  LinArgs a1{}, a2{};
  a1.x = static_cast<const bf16_t *>(x1); a1.x_rs = x1_rs; a1.w = static_cast<const bf16_t *>(w1); a1.w_rs = w1_rs;
  a1.y = static_cast<bf16_t *>(y1); a1.y_rs = y1_rs; a1.M = M; a1.N = N1; a1.K = K1;
  a2.x = static_cast<const bf16_t *>(x2); a2.x_rs = x2_rs; a2.w = static_cast<const bf16_t *>(w2); a2.w_rs = w2_rs;
  a2.y = static_cast<bf16_t *>(y2); a2.y_rs = y2_rs; a2.M = M; a2.N = N2; a2.K = K2;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // problem 1's tile as launch_epi would pick it: whole 64-row tiles when they still give ~100 workgroups
  const int cols = epilogue1 == EPI_SWIGLU ? 16 : 32, nout = epilogue1 == EPI_SWIGLU ? N1 / 2 : N1;
  const bool big = M > 32 && ((nout + cols - 1) / cols) >= 100;
  if (epilogue1 == EPI_SWIGLU) return big ? launch_pair<4, EPI_SWIGLU>(a1, a2, s) : launch_pair<2, EPI_SWIGLU>(a1, a2, s);
  return big ? launch_pair<4, EPI_NONE>(a1, a2, s) : launch_pair<2, EPI_NONE>(a1, a2, s);
}

extern "C" int motif_linear_rows_dual(const void *x1, int64_t x1_rs, const void *w1, int64_t w1_rs, int K1,
                                      const void *x2, int64_t x2_rs, const void *w2, int64_t w2_rs, int K2,
                                      const void *gate, int64_t gate_rs, const void *aux2, int64_t aux2_rs, void *y,
                                      int64_t y_rs, void *y2, int64_t y2_rs, int M, int N, void *stream) {
  using namespace motif;
  if (M < 0 || M > 64) return set_error(MOTIF_ERR_UNSUPPORTED, "linear_rows_dual: 1 .. 64 rows");
  if (!rows_ok(x1, x1_rs, w1, w1_rs, N, K1) || !rows_ok(x2, x2_rs, w2, w2_rs, N, K2) || !y || (y2 && !aux2))
    return set_error(MOTIF_ERR_UNSUPPORTED, "linear_rows_dual: unsupported shapes or alignment");
  if (M == 0) return MOTIF_OK;
  DualArgs a{};
  a.x1 = static_cast<const bf16_t *>(x1); a.x1_rs = x1_rs; a.w1 = static_cast<const bf16_t *>(w1); a.w1_rs = w1_rs;
  a.K1 = K1;
  a.x2 = static_cast<const bf16_t *>(x2); a.x2_rs = x2_rs; a.w2 = static_cast<const bf16_t *>(w2); a.w2_rs = w2_rs;
  a.K2 = K2;
  a.gate = static_cast<const bf16_t *>(gate); a.gate_rs = gate_rs;
  a.aux2 = static_cast<const bf16_t *>(aux2); a.aux2_rs = aux2_rs;
  a.y = static_cast<bf16_t *>(y); a.y_rs = y_rs; a.y2 = static_cast<bf16_t *>(y2); a.y2_rs = y2_rs;
  a.M = M; a.N = N;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return gate ? launch_dual<true>(a, s) : launch_dual<false>(a, s);
}
