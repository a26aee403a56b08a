// Chord attention (causal softmax with the gated geometric-decay bias) for gfx950.
//
// chord_fwd_kernel (prefill): flash-style online softmax on bf16 MFMA
// (v_mfma_f32_32x32x16_bf16, fp32 accumulation).  A workgroup is kParts parts of 4
// waves over the same query rows of one kv head; part p walks its own run of the key
// tiles and the partial softmaxes meet in LDS at the end.  A wave owns 32 score
// columns (16 queries of two GQA heads, or 32 queries of one head).  Scores are
// computed transposed, S^T = K Q^T, so lane l owns column l % 32 and its row max is 16
// in-lane values plus one lane swap; the output is accumulated transposed too,
// O^T += V^T P^T, with P^T fed straight from the score accumulators and V^T staged in
// LDS in the matching key order.  K / V tiles are double-buffered in LDS (padded rows),
// one barrier per 64-key tile, workgroups dispatched heaviest query blocks first.  The
// GGD bias depends only on d = key - i_abs: each wave evaluates it in registers (one new
// distance per lane per tile) into an LDS window; no bias is stored in HBM.
//
// chord_decode_kernel (decode / short queries over a long cache): split-K
// flash-decoding.  A workgroup owns (split, kv head, batch row) and serves all
// query rows of that kv head (GQA group x L <= 8), streaming K and V with fully
// coalesced 16-byte loads (8 lanes per key row); dot products are finished
// with 3 xor-shuffles.  Partials (m, l, acc) are merged across the 4 waves in
// LDS and across splits by chord_merge_kernel.
#include <algorithm>
#include <type_traits>

#include "capi_internal.h"
#include "chord_internal.h"
#include "common.h"

namespace motif {

struct ChordArgs {
  const void *q; int64_t q_sb, q_sh, q_st;
  const void *k; int64_t k_sb, k_sh, k_st;
  const void *v; int64_t v_sb, v_sh, v_st;
  const float *alpha, *beta, *mu, *ssmax;
  const float *log_n; int64_t ln_sb, ln_st;
  void *out; int64_t o_sb, o_sh, o_st;
  float *lse;
  int B, H, Hkv, L, S, q_start;
  float scale, eps;
  const int32_t *cu;  // packed sequences (B == 1) or nullptr
  // split-K partials
  float *part;        // [B][Hkv][splits][L * group][D + 2]
  int splits;         // key-range splits (decode kernel)
  int nqc;            // row chunks per (batch, kv head) (decode kernel)
  // device cursor (decode kernels): when set, *len_dev positions are cached, the L
  // new keys sit at [*len_dev, *len_dev + L), S holds the cache capacity, and the
  // merge pass advances *len_dev by L
  int *len_dev;
  const float *log_tab;  // ln(1 .. n) when log_n is NULL: log_n[b, i] = log_tab[q_start + i]
};

// Keys and query start of a decode launch: from the host arguments, or from the
// device cursor (clamped so the window stays inside the capacity).
struct DecodeWindow { int S, q_start; };
__device__ __forceinline__ DecodeWindow decode_window(const ChordArgs &a) {
  if (!a.len_dev) return {min(a.S, a.q_start + a.L), a.q_start};
  const int cached = min(max(__builtin_amdgcn_readfirstlane(*a.len_dev), 0), a.S - a.L);
  return {cached + a.L, cached};
}

__device__ __forceinline__ float log_n_at(const ChordArgs &a, int b, int i, int q_start) {
  return a.log_n ? a.log_n[b * a.ln_sb + int64_t(i) * a.ln_st] : a.log_tab[q_start + i];
}

constexpr int kD = 64;        // head dim
constexpr int kBN = 64;       // keys per tile

__device__ __forceinline__ float ggd_bias(float dist, float alpha, float beta, float mu, float eps) {
  // -alpha * (|d - mu| + eps)^beta, the power through exp2(beta * log2(.)).
  const float x = fabsf(dist - mu) + eps;
  return -alpha * fast_exp2(beta * fast_log2(x));
}

__device__ __forceinline__ __bf16 to_bf(float f) {
  const bf16_t b = f32_to_bf16(f);
  return __builtin_bit_cast(__bf16, b);
}

// ------------------------------------------------------------------ prefill
__device__ __forceinline__ f32x4 mma16(const bf16x8 &a, const bf16x8 &b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x16_bf16 (twice the work of 16x16x32 per issue slot on gfx950): A
// lane l holds row l % 32, k 8 (l / 32) + 0..7; B lane l column l % 32, the same k;
// accumulator register r of lane l holds row 8 (r / 4) + 4 (l / 32) + r % 4, column
// l % 32.
__device__ __forceinline__ f32x16 mma32(const bf16x8 &a, const bf16x8 &b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Position of key k in a V^T row.  P^T comes straight from S^T accumulators, whose
// lane half h holds keys 8a + 4h + (0..3) (a = 0, 1) of each 16-key group, so those
// eight keys are stored together at 8h + 4a: one 16-byte read is the matching A operand.
__device__ __forceinline__ int vperm32(int k) { return (k & ~15) | ((k & 4) << 1) | ((k & 8) >> 1) | (k & 3); }

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk2bf(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){x0, x1}, bf16x2v));
}

// Prefill logit form: q is multiplied by rho_h = sign(ssmax_h * scale) (exact; 0 when
// scale == 0) and each S^T = K Q^T MFMA starts from kappa_h * GGD(key - q_abs) for
// key <= q_abs (-inf above: the causal mask), kappa_h = sign(ssmax_h) / |scale|
// (sign(ssmax_h) when scale == 0), so acc = rho_h (q.k + bias / scale) and the logit is
// |ssmax_h log_n[i] scale| acc (|ssmax_h log_n[i]| acc when scale == 0).

// LDS tile rows of 64 bf16 are padded to 72 (144 B): the row-per-lane 16-byte reads of
// the MFMA operands are free of bank conflicts, and the pieces of one row sit at fixed
// offsets from its start, so every operand read of a step is one base register plus
// an immediate.
constexpr int kRow = 72;

// Each workgroup is kParts parts of 4 waves over the same query rows and heads: part p
// takes the p-th run of ceil(n / kParts) of the rows' n key tiles, each with its own
// double-buffered K / V tiles, and the partial softmaxes are merged through LDS at the
// end.  Splitting the keys four ways keeps the chain of tiles of the longest (last)
// query rows short; one 16-wave workgroup fills a CU (4 waves per SIMD).
//
// A wave owns 32 score columns: 16 queries of two heads of the GQA group (HPW >= 2)
// or 32 queries of one head, so S^T = K Q^T is a 32 x 32 accumulator per 32 keys.
// Lane l owns column l % 32 (its query row and head), and its keys in each 32-key
// sub-tile are 8 (r / 4) + 4 (l / 32) + r % 4: the row max is 16 in-lane values plus
// one swap with lane l ^ 32, and P^T enters O^T += V^T P^T from the same registers.
// Row sums of P (bf16, as P enters the output) by v_dot2 against ones.
//
// The GGD bias of a 64-key tile is read from a window of kappa GGD(key - q_abs) over the
// distances the wave meets in that tile (63 + queries per wave entries per head),
// evaluated in registers (one new entry per lane per tile: the window of tile t + 1
// starts at entry 64 of tile t's) and kept in LDS, where every lane reads its 4
// consecutive entries per key group with 4-byte loads.  Tile data
// is fetched two steps ahead: the loads issued in step i are written to LDS at the
// end of step i + 1.
constexpr int kParts = 4;

template <int HPW>  // query heads per part
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4, 4))) chord_fwd_kernel(ChordArgs a) {
  constexpr int RH = HPW >= 2 ? 2 : 1;  // heads per wave
  constexpr int RQ = 32 / RH;           // queries per wave
  constexpr int HGW = HPW / RH;         // head groups per part
  constexpr int QW = (4 / HGW) * RQ;    // queries per workgroup
  constexpr int kWin = 64 + RQ;         // bias window entries per copy (>= 63 + RQ)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int part = wv >> 2, w = wv & 3;
  const int htid = tid & 255;  // thread index inside the part
  const int lc = lane & 31, hh = lane >> 5;
  const int group = a.H / a.Hkv;
  // grid (head groups, query blocks, sequences): the head groups vary fastest, so the
  // dispatch order runs heaviest (latest) query blocks first across all heads
  const int hg = blockIdx.x, sq = blockIdx.z;

  // Sequence geometry (padded batch row, or one packed sequence).
  int batch, tok0, Lq, Skv, q_start;
  if (a.cu == nullptr) {
    batch = sq; tok0 = 0; Lq = a.L; Skv = a.S; q_start = a.q_start;
  } else {
    batch = 0; tok0 = a.cu[sq]; Lq = a.cu[sq + 1] - tok0; Skv = Lq; q_start = 0;
  }
  const int nqbg = (Lq + QW - 1) / QW;
  if (static_cast<int>(blockIdx.y) >= nqbg) return;
  const int qbg = nqbg - 1 - blockIdx.y;

  const int head0 = hg * HPW + (w % HGW) * RH;  // the wave's first head
  const int cq = lc % RQ;                         // this lane's query inside the wave
  const int head = head0 + lc / RQ;               // this lane's head
  const int kvh = (hg * HPW) / group;
  const int q0 = qbg * QW + (w / HGW) * RQ;
  const int my_q = q0 + cq;
  const bool q_valid = my_q < Lq;

  const int wg_q_last = min(Lq, (qbg + 1) * QW) - 1;
  const int kv_end = min(Skv, q_start + wg_q_last + 1);
  const int ntiles = (kv_end + kBN - 1) / kBN;
  const int nsteps = (ntiles + kParts - 1) / kParts;    // tiles of each part but the last ones
  const int t_first = part * nsteps;
  const int t_count = max(0, min(nsteps, ntiles - t_first));
  const int wave_kv_end = min(Skv, q_start + min(Lq, q0 + RQ));
  // Keys past the cache end are masked here unless no query sits past it.
  const bool kmask = q_start + min(Lq, q0 + RQ) > Skv;

  const bf16_t *kp = static_cast<const bf16_t *>(a.k) + batch * a.k_sb + kvh * a.k_sh + int64_t(tok0) * a.k_st;
  const bf16_t *vp = static_cast<const bf16_t *>(a.v) + batch * a.v_sb + kvh * a.v_sh + int64_t(tok0) * a.v_st;

  // logit = a_row * acc (the prefill logit form above), a_row = |ssmax log_n scale|;
  // the kernel works in log2 units, p = exp2(A (acc - m)) with A = log2e a_row.
  const float ssm = a.ssmax[head];
  const float sg = ssm < 0.f ? -1.f : 1.f;
  const float rho = a.scale > 0.f ? sg : a.scale < 0.f ? -sg : 0.f;
  const float a_head = fabsf(ssm) * (a.scale != 0.f ? fabsf(a.scale) : 1.f) * kLog2e;
  const float lnv = a.log_n[batch * a.ln_sb + int64_t(tok0 + min(my_q, Lq - 1)) * a.ln_st];
  // A > 0 keeps masked keys at exactly 0 (exp2(-inf)); a row with a_row = 0 has
  // finite logits A * acc that round to 0 against the max, as the exact 0 logits do.
  const float A = q_valid ? fmaxf(a_head * lnv, 1e-30f) : 1.f;

  // rho Q^T as the B operand: lane holds rho Q[my_q][16 ds + 8 hh .. +8] of its head
  // (exact: rho in {-1, 0, 1}); rows past Lq are zero.
  bf16x8 qreg[4];
  {
    const bf16_t *qrow = static_cast<const bf16_t *>(a.q) + batch * a.q_sb + head * a.q_sh +
                         int64_t(tok0 + min(my_q, max(Lq - 1, 0))) * a.q_st;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      uint4 u = *reinterpret_cast<const uint4 *>(qrow + 16 * ds + 8 * hh);
      if (rho < 0.f) { u.x ^= 0x80008000u; u.y ^= 0x80008000u; u.z ^= 0x80008000u; u.w ^= 0x80008000u; }
      if (rho == 0.f || !q_valid) u = uint4{0u, 0u, 0u, 0u};
      qreg[ds] = __builtin_bit_cast(bf16x8, u);
    }
  }

  // [part][buffer] K rows and V^T rows (keys in vperm32 order), then per wave a window
  // per head (at least 128 floats: the merge keeps (l, m) there); the merge puts the
  // output partials of parts 1.. over the K / V buffers
  constexpr int kTile = kBN * kRow;  // bf16 elements of one K (or V^T) buffer
  constexpr int kWinF = RH * kWin > 128 ? RH * kWin : 128;
  __shared__ __attribute__((aligned(16))) bf16_t sKV[2][kParts][2][kTile];
  __shared__ __attribute__((aligned(16))) float sB[4 * kParts][kWinF];
  bf16_t (*sK)[2][kTile] = sKV[0];
  bf16_t (*sV)[2][kTile] = sKV[1];

  // Bias window of tile t for wave head hw: entry j (0 .. 63 + RQ - 1) is distance
  // key - q_abs = t kBN - q_start - q0 - (RQ - 1) + j; lane l computes entries l and
  // 64 + l: kappa GGD(distance) for distance <= 0 and -inf past the diagonal (the
  // causal mask), kappa = sign(ssmax) / |scale| (sign(ssmax) when scale == 0).
  const int dist0 = -q_start - q0 - (RQ - 1) + lane;
  float gal[RH], gbe[RH], gmu[RH], gka[RH];
#pragma unroll
  for (int hw = 0; hw < RH; ++hw) {
    gal[hw] = a.alpha[head0 + hw];
    gbe[hw] = a.beta[head0 + hw];
    gmu[hw] = a.mu[head0 + hw];
    const float sgh = a.ssmax[head0 + hw] < 0.f ? -1.f : 1.f;
    gka[hw] = a.scale != 0.f ? sgh / fabsf(a.scale) : sgh;
  }
  auto eval_bias = [&](int hw, int dist) {
    return dist <= 0 ? gka[hw] * ggd_bias(static_cast<float>(dist), gal[hw], gbe[hw], gmu[hw], a.eps) : -INFINITY;
  };
  float bwin[RH][2];
#pragma unroll
  for (int hw = 0; hw < RH; ++hw) {
    bwin[hw][0] = eval_bias(hw, t_first * kBN + dist0);
    bwin[hw][1] = eval_bias(hw, t_first * kBN + dist0 + 64);
  }
  // (entries past 63 + RQ - 1 are never read)
  float *bw = &sB[wv][0];
  auto store_window = [&]() {
#pragma unroll
    for (int hw = 0; hw < RH; ++hw) {
      bw[hw * kWin + lane] = bwin[hw][0];
      if (lane < RQ) bw[hw * kWin + 64 + lane] = bwin[hw][1];
    }
  };
  // This lane's entries for keys 32 kt + 8 q4 + 4 hh + (0..3): j = 32 kt + 8 q4 + jb0 + p
  // with jb0 = 4 hh - cq + RQ - 1.
  const float *bwr = bw + (lc / RQ) * kWin + 4 * hh - cq + RQ - 1;

  // Tile staging by the part's 256 threads: K rows (2 x 16 B per thread); V as key
  // pairs (2 keys x 8 d).  The per-lane offsets are fixed; step t moves the buffer
  // base to its first key (the range shrinks with it, so keys past kv_end read 0).
  uint4 kst[2], vst[2];
  const int vpair = htid & 31, vseg = htid >> 5;
  const uint32_t koff = static_cast<uint32_t>(((htid >> 3) * a.k_st + (htid & 7) * 8) * 2);
  const uint32_t koff2 = koff + static_cast<uint32_t>(32 * a.k_st * 2);
  const uint32_t voff = static_cast<uint32_t>((2 * vpair * a.v_st + 8 * vseg) * 2);
  const uint32_t voff2 = voff + static_cast<uint32_t>(a.v_st * 2);
  const int64_t kbytes = kv_end > 0 ? ((kv_end - 1) * a.k_st + kD) * 2 : 0;
  const int64_t vbytes = kv_end > 0 ? ((kv_end - 1) * a.v_st + kD) * 2 : 0;
  auto load_tile = [&](int t) {
    const int64_t kskip = int64_t(t) * kBN * a.k_st, vskip = int64_t(t) * kBN * a.v_st;
    const int64_t krem = kbytes - 2 * kskip, vrem = vbytes - 2 * vskip;
    const buf_t kr = make_buf(kp + kskip, krem > 0 ? static_cast<uint32_t>(krem) : 0u);
    const buf_t vr = make_buf(vp + vskip, vrem > 0 ? static_cast<uint32_t>(vrem) : 0u);
    kst[0] = buf_ld16(kr, koff);
    kst[1] = buf_ld16(kr, koff2);
    vst[0] = buf_ld16(vr, voff);
    vst[1] = buf_ld16(vr, voff2);
  };
  // K rows (htid >> 3) and (htid >> 3) + 32 of this thread, V^T rows 8 vseg + m
  const int ks_off = (htid >> 3) * kRow + (htid & 7) * 8;
  const int vs_off = 8 * vseg * kRow + vperm32(2 * vpair);
  auto store_tile = [&](auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    *reinterpret_cast<uint4 *>(&sK[part][buf][ks_off]) = kst[0];
    *reinterpret_cast<uint4 *>(&sK[part][buf][ks_off + 32 * kRow]) = kst[1];
    const uint32_t *v0 = reinterpret_cast<const uint32_t *>(&vst[0]);
    const uint32_t *v1 = reinterpret_cast<const uint32_t *>(&vst[1]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = (v0[i] & 0xffffu) | (v1[i] << 16);      // d = 8 vseg + 2i
      const uint32_t hi = (v0[i] >> 16) | (v1[i] & 0xffff0000u);  // d = 8 vseg + 2i + 1
      *reinterpret_cast<uint32_t *>(&sV[part][buf][vs_off + (2 * i) * kRow]) = lo;
      *reinterpret_cast<uint32_t *>(&sV[part][buf][vs_off + (2 * i + 1) * kRow]) = hi;
    }
  };

  float m_run = -INFINITY;  // in acc units, per column (both lane halves agree)
  float l_run = 0.f;        // this lane's share of the column's row sum of P
  f32x16 oacc[2];           // O^T rows d = 32 dt + 8 (r / 4) + 4 hh + r % 4, column lc
  oacc[0] = f32x16{};
  oacc[1] = f32x16{};
  const bf16x2v ones2 = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};

  // Prologue: tile and window of the first step in LDS, the second step's in flight.
  // Every load and store of the loop is unconditional (tiles and entries past the end
  // read zeros through the range checks), so the wait counts are path independent.
  load_tile(t_first);
  store_tile(std::integral_constant<int, 0>());
  store_window();
  load_tile(t_first + 1);
  __syncthreads();

  // One step: tile t_first + i from LDS buffer BUF (a constant, so every LDS address
  // is a fixed register plus an immediate).
  auto step = [&](int i, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const int n0 = (t_first + i) * kBN;
    // the new entries of the next step's windows, evaluated ahead of this step's work
    float bnew[RH];
#pragma unroll
    for (int hw = 0; hw < RH; ++hw) bnew[hw] = eval_bias(hw, n0 + 2 * kBN + dist0);
    if (i < t_count && n0 < wave_kv_end) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        // acc^T = bias + rho K Q^T over keys n0 + 32 kt + ..
        f32x16 acc;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
          for (int p4 = 0; p4 < 4; ++p4) acc[4 * q4 + p4] = bwr[32 * kt + 8 * q4 + p4];
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) {
          const bf16x8 kop = *reinterpret_cast<const bf16x8 *>(&sK[part][buf][(32 * kt + lc) * kRow + 16 * ds + 8 * hh]);
          acc = mma32(kop, qreg[ds], acc);
        }
        if (kmask && n0 + 32 * kt + 32 > Skv) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (n0 + 32 * kt + 8 * (r >> 2) + 4 * hh + (r & 3) >= Skv) acc[r] = -INFINITY;
        }
        float mx = acc[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, acc[r]);
        {
          const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
          mx = fmaxf(__uint_as_float(s32[0]), __uint_as_float(s32[1]));
        }
        // Lazy rescaling: the running max moves only when the sub-tile exceeds it by
        // more than 8 (log2 units of the logits), so p <= 2^8 and most sub-tiles skip
        // the rescale of the output accumulators.
        const bool grow = A * (mx - m_run) > 8.f || m_run == -INFINITY;
        const float m_new = grow ? mx : m_run;
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float resc = m_run == -INFINITY ? 0.f : fast_exp2(A * (m_run - m_use));
        const float nb = -A * m_use;
        if (__builtin_amdgcn_read_exec() & __ballot(grow)) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            oacc[0][r] *= resc;
            oacc[1][r] *= resc;
          }
          l_run *= resc;
        }
        m_run = m_new;
        // p = exp2(A (acc - m)); masked keys (acc = -inf) give exactly 0.  P^T k-steps
        // 2 kt and 2 kt + 1 are registers 0..7 and 8..15.
#pragma unroll
        for (int hk = 0; hk < 2; ++hk) {
          uint32_t pw[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pw[e] = pk2bf(fast_exp2(fmaf(acc[8 * hk + 2 * e], A, nb)), fast_exp2(fmaf(acc[8 * hk + 2 * e + 1], A, nb)));
            l_run = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, pw[e]), ones2, l_run, false);
          }
          const bf16x8 pb = __builtin_bit_cast(bf16x8, uint4{pw[0], pw[1], pw[2], pw[3]});
          const int ks = 2 * kt + hk;
#pragma unroll
          for (int dt = 0; dt < 2; ++dt) {
            const bf16x8 va = *reinterpret_cast<const bf16x8 *>(&sV[part][buf][(32 * dt + lc) * kRow + 16 * ks + 8 * hh]);
            oacc[dt] = mma32(va, pb, oacc[dt]);
          }
        }
      }
    }

    // The next step's windows and tile (fetched one step ago) into LDS, the tile after
    // into flight.  The window region is this wave's own (its reads above come first
    // in program order); the tile buffer was last read before the previous barrier.
#pragma unroll
    for (int hw = 0; hw < RH; ++hw) {
      bwin[hw][0] = bwin[hw][1];
      bwin[hw][1] = bnew[hw];
    }
    store_window();
    store_tile(std::integral_constant<int, buf ^ 1>());
    load_tile(t_first + i + 2);
    __syncthreads();
  };
  int i = 0;
  for (; i + 1 < nsteps; i += 2) {
    step(i, std::integral_constant<int, 0>());
    step(i + 1, std::integral_constant<int, 1>());
  }
  if (i < nsteps) step(i, std::integral_constant<int, 0>());

  // The column's row sum: this lane's keys plus those of lane l ^ 32.
  {
    const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
    l_run = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
  }

  // Merge: parts 1.. leave O^T (32 floats per lane) over the K / V buffers and (l, m)
  // in their window rows; part 0 combines them and writes the rows.
  float *mo = reinterpret_cast<float *>(&sKV[0][0][0][0]) + lane;  // [(part - 1) * 4 + w][32][64]
  if (part > 0) {
    float *dst = mo + ((part - 1) * 4 + w) * 32 * 64;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dst[r * 64] = oacc[0][r];
      dst[(16 + r) * 64] = oacc[1][r];
    }
    sB[wv][lane] = l_run;
    sB[wv][64 + lane] = m_run;
  }
  __syncthreads();
  if (part == 0 && q_valid) {
    float m = m_run;
#pragma unroll
    for (int p = 1; p < kParts; ++p) m = fmaxf(m, sB[4 * p + w][64 + lane]);
    float f[kParts];
    f[0] = m_run == -INFINITY ? 0.f : fast_exp2(A * (m_run - m));
    float l = l_run * f[0];
#pragma unroll
    for (int p = 1; p < kParts; ++p) {
      const float mp = sB[4 * p + w][64 + lane];
      f[p] = mp == -INFINITY ? 0.f : fast_exp2(A * (mp - m));
      l += sB[4 * p + w][lane] * f[p];
    }
    const float inv = 1.f / fmaxf(l, 1e-20f);
    bf16_t *op = static_cast<bf16_t *>(a.out) + batch * a.o_sb + head * a.o_sh + int64_t(tok0 + my_q) * a.o_st;
    // lane holds O[my_q][32 dt + 8 q4 + 4 hh + (0..3)]
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        float o[4];
#pragma unroll
        for (int p4 = 0; p4 < 4; ++p4) {
          const int r = 4 * q4 + p4;
          float x = oacc[dt][r] * f[0];
#pragma unroll
          for (int p = 1; p < kParts; ++p) x += mo[(((p - 1) * 4 + w) * 32 + 16 * dt + r) * 64] * f[p];
          o[p4] = x * inv;
        }
        *reinterpret_cast<uint2 *>(op + 32 * dt + 8 * q4 + 4 * hh) = uint2{pk2bf(o[0], o[1]), pk2bf(o[2], o[3])};
      }
    if (a.lse && hh == 0)
      a.lse[(static_cast<size_t>(batch) * a.H + head) * a.L + tok0 + my_q] = A * (m == -INFINITY ? 0.f : m) + fast_log2(l);
  }
}

// ------------------------------------------------------------------ decode

// GGD bias table per head in log2 units: entry j holds delta = j - kTabPad (delta =
// i_abs - key; the kTabPad leading entries, delta < 0, belong to masked keys and only
// keep every 32-byte read that contains a visible key inside the table):
// tab[h][j] = log2e * (-alpha_h (|-delta - mu_h| + eps)^beta_h).
constexpr int kTabPad = 8;
__global__ void __launch_bounds__(256) chord_bias_table_kernel(ChordArgs a, float *tab, int n) {
  const int h = blockIdx.y, j = blockIdx.x * 256 + threadIdx.x;
  if (j < n)
    tab[static_cast<size_t>(h) * n + j] =
        kLog2e * ggd_bias(static_cast<float>(kTabPad - j), a.alpha[h], a.beta[h], a.mu[h], a.eps);
}

// Sum over the 8 lanes of an aligned 8-lane group (DPP: quad swaps, then half-row mirror).
__device__ __forceinline__ float sum8(float x) {
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, false));  // row_half_mirror
  return x;
}


// 8 features of one K / V / q row kept packed as loaded: bf16 dots use v_dot2_f32_bf16
// on the packed pairs (the products are exact in fp32), fp32 rows take two loads.
template <typename T> struct Row8;
template <> struct Row8<bf16_t> {
  uint4 u;
  __device__ __forceinline__ void load(buf_t r, uint32_t off) { u = buf_ld16(r, off); }
  __device__ __forceinline__ void load(const bf16_t *p) { u = *reinterpret_cast<const uint4 *>(p); }
  __device__ __forceinline__ float dot(const Row8 &o, float acc) const {
    typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf2;
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, u.x), __builtin_bit_cast(bf2, o.u.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, u.y), __builtin_bit_cast(bf2, o.u.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, u.z), __builtin_bit_cast(bf2, o.u.z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, u.w), __builtin_bit_cast(bf2, o.u.w), acc, false);
    return acc;
  }
  __device__ __forceinline__ void unpack(float x[8]) const {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = __uint_as_float(w[e] << 16);
      x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
    }
  }
};
template <> struct Row8<float> {
  uint4 u, v;
  __device__ __forceinline__ void load(buf_t r, uint32_t off) { u = buf_ld16(r, off); v = buf_ld16(r, off + 16); }
  __device__ __forceinline__ void load(const float *p) {
    u = *reinterpret_cast<const uint4 *>(p);
    v = *reinterpret_cast<const uint4 *>(p + 4);
  }
  __device__ __forceinline__ float dot(const Row8 &o, float acc) const {
    float x[8], y[8];
    unpack(x);
    o.unpack(y);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf(x[e], y[e], acc);
    return acc;
  }
  __device__ __forceinline__ void unpack(float x[8]) const {
    x[0] = __uint_as_float(u.x); x[1] = __uint_as_float(u.y); x[2] = __uint_as_float(u.z); x[3] = __uint_as_float(u.w);
    x[4] = __uint_as_float(v.x); x[5] = __uint_as_float(v.y); x[6] = __uint_as_float(v.z); x[7] = __uint_as_float(v.w);
  }
};

template <> struct Row8<f16_t> {
  uint4 u;
  __device__ __forceinline__ void load(buf_t r, uint32_t off) { u = buf_ld16(r, off); }
  __device__ __forceinline__ void load(const f16_t *p) { u = *reinterpret_cast<const uint4 *>(p); }
  __device__ __forceinline__ float dot(const Row8 &o, float acc) const {
    float x[8], y[8];
    unpack(x);
    o.unpack(y);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf(x[e], y[e], acc);
    return acc;
  }
  __device__ __forceinline__ void unpack(float x[8]) const {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = static_cast<float>(__builtin_bit_cast(f16_t, static_cast<uint16_t>(w[e] & 0xffffu)));
      x[2 * e + 1] = static_cast<float>(__builtin_bit_cast(f16_t, static_cast<uint16_t>(w[e] >> 16)));
    }
  }
};

// Sum over the LPK lanes that share a key (LPK = D / 8 lanes of 8 features each).
template <int LPK>
__device__ __forceinline__ float sum_key(float x) {
  if constexpr (LPK == 8) {
    return sum8(x);
  } else {
#pragma unroll
    for (int off = 1; off < LPK; off <<= 1) x += __shfl_xor(x, off, 64);
    return x;
  }
}

constexpr int kDecKeys = 4;                 // keys per lane group per step

// Rows of a workgroup: global row gr = qc * R + r over the L * group (query,
// head) pairs of one kv head, query i = gr / group, head = kvh * group + gr % group.
// A key row of D features is held by LPK = D / 8 lanes (8 features each), so a wave
// has KG = 64 / LPK lane groups and takes KG * 4 consecutive keys per step: lane
// (ksub = lane / LPK, features 8 (lane % LPK) ..) owns keys n0 + 4 ksub + it, it < 4,
// whose 4 bias entries are one 16-byte read of the head's table.  The next step's
// K / V rows and bias entries are loaded before the current step is computed (two
// register stages), so a wave keeps a step of loads in flight.  Each lane group keeps
// its own running max / sum / output (merged at the end): the step has no cross-lane
// traffic besides the LPK-lane dot-product sums.  This kernel serves every dtype
// (fp32, bf16, fp16) and head dim (16, 32, 64, 128); bf16 at D = 64 has MFMA kernels.
template <typename T, int R, int D>
__global__ void __launch_bounds__(256) chord_decode_kernel(ChordArgs a, const float *tab, int tab_n) {
  constexpr int LPK = D / 8, KG = 64 / LPK, kDecStep = KG * kDecKeys;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int split = blockIdx.x, kvh = blockIdx.y;
  const int b = blockIdx.z / a.nqc, qc = blockIdx.z % a.nqc;
  const int group = a.H / a.Hkv;
  const int total_rows = a.L * group;
  const int dc = (lane % LPK) * 8;  // this lane's 8 feature columns
  const int ksub = lane / LPK;      // key group of this lane
  const T *qg = static_cast<const T *>(a.q);
  T *og = static_cast<T *>(a.out);

  const DecodeWindow win = decode_window(a);
  const int kv_len = win.S, q_start = win.q_start;
  const int per = ((kv_len + a.splits - 1) / a.splits + kBN - 1) / kBN * kBN;
  const int i_last = min(a.L - 1, (qc * R + R - 1) / group);
  const int k_lo = split * per;
  const int k_hi = min(min(kv_len, k_lo + per), q_start + i_last + 1);

  Row8<T> q[R];
  float c_qk[R], c_b[R];
  int qabs[R];
  buf_t tb[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int gr = qc * R + r;
    const bool ok = gr < total_rows;
    const int head = kvh * group + (ok ? gr % group : 0);
    const int i = ok ? gr / group : 0;
    q[r].load(qg + b * a.q_sb + head * a.q_sh + int64_t(i) * a.q_st + dc);
    const float mul = ok ? a.ssmax[head] * log_n_at(a, b, i, q_start) : 0.f;
    c_qk[r] = mul * a.scale * kLog2e;
    c_b[r] = mul;  // the table is in log2 units already
    qabs[r] = ok ? q_start + i : -1;
    tb[r] = make_buf(tab + static_cast<size_t>(head) * tab_n, static_cast<uint32_t>(tab_n) * 4u);
  }

  float m[R], l[R], acc[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY; l[r] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.f;
  }

  const T *kp = static_cast<const T *>(a.k) + b * a.k_sb + kvh * a.k_sh;
  const T *vp = static_cast<const T *>(a.v) + b * a.v_sb + kvh * a.v_sh;
  // rows past k_hi (the prefetch past the range) read as zeros
  const buf_t kbuf = make_buf(kp, k_hi > 0 ? static_cast<uint32_t>(((k_hi - 1) * a.k_st + D) * sizeof(T)) : 0u);
  const buf_t vbuf = make_buf(vp, k_hi > 0 ? static_cast<uint32_t>(((k_hi - 1) * a.v_st + D) * sizeof(T)) : 0u);

  struct Stage {
    Row8<T> k[kDecKeys], v[kDecKeys];
    uint4 bias[R];  // entries delta = qabs - kb - 3 .. qabs - kb (it = 3 .. 0)
  };
  auto load_stage = [&](int n0, Stage &st) {
    const int kb = n0 + kDecKeys * ksub;
#pragma unroll
    for (int it = 0; it < kDecKeys; ++it) {
      st.k[it].load(kbuf, static_cast<uint32_t>(((kb + it) * a.k_st + dc) * sizeof(T)));
      st.v[it].load(vbuf, static_cast<uint32_t>(((kb + it) * a.v_st + dc) * sizeof(T)));
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
      st.bias[r] = buf_ld16(tb[r], static_cast<uint32_t>(qabs[r] - kb - (kDecKeys - 1) + kTabPad) * 4u);
  };

  int n0 = k_lo + w * kDecStep;
  Stage cur;
  if (n0 < k_hi) load_stage(n0, cur);
  for (; n0 < k_hi; n0 += 4 * kDecStep) {
    Stage nxt;
    load_stage(n0 + 4 * kDecStep, nxt);
    // the next stage's loads stay ahead of this step's arithmetic
    __builtin_amdgcn_sched_barrier(0);
    const int kb = n0 + kDecKeys * ksub;
    float vf[kDecKeys][8];
#pragma unroll
    for (int it = 0; it < kDecKeys; ++it) cur.v[it].unpack(vf[it]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float bt[4] = {__uint_as_float(cur.bias[r].w), __uint_as_float(cur.bias[r].z),
                           __uint_as_float(cur.bias[r].y), __uint_as_float(cur.bias[r].x)};
      float sv[kDecKeys], mx = -INFINITY;
#pragma unroll
      for (int it = 0; it < kDecKeys; ++it) {
        const float d = sum_key<LPK>(cur.k[it].dot(q[r], 0.f));
        const int key = kb + it;
        const bool ok = key < k_hi && key <= qabs[r];
        sv[it] = ok ? fmaf(d, c_qk[r], c_b[r] * bt[it]) : -INFINITY;
        mx = fmaxf(mx, sv[it]);
      }
      const float m_new = fmaxf(m[r], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float resc = m[r] == -INFINITY ? 0.f : fast_exp2(m[r] - m_use);
      float ps = 0.f;
#pragma unroll
      for (int it = 0; it < kDecKeys; ++it) {
        sv[it] = sv[it] == -INFINITY ? 0.f : fast_exp2(sv[it] - m_use);
        ps += sv[it];
      }
      l[r] = l[r] * resc + ps;
      m[r] = m_new;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float x = acc[r][e] * resc;
#pragma unroll
        for (int it = 0; it < kDecKeys; ++it) x = fmaf(sv[it], vf[it][e], x);
        acc[r][e] = x;
      }
    }
    cur = nxt;
  }

  // Merge the KG key groups of the wave (lanes l, l ^ LPK, l ^ 2 LPK, ... share features).
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float M = m[r];
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    const float f = m[r] == -INFINITY ? 0.f : fast_exp2(m[r] - (M == -INFINITY ? 0.f : M));
    float lx = l[r] * f;
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) lx += __shfl_xor(lx, off, 64);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = acc[r][e] * f;
#pragma unroll
      for (int off = LPK; off < 64; off <<= 1) x += __shfl_xor(x, off, 64);
      acc[r][e] = x;
    }
    m[r] = M;
    l[r] = lx;
  }

  // Merge the 4 waves in LDS.
  __shared__ float sm[4][R], sl[4][R], sacc[4][R][D];
  if (lane < LPK) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) sacc[w][r][dc + e] = acc[r][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) { sm[w][r] = m[r]; sl[w][r] = l[r]; }
  }
  __syncthreads();
  for (int e = tid; e < R * D; e += 256) {
    const int r = e / D, d = e % D;
    const int gr = qc * R + r;
    if (gr >= total_rows) continue;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, sm[ww][r]);
    const float Mu = M == -INFINITY ? 0.f : M;
    float o = 0.f, Ls = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float f = fast_exp2(sm[ww][r] - Mu);
      o += sacc[ww][r][d] * f;
      Ls += sl[ww][r] * f;
    }
    if (!a.part) {
      const int head = kvh * group + gr % group, i = gr / group;
      st(og + b * a.o_sb + head * a.o_sh + int64_t(i) * a.o_st + d, o / fmaxf(Ls, 1e-20f));
      if (a.lse && d == 0) a.lse[(static_cast<size_t>(b) * a.H + head) * a.L + i] = M + fast_log2(Ls);
    } else {
      float *pp = a.part + ((((static_cast<size_t>(b) * a.Hkv + kvh) * a.splits + split) * total_rows + gr) * (D + 2));
      pp[d] = o;
      if (d == 0) { pp[D] = M; pp[D + 1] = Ls; }
    }
  }
}

// bf16 decode on MFMA (up to 16 (query, head) rows of one kv head per workgroup).
// Per wave step of 32 keys (two 16-key tiles):
//   S^T = K Q^T on v_mfma_f32_16x16x32_bf16 -- A = K (lane: key l % 16, features
//   16 g + {0..7} then + {8..15} for the two k-steps, g = l / 16: two adjacent 16-byte
//   loads covering each key row's 128-byte line), B = Q^T (lane: query row l % 16, the
//   same features).  The accumulator gives lane l the scores of row l % 16 for keys
//   4 g + i, so the softmax statistics of a row live in the 4 lanes l % 16 + 16 g.
//   O^T += V^T P^T -- B = P^T straight from the scores (slots 0..3: tile 0 keys 4 g + i,
//   slots 4..7: tile 1 keys 16 + 4 g + i), A = V^T with the same key slots, gathered
//   from the wave's V tile in LDS (V rows are loaded with 16-byte coalesced reads and
//   written row-major).  O^T's accumulator gives lane l features 16 ft + 4 g + i of
//   row l % 16, so no cross-lane sum is needed for O.
// The GGD bias of each (row, key) is evaluated in registers (one exp2 / log2 pair), so
// this kernel needs no bias table.  The next step's K / V loads are issued before the
// current step's arithmetic.
constexpr int kMfmaRows = 16;
constexpr int kVRow = 72;  // LDS V row stride (bf16): 144 bytes, conflict-free gathers

// The whole decode step of a Chord layer in one launch (motif_chord_decode_step): q, k
// and v come from the layer's projection rows, q and k RMSNormed here exactly as
// chord_prep_kernel does it; the workgroup whose split holds a new position appends
// its key / value row to the cache before any of its loads; the last workgroup of
// each (batch row, kv head) to finish merges the splits' partials (chord_merge_kernel's
// arithmetic), and the last of those advances the cursor.  `cnt` holds B * Hkv + 1
// arrival counters that are zero between launches (each launch leaves them zero).
struct StepArgs {
  const bf16_t *proj; int64_t p_sb, p_st;  // [B, L, ncols]
  int q_off, k_off, v_off;
  const bf16_t *qw, *kw;                    // RMSNorm weights [D]
  float neps;
  int *cnt;
};

// RMSNorm of 16 features per lane, the row's 64 features over lanes l, l ^ 16, l ^ 32,
// l ^ 48 (16 g .. 16 g + 15 on lane group g): T(x * rsqrt(mean(x^2) + eps)) * w.  The
// sum of squares is formed in chord_prep_kernel's order (an fma chain per 8-element
// piece, then the pieces added pairwise as its 8-lane butterfly adds them), so both
// kernels produce the same bits.
__device__ __forceinline__ void rms_norm16(uint4 &u0, uint4 &u1, const uint4 w0, const uint4 w1, float eps) {
  float x0[8], x1[8], wa[8], wb[8];
  const uint32_t a0[4] = {u0.x, u0.y, u0.z, u0.w}, a1[4] = {u1.x, u1.y, u1.z, u1.w};
  const uint32_t b0[4] = {w0.x, w0.y, w0.z, w0.w}, b1[4] = {w1.x, w1.y, w1.z, w1.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x0[2 * i] = __uint_as_float(a0[i] << 16); x0[2 * i + 1] = __uint_as_float(a0[i] & 0xffff0000u);
    x1[2 * i] = __uint_as_float(a1[i] << 16); x1[2 * i + 1] = __uint_as_float(a1[i] & 0xffff0000u);
    wa[2 * i] = __uint_as_float(b0[i] << 16); wa[2 * i + 1] = __uint_as_float(b0[i] & 0xffff0000u);
    wb[2 * i] = __uint_as_float(b1[i] << 16); wb[2 * i + 1] = __uint_as_float(b1[i] & 0xffff0000u);
  }
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    s0 = fmaf(x0[e], x0[e], s0);
    s1 = fmaf(x1[e], x1[e], s1);
  }
  float ss = s0 + s1;
  ss += __shfl_xor(ss, 16, 64);
  ss += __shfl_xor(ss, 32, 64);
  const float rs = rsqrtf(ss / kD + eps);
  uint32_t o0[4], o1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o0[i] = static_cast<uint32_t>(f32_to_bf16(bf16_to_f32(f32_to_bf16(x0[2 * i] * rs)) * wa[2 * i])) |
            (static_cast<uint32_t>(f32_to_bf16(bf16_to_f32(f32_to_bf16(x0[2 * i + 1] * rs)) * wa[2 * i + 1])) << 16);
    o1[i] = static_cast<uint32_t>(f32_to_bf16(bf16_to_f32(f32_to_bf16(x1[2 * i] * rs)) * wb[2 * i])) |
            (static_cast<uint32_t>(f32_to_bf16(bf16_to_f32(f32_to_bf16(x1[2 * i + 1] * rs)) * wb[2 * i + 1])) << 16);
  }
  u0 = uint4{o0[0], o0[1], o0[2], o0[3]};
  u1 = uint4{o1[0], o1[1], o1[2], o1[3]};
}

template <bool STEP>
__global__ void __launch_bounds__(256) chord_decode_mfma_kernel(ChordArgs a, StepArgs sa) {
  // wave index in an SGPR: the key loop below is then scalar (MFMAs must not sit
  // under a lane-mask branch, as they ignore EXEC)
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, g = lane >> 4;
  const int split = blockIdx.x, kvh = blockIdx.y;
  const int b = blockIdx.z / a.nqc, qc = blockIdx.z % a.nqc;
  const int group = a.H / a.Hkv;
  const int total_rows = a.L * group;
  const bf16_t *qg = static_cast<const bf16_t *>(a.q);

  // this lane's query row (column of the B / C operands)
  const int gr = qc * kMfmaRows + c16;
  const bool row_ok = gr < total_rows;
  const int head = kvh * group + (row_ok ? gr % group : 0);
  const int qi = row_ok ? gr / group : 0;
  bf16x8 qb[2];
  if constexpr (STEP) {
    // the raw q row of the projection, normalised here (every lane joins the sums)
    const bf16_t *qr = sa.proj + b * sa.p_sb + int64_t(qi) * sa.p_st + sa.q_off + head * kD + 16 * g;
    uint4 u0 = *reinterpret_cast<const uint4 *>(qr), u1 = *reinterpret_cast<const uint4 *>(qr + 8);
    rms_norm16(u0, u1, *reinterpret_cast<const uint4 *>(sa.qw + 16 * g),
               *reinterpret_cast<const uint4 *>(sa.qw + 16 * g + 8), sa.neps);
    const uint4 z{0, 0, 0, 0};
    qb[0] = __builtin_bit_cast(bf16x8, row_ok ? u0 : z);
    qb[1] = __builtin_bit_cast(bf16x8, row_ok ? u1 : z);
  } else {
    const bf16_t *qr = qg + b * a.q_sb + head * a.q_sh + int64_t(qi) * a.q_st + 16 * g;
    const uint4 u0 = *reinterpret_cast<const uint4 *>(qr), u1 = *reinterpret_cast<const uint4 *>(qr + 8);
    const uint4 z{0, 0, 0, 0};
    qb[0] = __builtin_bit_cast(bf16x8, row_ok ? u0 : z);
    qb[1] = __builtin_bit_cast(bf16x8, row_ok ? u1 : z);
  }
  const DecodeWindow win = decode_window(a);
  const int q_start = win.q_start;
  const float mul = row_ok ? a.ssmax[head] * log_n_at(a, b, qi, q_start) : 0.f;
  const float c_qk = mul * a.scale * kLog2e, c_b = mul;
  const int qabs = row_ok ? q_start + qi : -1;
  // GGD bias of (row, key) evaluated in registers, log2 units (the same function the
  // bias table holds): no table pass, no bias loads
  const float g_alpha = a.alpha[head] * kLog2e, g_beta = a.beta[head], g_mu = a.mu[head];

  const int kv_len = win.S;
  const int per = ((kv_len + a.splits - 1) / a.splits + kBN - 1) / kBN * kBN;
  const int i_last = min(a.L - 1, (qc * kMfmaRows + kMfmaRows - 1) / group);
  const int k_lo = split * per;
  const int k_hi = min(min(kv_len, k_lo + per), q_start + i_last + 1);

  const bf16_t *kp = static_cast<const bf16_t *>(a.k) + b * a.k_sb + kvh * a.k_sh;
  const bf16_t *vp = static_cast<const bf16_t *>(a.v) + b * a.v_sb + kvh * a.v_sh;
  // rows past k_hi read as zeros
  const buf_t kbuf = make_buf(kp, k_hi > 0 ? static_cast<uint32_t>(((k_hi - 1) * a.k_st + kD) * 2) : 0u);
  const buf_t vbuf = make_buf(vp, k_hi > 0 ? static_cast<uint32_t>(((k_hi - 1) * a.v_st + kD) * 2) : 0u);

  __shared__ __attribute__((aligned(16))) bf16_t sV[4][32 * kVRow];
  // per wave: the step's 32 K rows (128 bytes each, 16-byte chunks XOR-swizzled by row),
  // filled by buffer-to-LDS loads of whole rows, 8 rows per instruction (the operand
  // layout would read 16 rows x 64 bytes per instruction: half of each line)
  __shared__ __attribute__((aligned(16))) bf16_t sKs[4][32 * 64];
  bf16_t *myV = sV[w], *myK = sKs[w];

  struct Stage {
    uint4 v[4];      // V rows 8 r + lane / 8, features 8 (lane % 8)
  };
  // K: instruction i, lane l: row 8 i + l / 8, physical chunk l % 8 = logical chunk
  // (features 8 c .. 8 c + 7) c = (l % 8) ^ (row % 8)
  uint32_t kdo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 8 * i + (lane >> 3);
    kdo[i] = static_cast<uint32_t>((r * a.k_st + 8 * ((lane & 7) ^ (r & 7))) * 2);
  }
  auto load_stage = [&](int n0, Stage &st) {
    const uint32_t ks = static_cast<uint32_t>(n0 * a.k_st * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) buf_ld16_lds<2>(kbuf, myK + 8 * i * 64, kdo[i], ks);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      st.v[r] = buf_ld16_nt(vbuf, static_cast<uint32_t>(((n0 + 8 * r + (lane >> 3)) * a.v_st + 8 * (lane & 7)) * 2));
  };

  float m = -INFINITY, lsum = 0.f;
  f32x4 o[4];
#pragma unroll
  for (int ft = 0; ft < 4; ++ft) o[ft] = f32x4{0.f, 0.f, 0.f, 0.f};

  if constexpr (STEP) {
    // The new positions [q_start, q_start + L) this split holds: wave 0 appends their key
    // (RMSNormed, chord_prep_kernel's order: an fma chain per lane, then the 8-lane
    // butterfly) and value rows, lane = 32 (value?) + 8 t + piece, before any load of
    // this workgroup reads them; no other workgroup reads these positions.
    if (w == 0) {
      const int is_v = lane >> 5, t = (lane >> 3) & 3, piece = lane & 7;
      const int pos = q_start + t;
      const bool mine = t < a.L && pos >= k_lo && pos < k_lo + per && pos < a.S;
      const bf16_t *src = sa.proj + b * sa.p_sb + int64_t(min(t, a.L - 1)) * sa.p_st + (is_v ? sa.v_off : sa.k_off) +
                          kvh * kD + 8 * piece;
      const uint4 u = *reinterpret_cast<const uint4 *>(src);
      const uint4 wr = *reinterpret_cast<const uint4 *>(sa.kw + 8 * piece);
      float x[8], wk[8];
      const uint32_t ua[4] = {u.x, u.y, u.z, u.w}, wa[4] = {wr.x, wr.y, wr.z, wr.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[2 * i] = __uint_as_float(ua[i] << 16); x[2 * i + 1] = __uint_as_float(ua[i] & 0xffff0000u);
        wk[2 * i] = __uint_as_float(wa[i] << 16); wk[2 * i + 1] = __uint_as_float(wa[i] & 0xffff0000u);
      }
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
#pragma unroll
      for (int off = 1; off < 8; off <<= 1) ss += __shfl_xor(ss, off, 64);
      uint4 o = u;
      if (!is_v) {
        const float rs = rsqrtf(ss / kD + sa.neps);
        uint32_t ow[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          ow[i] = static_cast<uint32_t>(f32_to_bf16(bf16_to_f32(f32_to_bf16(x[2 * i] * rs)) * wk[2 * i])) |
                  (static_cast<uint32_t>(f32_to_bf16(bf16_to_f32(f32_to_bf16(x[2 * i + 1] * rs)) * wk[2 * i + 1]))
                   << 16);
        o = uint4{ow[0], ow[1], ow[2], ow[3]};
      }
      if (mine) {
        bf16_t *dst = is_v ? static_cast<bf16_t *>(const_cast<void *>(a.v)) + b * a.v_sb + kvh * a.v_sh + int64_t(pos) * a.v_st
                           : static_cast<bf16_t *>(const_cast<void *>(a.k)) + b * a.k_sb + kvh * a.k_sh + int64_t(pos) * a.k_st;
        *reinterpret_cast<uint4 *>(dst + 8 * piece) = o;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }

  int n0 = k_lo + w * 32;
  Stage cur;
  if (n0 < k_hi) load_stage(n0, cur);
  for (; n0 < k_hi; n0 += 4 * 32) {
    // this step's K rows have landed in LDS (and its V rows in registers): operands out,
    // then the buffer takes the next step's rows
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    uint4 kop[2][2];  // [tile][piece]: key 16 t + c16, features 16 g + 8 piece .. + 7
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int pc = 0; pc < 2; ++pc)
        kop[t][pc] = *reinterpret_cast<const uint4 *>(myK + (16 * t + c16) * 64 + 8 * ((2 * g + pc) ^ (c16 & 7)));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    Stage nxt;
    load_stage(n0 + 4 * 32, nxt);
    __builtin_amdgcn_sched_barrier(0);
    // V rows of this step into the wave's LDS tile (row-major, padded rows)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *reinterpret_cast<uint4 *>(myV + (8 * r + (lane >> 3)) * kVRow + 8 * (lane & 7)) = cur.v[r];
    // scores
    float sc[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
      sacc = mma16(__builtin_bit_cast(bf16x8, kop[t][0]), qb[0], sacc);
      sacc = mma16(__builtin_bit_cast(bf16x8, kop[t][1]), qb[1], sacc);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = n0 + 16 * t + 4 * g + i;
        const bool ok = key < k_hi && key <= qabs;
        const float bt = ggd_bias(static_cast<float>(key - qabs), g_alpha, g_beta, g_mu, a.eps);
        sc[t][i] = ok ? fmaf(sacc[i], c_qk, c_b * bt) : -INFINITY;
      }
    }
    // row max over the 32 keys (4 lanes share a row)
    float mx = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                     fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float resc = m == -INFINITY ? 0.f : fast_exp2(m - m_use);
    m = m_new;
    float ps = 0.f;
    bf16_t pb[8];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pv = sc[t][i] == -INFINITY ? 0.f : fast_exp2(sc[t][i] - m_use);
        ps += pv;
        pb[4 * t + i] = f32_to_bf16(pv);
      }
    lsum = lsum * resc + ps;
    bf16x8 pB;
    {
      uint4 u;
      u.x = pb[0] | (static_cast<uint32_t>(pb[1]) << 16);
      u.y = pb[2] | (static_cast<uint32_t>(pb[3]) << 16);
      u.z = pb[4] | (static_cast<uint32_t>(pb[5]) << 16);
      u.w = pb[6] | (static_cast<uint32_t>(pb[7]) << 16);
      pB = __builtin_bit_cast(bf16x8, u);
    }
    // O^T += V^T P^T per 16-feature tile
#pragma unroll
    for (int ft = 0; ft < 4; ++ft) {
      const int e = 16 * ft + c16;
      uint32_t wv[4];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const bf16_t *col = myV + (16 * h + 4 * g) * kVRow + e;
        wv[2 * h] = col[0] | (static_cast<uint32_t>(col[kVRow]) << 16);
        wv[2 * h + 1] = col[2 * kVRow] | (static_cast<uint32_t>(col[3 * kVRow]) << 16);
      }
      const bf16x8 vA = __builtin_bit_cast(bf16x8, uint4{wv[0], wv[1], wv[2], wv[3]});
      o[ft] *= resc;
      o[ft] = mma16(vA, pB, o[ft]);
    }
    cur = nxt;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last (empty) K fill has landed

  // row sum over the 4 lanes of a row
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);

  // merge the 4 waves through LDS (reusing the V tiles' space is not needed: small)
  __shared__ float sm[4][kMfmaRows], sl[4][kMfmaRows], so[4][kMfmaRows][kD + 1];
  if (g == 0) { sm[w][c16] = m; sl[w][c16] = lsum; }
#pragma unroll
  for (int ft = 0; ft < 4; ++ft)
#pragma unroll
    for (int i = 0; i < 4; ++i) so[w][c16][16 * ft + 4 * g + i] = o[ft][i];
  __syncthreads();
  for (int e = tid; e < kMfmaRows * kD; e += 256) {
    const int r = e / kD, d = e % kD;
    const int grr = qc * kMfmaRows + r;
    if (grr >= total_rows) continue;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, sm[ww][r]);
    const float Mu = M == -INFINITY ? 0.f : M;
    float ov = 0.f, Ls = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float f = fast_exp2(sm[ww][r] - Mu);
      ov += so[ww][r][d] * f;
      Ls += sl[ww][r] * f;
    }
    if (!a.part) {
      const int hh = kvh * group + grr % group, ii = grr / group;
      st(static_cast<bf16_t *>(a.out) + b * a.o_sb + hh * a.o_sh + int64_t(ii) * a.o_st + d, ov / fmaxf(Ls, 1e-20f));
      if (a.lse && d == 0) a.lse[(static_cast<size_t>(b) * a.H + hh) * a.L + ii] = M + fast_log2(Ls);
    } else {
      float *pp = a.part + ((((static_cast<size_t>(b) * a.Hkv + kvh) * a.splits + split) * total_rows + grr) * (kD + 2));
      if constexpr (STEP) {
        // device-coherent stores (through to memory): the merging workgroup may run on
        // another XCD, and a device-wide release fence would write back a whole L2
        __hip_atomic_store(&pp[d], ov, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == 0) {
          __hip_atomic_store(&pp[kD], M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(&pp[kD + 1], Ls, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else {
        pp[d] = ov;
        if (d == 0) { pp[kD] = M; pp[kD + 1] = Ls; }
      }
    }
  }
  if constexpr (STEP) {
    // Arrival of this split once every thread's partial stores have completed; the
    // last split of the (batch row, kv head) merges, as chord_merge_kernel does, row by
    // row, reading the partials with device-coherent loads.
    __shared__ int s_last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int slot = b * a.Hkv + kvh;  // one row chunk per (batch row, kv head) on this path
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(&sa.cnt[slot], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.splits - 1;
    __syncthreads();
    if (!s_last) return;
    auto ldp = [](const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    // this (batch row, kv head)'s partials [splits][rows][D + 2] are one block: staged
    // into LDS with every load in flight together when they fit (one memory round trip)
    // (over the K tiles' LDS, dead since the loop: splits x rows x 66 floats at the
    // model's shape is 1056 of its 4096)
    constexpr int kMergeLds = static_cast<int>(sizeof(sKs) / sizeof(float));
    float *s_part = reinterpret_cast<float *>(&sKs[0][0]);
    const int nfl = a.splits * total_rows * (kD + 2);
    const float *blk = a.part + (static_cast<size_t>(b) * a.Hkv + kvh) * a.splits * total_rows * (kD + 2);
    const bool staged = nfl <= kMergeLds;
    if (staged) {
      float tmp[kMergeLds / 256];
#pragma unroll
      for (int j = 0; j < kMergeLds / 256; ++j) {
        const int i = j * 256 + tid;
        tmp[j] = i < nfl ? ldp(blk + i) : 0.f;
      }
#pragma unroll
      for (int j = 0; j < kMergeLds / 256; ++j) {
        const int i = j * 256 + tid;
        if (i < nfl) s_part[i] = tmp[j];
      }
      __syncthreads();
    }
    auto part_at = [&](int i) { return staged ? s_part[i] : ldp(blk + i); };
    const int sstride = total_rows * (kD + 2);
    for (int e = tid; e < total_rows * kD; e += 256) {
      const int r = e / kD, d = e % kD;
      const int pr = r * (kD + 2);
      float M = -INFINITY;
      for (int sp = 0; sp < a.splits; ++sp) M = fmaxf(M, part_at(sp * sstride + pr + kD));
      const float Mu = M == -INFINITY ? 0.f : M;
      float o = 0.f, Ls = 0.f;
      for (int sp = 0; sp < a.splits; ++sp) {
        const float f = fast_exp2(part_at(sp * sstride + pr + kD) - Mu);
        o += part_at(sp * sstride + pr + d) * f;
        Ls += part_at(sp * sstride + pr + kD + 1) * f;
      }
      const int hh = kvh * group + r % group, ii = r / group;
      st(static_cast<bf16_t *>(a.out) + b * a.o_sb + hh * a.o_sh + int64_t(ii) * a.o_st + d, o / fmaxf(Ls, 1e-20f));
    }
    if (tid == 0) {
      __hip_atomic_store(&sa.cnt[slot], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // every workgroup has read the cursor before it arrived: the last (batch row, kv
      // head) to finish advances it
      const int all = a.B * a.Hkv;
      if (__hip_atomic_fetch_add(&sa.cnt[all], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == all - 1) {
        __hip_atomic_store(&sa.cnt[all], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *a.len_dev = min(*a.len_dev + a.L, a.S);
      }
    }
  }
}

template <typename T, int D = kD>
__global__ void __launch_bounds__(128) chord_merge_kernel(ChordArgs a) {
  const int gr = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, d = threadIdx.x;
  const int group = a.H / a.Hkv;
  const int total_rows = a.L * group;
  const float *pp = a.part + (((static_cast<size_t>(b) * a.Hkv + kvh) * a.splits) * total_rows + gr) * (D + 2);
  const size_t sstride = static_cast<size_t>(total_rows) * (D + 2);
  float M = -INFINITY;
  for (int s = 0; s < a.splits; ++s) M = fmaxf(M, pp[s * sstride + D]);
  const float Mu = M == -INFINITY ? 0.f : M;
  float o = 0.f, Ls = 0.f;
  for (int s = 0; s < a.splits; ++s) {
    const float f = fast_exp2(pp[s * sstride + D] - Mu);
    o += pp[s * sstride + d] * f;
    Ls += pp[s * sstride + D + 1] * f;
  }
  const int head = kvh * group + gr % group, i = gr / group;
  st(static_cast<T *>(a.out) + b * a.o_sb + head * a.o_sh + int64_t(i) * a.o_st + d, o / fmaxf(Ls, 1e-20f));
  if (a.lse && d == 0) a.lse[(static_cast<size_t>(b) * a.H + head) * a.L + i] = M + fast_log2(Ls);
  // the decode kernel (previous launch) has read the cursor; this kernel never does,
  // so one thread may advance it
  if (a.len_dev && (gr | kvh | b | d) == 0) *a.len_dev = min(*a.len_dev + a.L, a.S);
}

// ------------------------------------------------------------------ planning
static int device_cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  return n;
}

constexpr int kDecodeMaxRows = 8;

// Short query blocks over a long cache take the split-K vector kernel.
static bool use_decode(int H, int Hkv, int L, bool packed) {
  return !packed && (H / Hkv) * L <= kDecodeMaxRows;
}

static int decode_splits(int B, int Hkv, int S) {
  const int kv_len = std::max(1, S);
  const int base = std::max(1, B * Hkv);
  // ~3 workgroups per CU (B=64, Hkv=3, S=4097: 3 splits 41.2 us, 4 splits 38.6 us,
  // 6 splits 39.8 us, 11 splits 42.7 us)
  int want = (3 * device_cu_count() + base - 1) / base;
  want = std::min(want, (kv_len + 4 * kBN - 1) / (4 * kBN));  // >= one 64-key tile per wave
  return std::max(1, std::min(want, 32));
}

template <typename T, int D>
static void launch_decode_d(const ChordArgs &a, int R, const float *tab, int tab_n, hipStream_t s) {
  const dim3 grid(a.splits, a.Hkv, a.B * a.nqc), block(256);
  if (R <= 1) chord_decode_kernel<T, 1, D><<<grid, block, 0, s>>>(a, tab, tab_n);
  else if (R <= 2) chord_decode_kernel<T, 2, D><<<grid, block, 0, s>>>(a, tab, tab_n);
  else if (R <= 4) chord_decode_kernel<T, 4, D><<<grid, block, 0, s>>>(a, tab, tab_n);
  else chord_decode_kernel<T, 8, D><<<grid, block, 0, s>>>(a, tab, tab_n);
}

// The vector kernel and (with splits) its merge, for head dim D in {16, 32, 64, 128}.
template <typename T>
static int launch_vector(const ChordArgs &a, int R, int D, const float *tab, int tab_n, hipStream_t s) {
  switch (D) {
    case 16: launch_decode_d<T, 16>(a, R, tab, tab_n, s); break;
    case 32: launch_decode_d<T, 32>(a, R, tab, tab_n, s); break;
    case 64: launch_decode_d<T, 64>(a, R, tab, tab_n, s); break;
    default: launch_decode_d<T, 128>(a, R, tab, tab_n, s); break;
  }
  int rc = check_launch("chord_decode_kernel");
  if (rc || !a.part) return rc;  // partials (split keys, or the cursor decode): merge them
  const dim3 grid((a.H / a.Hkv) * a.L, a.Hkv, a.B);
  switch (D) {
    case 16: chord_merge_kernel<T, 16><<<grid, dim3(16), 0, s>>>(a); break;
    case 32: chord_merge_kernel<T, 32><<<grid, dim3(32), 0, s>>>(a); break;
    case 64: chord_merge_kernel<T, 64><<<grid, dim3(64), 0, s>>>(a); break;
    default: chord_merge_kernel<T, 128><<<grid, dim3(128), 0, s>>>(a); break;
  }
  return check_launch("chord_merge_kernel");
}

static int launch_vector_dt(int dtype, const ChordArgs &a, int R, int D, const float *tab, int tab_n, hipStream_t s) {
  if (dtype == MOTIF_BF16) return launch_vector<bf16_t>(a, R, D, tab, tab_n, s);
  if (dtype == MOTIF_F16) return launch_vector<f16_t>(a, R, D, tab, tab_n, s);
  return launch_vector<float>(a, R, D, tab, tab_n, s);
}

static bool head_dim_ok(int D) { return D == 16 || D == 32 || D == 64 || D == 128; }
// bf16 at the model's head dim takes the MFMA kernels; everything else the vector kernel
static bool mfma_path(int dtype, int D) { return dtype == MOTIF_BF16 && D == kD; }

// Workspace of the decode / fp32 paths: the bias table [H][S + 8] fp32 (read by the
// fp32 vector kernel; the bf16 MFMA kernel evaluates the bias in registers), then the
// split partials [B][Hkv][splits][rows][D + 2] fp32.
static int table_len(int S) { return std::max(S, 1) + kTabPad; }
static size_t table_bytes(int H, int S) {
  return (static_cast<size_t>(H) * table_len(S) * sizeof(float) + 255) / 256 * 256;
}


}  // namespace motif

using namespace motif;

extern "C" size_t motif_chord_workspace_bytes(int B, int H, int Hkv, int L, int S, int D, int *splits) {
  int sp = 1;
  if (B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0 && L > 0 && use_decode(H, Hkv, L, false))
    sp = decode_splits(B, Hkv, S);
  if (splits) *splits = sp;
  if (B <= 0 || H <= 0 || Hkv <= 0 || L <= 0) return 0;
  // the distance table of the vector kernel (decode shapes and fp32 / fp16 / other head
  // dims); the bf16 prefill kernel evaluates its bias in registers and needs none
  size_t n = table_bytes(H, S);
  if (sp > 1) n += static_cast<size_t>(B) * Hkv * sp * (static_cast<size_t>(H / Hkv) * L) * (D + 2) * sizeof(float);
  return n;
}

extern "C" int motif_chord_fwd(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    const float *alpha, const float *beta, const float *mu, const float *ssmax,
    const float *log_n, int64_t ln_sb, int64_t ln_st,
    void *out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    float *lse,
    int B, int H, int Hkv, int L, int S, int D,
    int q_start, float scale, float eps,
    const int32_t *cu_seqlens, int nseq, int max_seqlen,
    void *workspace, size_t workspace_bytes,
    int dtype, void *stream) {
  if (B < 0 || H <= 0 || Hkv <= 0 || L < 0 || S < 0 || q_start < 0)
    return set_error(MOTIF_ERR_INVALID, "chord_fwd: bad size or negative q_start");
  if (H % Hkv != 0) return set_error(MOTIF_ERR_INVALID, "chord_fwd: H must be a multiple of Hkv");
  if (!head_dim_ok(D)) return set_error(MOTIF_ERR_UNSUPPORTED, "chord_fwd: head_dim must be 16, 32, 64 or 128");
  if (dtype != MOTIF_BF16 && dtype != MOTIF_F32 && dtype != MOTIF_F16)
    return set_error(MOTIF_ERR_UNSUPPORTED, "chord_fwd: dtype must be bf16, fp16 or fp32");
  const bool packed = cu_seqlens != nullptr;
  if (packed && (B != 1 || nseq <= 0 || L != S))
    return set_error(MOTIF_ERR_INVALID, "chord_fwd: packed sequences need B == 1, nseq > 0 and L == S");
  if (packed && !mfma_path(dtype, D))
    return set_error(MOTIF_ERR_UNSUPPORTED, "chord_fwd: packed sequences are implemented for bf16, head_dim 64");
  if (!packed && nseq != B) return set_error(MOTIF_ERR_INVALID, "chord_fwd: nseq must equal B");
  if (B == 0 || L == 0) return MOTIF_OK;
  if (!q || !k || !v || !alpha || !beta || !mu || !ssmax || !log_n || !out)
    return set_error(MOTIF_ERR_INVALID, "chord_fwd: NULL pointer");
  const int64_t vec = dtype == MOTIF_F32 ? 4 : 8;  // elements per 16 bytes
  if (((q_st | k_st | v_st | o_st | q_sh | k_sh | v_sh | o_sh | q_sb | k_sb | v_sb | o_sb) % vec) != 0 ||
      ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
        reinterpret_cast<uintptr_t>(out)) & 15) != 0)
    return set_error(MOTIF_ERR_UNSUPPORTED, "chord_fwd: q/k/v/out need 16-byte aligned rows");

  ChordArgs a;
  a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.k = k; a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v = v; a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.alpha = alpha; a.beta = beta; a.mu = mu; a.ssmax = ssmax;
  a.log_n = log_n; a.ln_sb = ln_sb; a.ln_st = ln_st;
  a.out = out; a.o_sb = o_sb; a.o_sh = o_sh; a.o_st = o_st;
  a.lse = lse;
  a.B = B; a.H = H; a.Hkv = Hkv; a.L = L; a.S = S; a.q_start = q_start;
  a.scale = scale; a.eps = eps;
  a.cu = cu_seqlens;
  a.part = nullptr; a.splits = 1; a.nqc = 1;
  a.len_dev = nullptr; a.log_tab = nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int group = H / Hkv;
  const int rows = group * L;

  if (!mfma_path(dtype, D) || use_decode(H, Hkv, L, packed)) {
    if (S == 0) return set_error(MOTIF_ERR_INVALID, "chord_fwd: empty key cache");
    const bool mfma = mfma_path(dtype, D);  // bf16 decode shapes at D = 64: the MFMA kernel
    int R = 8;
    if (rows <= 8) {
      R = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8;
      a.splits = decode_splits(B, Hkv, S);
    }
    if (mfma) R = kMfmaRows;
    a.nqc = (rows + R - 1) / R;
    const size_t tb = table_bytes(H, S);
    const size_t need = tb + (a.splits > 1 ? static_cast<size_t>(B) * Hkv * a.splits * rows * (D + 2) * sizeof(float) : 0);
    if (!workspace || workspace_bytes < need)
      return set_error(MOTIF_ERR_INVALID, "chord_fwd: workspace too small (need " + std::to_string(need) + " bytes)");
    float *tab = static_cast<float *>(workspace);
    if (a.splits > 1) a.part = reinterpret_cast<float *>(static_cast<char *>(workspace) + tb);
    const int tn = table_len(S);
    int rc = MOTIF_OK;
    if (!mfma) {  // the vector kernel reads the bias from a per-head table
      chord_bias_table_kernel<<<dim3((tn + 255) / 256, H), dim3(256), 0, s>>>(a, tab, tn);
      rc = check_launch("chord_bias_table_kernel");
      if (rc) return rc;
    }
    if (!mfma) return launch_vector_dt(dtype, a, R, D, tab, tn, s);
    chord_decode_mfma_kernel<false><<<dim3(a.splits, Hkv, B * a.nqc), dim3(256), 0, s>>>(a, StepArgs{});
    rc = check_launch("chord_decode_kernel");
    if (rc || a.splits == 1) return rc;
    chord_merge_kernel<bf16_t><<<dim3(rows, Hkv, B), dim3(64), 0, s>>>(a);
    return check_launch("chord_merge_kernel");
  }

  const int hpw = (group % 4 == 0) ? 4 : (group % 2 == 0) ? 2 : 1;
  // queries per workgroup: 4 waves x 32 columns per half, the columns being 16 queries
  // of two heads (hpw >= 2) or 32 queries of one head
  const int qw = hpw == 4 ? 32 : hpw == 2 ? 64 : 128;
  const int maxlen = packed ? max_seqlen : L;
  if (maxlen <= 0) return MOTIF_OK;
  if (std::max<int64_t>(S, int64_t(q_start) + L) > (int64_t(1) << 28))
    return set_error(MOTIF_ERR_UNSUPPORTED, "chord_fwd: sequence too long");
  const int nqbg = (maxlen + qw - 1) / qw;
  dim3 grid(H / hpw, nqbg, packed ? nseq : B), block(256 * kParts);
  if (hpw == 4) chord_fwd_kernel<4><<<grid, block, 0, s>>>(a);
  else if (hpw == 2) chord_fwd_kernel<2><<<grid, block, 0, s>>>(a);
  else chord_fwd_kernel<1><<<grid, block, 0, s>>>(a);
  return check_launch("chord_fwd_kernel");
}

// ------------------------------------------------------------------ decode over a cursor

namespace motif {

// Workspace of motif_chord_decode: the fp32 path's bias table sized for the capacity,
// then the split partials (always present: the merge pass advances the cursor).
static size_t decode_ws_bytes(int B, int H, int Hkv, int L, int capacity, int D, int splits, bool fp32) {
  const size_t tb = fp32 ? table_bytes(H, capacity) : 0;
  return tb + static_cast<size_t>(B) * Hkv * splits * (static_cast<size_t>(H / Hkv) * L) * (D + 2) * sizeof(float);
}

}  // namespace motif

extern "C" size_t motif_chord_decode_workspace_bytes(int B, int H, int Hkv, int L, int capacity, int D, int dtype,
                                                     int *splits) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || L <= 0 || capacity < L) {
    if (splits) *splits = 1;
    return 0;
  }
  const int sp = decode_splits(B, Hkv, capacity);
  if (splits) *splits = sp;
  return decode_ws_bytes(B, H, Hkv, L, capacity, D, sp, !mfma_path(dtype, D));
}

int motif::chord_decode_run(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int *length_dev, int capacity,
    const float *alpha, const float *beta, const float *mu, const float *ssmax,
    const float *log_n, int64_t ln_sb, int64_t ln_st, const float *log_table, int log_table_len,
    void *out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int Hkv, int L, int D, float scale, float eps,
    void *workspace, size_t workspace_bytes, int dtype, void *stream) {
  if (B < 0 || H <= 0 || Hkv <= 0 || L < 0 || H % Hkv)
    return set_error(MOTIF_ERR_INVALID, "chord_decode: bad size");
  if (!head_dim_ok(D)) return set_error(MOTIF_ERR_UNSUPPORTED, "chord_decode: head_dim must be 16, 32, 64 or 128");
  if (dtype != MOTIF_BF16 && dtype != MOTIF_F32 && dtype != MOTIF_F16)
    return set_error(MOTIF_ERR_UNSUPPORTED, "chord_decode: dtype must be bf16, fp16 or fp32");
  if (B == 0 || L == 0) return MOTIF_OK;
  if (capacity < L) return set_error(MOTIF_ERR_INVALID, "chord_decode: capacity below the query count");
  if (!q || !k_cache || !v_cache || !length_dev || !alpha || !beta || !mu || !ssmax || !out)
    return set_error(MOTIF_ERR_INVALID, "chord_decode: NULL pointer");
  if (!log_n && (!log_table || log_table_len < capacity))
    return set_error(MOTIF_ERR_INVALID, "chord_decode: log_n is NULL and the log table is shorter than the capacity");
  const int64_t vec = dtype == MOTIF_F32 ? 4 : 8;
  if (((q_st | k_st | v_st | o_st | q_sh | k_sh | v_sh | o_sh | q_sb | k_sb | v_sb | o_sb) % vec) != 0 ||
      ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) |
        reinterpret_cast<uintptr_t>(v_cache) | reinterpret_cast<uintptr_t>(out)) & 15) != 0)
    return set_error(MOTIF_ERR_UNSUPPORTED, "chord_decode: q/k/v/out need 16-byte aligned rows");
  const bool fp32 = !mfma_path(dtype, D);  // the vector kernel (with its bias table)
  const int splits = decode_splits(B, Hkv, capacity);
  const size_t need = decode_ws_bytes(B, H, Hkv, L, capacity, D, splits, fp32);
  if (!workspace || workspace_bytes < need)
    return set_error(MOTIF_ERR_INVALID, "chord_decode: workspace too small (need " + std::to_string(need) + " bytes)");

  ChordArgs a;
  a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.k = k_cache; a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v = v_cache; a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.alpha = alpha; a.beta = beta; a.mu = mu; a.ssmax = ssmax;
  a.log_n = log_n; a.ln_sb = ln_sb; a.ln_st = ln_st;
  a.out = out; a.o_sb = o_sb; a.o_sh = o_sh; a.o_st = o_st;
  a.lse = nullptr;
  a.B = B; a.H = H; a.Hkv = Hkv; a.L = L; a.S = capacity; a.q_start = 0;
  a.scale = scale; a.eps = eps;
  a.cu = nullptr;
  a.splits = splits;
  a.len_dev = length_dev; a.log_tab = log_table;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rows = (H / Hkv) * L;
  const size_t tb = fp32 ? table_bytes(H, capacity) : 0;
  a.part = reinterpret_cast<float *>(static_cast<char *>(workspace) + tb);
  int rc = MOTIF_OK;
  if (fp32) {
    const int R = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8;
    a.nqc = (rows + R - 1) / R;
    float *tab = static_cast<float *>(workspace);
    const int tn = table_len(capacity);
    chord_bias_table_kernel<<<dim3((tn + 255) / 256, H), dim3(256), 0, s>>>(a, tab, tn);
    if ((rc = check_launch("chord_bias_table_kernel"))) return rc;
    return launch_vector_dt(dtype, a, R, D, tab, tn, s);  // its merge advances the cursor
  }
  a.nqc = (rows + kMfmaRows - 1) / kMfmaRows;
  chord_decode_mfma_kernel<false><<<dim3(splits, Hkv, B * a.nqc), dim3(256), 0, s>>>(a, StepArgs{});
  if ((rc = check_launch("chord_decode_kernel"))) return rc;
  chord_merge_kernel<bf16_t><<<dim3(rows, Hkv, B), dim3(64), 0, s>>>(a);
  return check_launch("chord_merge_kernel");
}

extern "C" int motif_chord_decode(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int *length_dev, int capacity,
    const float *alpha, const float *beta, const float *mu, const float *ssmax,
    const float *log_n, int64_t ln_sb, int64_t ln_st, const float *log_table, int log_table_len,
    void *out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int Hkv, int L, int D, float scale, float eps,
    void *workspace, size_t workspace_bytes, int dtype, void *stream) {
  return motif::chord_decode_run(q, q_sb, q_sh, q_st, k_cache, k_sb, k_sh, k_st, v_cache, v_sb, v_sh, v_st,
                                 length_dev, capacity, alpha, beta, mu, ssmax, log_n, ln_sb, ln_st, log_table,
                                 log_table_len, out, o_sb, o_sh, o_st, B, H, Hkv, L, D, scale, eps, workspace,
                                 workspace_bytes, dtype, stream);
}

// ------------------------------------------------------------------ fused decode step

namespace motif {

static size_t step_ws_bytes(int B, int H, int Hkv, int L, int splits) {
  const size_t part = static_cast<size_t>(B) * Hkv * splits * (static_cast<size_t>(H / Hkv) * L) * (kD + 2) * sizeof(float);
  return part + (static_cast<size_t>(B) * Hkv + 1) * sizeof(int);
}

}  // namespace motif

extern "C" size_t motif_chord_decode_step_workspace_bytes(int B, int H, int Hkv, int L, int capacity) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || L <= 0 || capacity < L) return 0;
  return motif::step_ws_bytes(B, H, Hkv, L, motif::decode_splits(B, Hkv, capacity));
}

extern "C" int motif_chord_decode_step(
    const void *proj, int64_t p_sb, int64_t p_st, int q_off, int k_off, int v_off,
    const void *q_norm_weight, const void *k_norm_weight, float norm_eps,
    void *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st,
    void *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int *length_dev, int capacity,
    const float *alpha, const float *beta, const float *mu, const float *ssmax,
    const float *log_table, int log_table_len,
    void *out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int Hkv, int L, int D, float scale, float eps,
    void *workspace, size_t workspace_bytes, void *stream) {
  using namespace motif;
  if (B < 0 || H <= 0 || Hkv <= 0 || L < 0 || H % Hkv)
    return set_error(MOTIF_ERR_INVALID, "chord_decode_step: bad size");
  if (D != kD || (H / Hkv) * L > kMfmaRows)
    return set_error(MOTIF_ERR_UNSUPPORTED, "chord_decode_step: head_dim 64 and at most 16 query rows per kv head");
  if (B == 0 || L == 0) return MOTIF_OK;
  if (capacity < L) return set_error(MOTIF_ERR_INVALID, "chord_decode_step: capacity below the query count");
  if (!proj || !q_norm_weight || !k_norm_weight || !k_cache || !v_cache || !length_dev || !alpha || !beta || !mu ||
      !ssmax || !log_table || !out)
    return set_error(MOTIF_ERR_INVALID, "chord_decode_step: NULL pointer");
  if (log_table_len < capacity)
    return set_error(MOTIF_ERR_INVALID, "chord_decode_step: the log table is shorter than the capacity");
  if (((p_sb | p_st | q_off | k_off | v_off | k_st | v_st | o_st | k_sh | v_sh | o_sh | k_sb | v_sb | o_sb) % 8) != 0 ||
      ((reinterpret_cast<uintptr_t>(proj) | reinterpret_cast<uintptr_t>(q_norm_weight) |
        reinterpret_cast<uintptr_t>(k_norm_weight) | reinterpret_cast<uintptr_t>(k_cache) |
        reinterpret_cast<uintptr_t>(v_cache) | reinterpret_cast<uintptr_t>(out)) & 15) != 0)
    return set_error(MOTIF_ERR_UNSUPPORTED, "chord_decode_step: rows must be 16-byte aligned");
  const int splits = decode_splits(B, Hkv, capacity);
  const size_t need = step_ws_bytes(B, H, Hkv, L, splits);
  if (!workspace || workspace_bytes < need)
    return set_error(MOTIF_ERR_INVALID, "chord_decode_step: workspace too small (need " + std::to_string(need) + " bytes)");

  ChordArgs a;
  a.q = nullptr; a.q_sb = a.q_sh = a.q_st = 0;
  a.k = k_cache; a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v = v_cache; a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.alpha = alpha; a.beta = beta; a.mu = mu; a.ssmax = ssmax;
  a.log_n = nullptr; a.ln_sb = a.ln_st = 0;
  a.out = out; a.o_sb = o_sb; a.o_sh = o_sh; a.o_st = o_st;
  a.lse = nullptr;
  a.B = B; a.H = H; a.Hkv = Hkv; a.L = L; a.S = capacity; a.q_start = 0;
  a.scale = scale; a.eps = eps;
  a.cu = nullptr;
  a.part = static_cast<float *>(workspace);
  a.splits = splits;
  a.nqc = 1;
  a.len_dev = length_dev; a.log_tab = log_table;
  StepArgs sa;
  sa.proj = static_cast<const bf16_t *>(proj); sa.p_sb = p_sb; sa.p_st = p_st;
  sa.q_off = q_off; sa.k_off = k_off; sa.v_off = v_off;
  sa.qw = static_cast<const bf16_t *>(q_norm_weight); sa.kw = static_cast<const bf16_t *>(k_norm_weight);
  sa.neps = norm_eps;
  sa.cnt = reinterpret_cast<int *>(static_cast<char *>(workspace) + (need - (static_cast<size_t>(B) * Hkv + 1) * sizeof(int)));
  hipStream_t s = static_cast<hipStream_t>(stream);
  chord_decode_mfma_kernel<true><<<dim3(splits, Hkv, B), dim3(256), 0, s>>>(a, sa);
  return check_launch("chord_decode_step");
}
