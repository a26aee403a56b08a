// Chord attention backward on bf16 MFMA (gfx950), head dim 64.
//
// For logits z_ij = c_i r_ij with r_ij = s q_i.k_j + b_h(j - i_abs), c_i = ssmax_h
// log_n[b, i], b_h(d) = -alpha_h (|d - mu_h| + eps)^beta_h, keys j <= i_abs, softmax
// P over keys and O = P V, the gradients of an upstream dO are
//   dP = dO V^T,  Delta_i = dO_i . O_i,  dZ = P * (dP - Delta),
//   dV = P^T dO,  dQ = s (c dZ) K,  dK = s (c dZ)^T Q,
//   d alpha_h = sum c dZ * (-(x^beta)),  d beta_h = sum c dZ * b ln x,
//   d mu_h = sum c dZ * alpha beta x^(beta-1) sign(d - mu),  d ssmax_h = sum log_n dZ r
// with x = |d - mu| + eps (the reference's backward: motif/ops/chord_attention.py:518-949,
// :1348-1470).  P is rebuilt from the forward's log-sum-exp (log2 units), as there.
//
// chord_bwd_dq_kernel: one workgroup per (head, 128 queries, chunk of key tiles, batch
// row), a wave per 32 queries.  S^T = K Q^T and dP^T = V dO^T per 32-key tile on 32x32x16
// MFMAs (lane l owns query column l % 32, so the row values -- Delta, the log-sum-exp, c --
// are scalars per lane), dQ^T += K^T (s c dZ)^T from the same registers.  It also
// computes Delta (written for the second kernel) and partial sums of the four parameter
// gradients.
// chord_bwd_dkdv_kernel: one workgroup per (query head, 128 keys, chunk of query tiles,
// batch row), a wave per 32 keys (lane l owns key column l % 32): S = Q K^T, dP = dO V^T,
// dV^T += dO^T P, dK^T += Q^T (s c dZ).
// The causal loop of a block is cut into chunks of at most `cq` / `ckv` tiles so that no
// workgroup runs much longer than the average (the heaviest block otherwise sets the
// kernel's length); chunks write fp32 partials that chord_bwd_reduce_*_kernel sum in a
// fixed order (with one chunk and no GQA sharing the kernels write bf16 directly).
// Both loops keep two LDS tile buffers (one barrier per tile) and the next tile's global
// loads in registers.  The GGD bias (and, in the dQ kernel, its three parameter
// derivatives) come from per-wave windows over the 63 distances a 32 x 32 tile meets,
// evaluated in registers; tiles wholly below the causal diagonal skip the masks.
#include <algorithm>
#include <string>

#include "capi_internal.h"
#include "common.h"

namespace motif {

namespace {

constexpr int kBD = 64;    // head dim
constexpr int kT = 32;     // keys (dQ kernel) or queries (dK / dV kernel) per tile
constexpr int kRowP = 72;  // padded LDS row of 64 bf16 (144 B)
constexpr int kTRow = 40;  // padded LDS row of a transposed 32-element tile (80 B)
constexpr int kBlk = 128;  // queries (dQ kernel) or keys (dK / dV kernel) per workgroup

struct ChordBwdArgs {
  const bf16_t *q; int64_t q_sb, q_sh, q_st;
  const bf16_t *k; int64_t k_sb, k_sh, k_st;
  const bf16_t *v; int64_t v_sb, v_sh, v_st;
  const bf16_t *o; int64_t o_sb, o_sh, o_st;
  const bf16_t *dout; int64_t d_sb, d_sh, d_st;
  const float *lse;  // [B][H][L], log2 units
  const float *alpha, *beta, *mu, *ssmax;
  const float *log_n; int64_t ln_sb, ln_st;
  bf16_t *dq; int64_t dq_sb, dq_sh, dq_st;
  bf16_t *dk; int64_t dk_sb, dk_sh, dk_st;
  bf16_t *dv; int64_t dv_sb, dv_sh, dv_st;
  float *dparam;  // [4][H]: d alpha, d beta, d mu, d ssmax
  // workspace
  float *delta;   // [B][H][L]
  float *pparam;  // [nsq][B][nqb][H][4] parameter partial sums
  float *pq;      // [nsq][B][H][L][64] dQ partials (nsq > 1)
  float *pk, *pv; // [nskv][H][B][S][64] dK / dV partials (unless kv_direct)
  int B, H, Hkv, L, S, q_start, nqb, nkb;
  int cq, nsq, ckv, nskv, kv_direct;
  float scale, eps;
};

// Key tiles the dQ workgroup of query block qb visits, and query tiles the dK / dV
// workgroup of key block kb visits (first tile, end).
__host__ __device__ inline int dq_tiles(int qb, int L, int q_start) {
  const int last = std::min(L, qb * kBlk + kBlk) - 1;
  return (q_start + last + 1 + kT - 1) / kT;
}
__host__ __device__ inline int kv_first_tile(int kb, int q_start) { return std::max(0, kb * kBlk - q_start) / kT; }

__device__ __forceinline__ f32x16 mma32(const bf16x8 &a, const bf16x8 &b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// Position of element e (0..31) in a transposed tile row: accumulator lane half h holds
// elements 8a + 4h + (0..3) of each 16-element group, stored together at 8h + 4a.
__device__ __forceinline__ int tperm(int e) { return (e & ~15) | ((e & 4) << 1) | ((e & 8) >> 1) | (e & 3); }

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk2bf(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){x0, x1}, bf16x2v));
}
__device__ __forceinline__ bf16x8 pack8(const float *x) {
  return __builtin_bit_cast(bf16x8, uint4{pk2bf(x[0], x[1]), pk2bf(x[2], x[3]), pk2bf(x[4], x[5]), pk2bf(x[6], x[7])});
}
__device__ __forceinline__ uint4 ld16(const bf16_t *p) { return *reinterpret_cast<const uint4 *>(p); }

// Tile staging by 128 threads t: rows 2 (t & 15) and + 1, 8-element segment t >> 4 of a
// 32-row x 64 tile of [rows][64] bf16 rows (row r at base + r * st); rows at or past
// `nrows` read 0.  The loads go to registers one tile ahead of the stores.
struct Stage2 { uint4 a, b; };
__device__ __forceinline__ Stage2 stage_load(const bf16_t *base, int64_t st, int nrows, int t) {
  const int pr = t & 15, seg = t >> 4;
  const int r0 = 2 * pr, r1 = 2 * pr + 1;
  const uint4 z = {0u, 0u, 0u, 0u};
  return {r0 < nrows ? ld16(base + r0 * st + 8 * seg) : z, r1 < nrows ? ld16(base + r1 * st + 8 * seg) : z};
}
// The rows (padded) into `rows`, and, when `tr` is set, the transposed tile [64][32]
// (elements in tperm order) into `tr`.
__device__ __forceinline__ void stage_store(const Stage2 &g, int t, bf16_t *rows, bf16_t *tr) {
  const int pr = t & 15, seg = t >> 4;
  const int r0 = 2 * pr, r1 = 2 * pr + 1;
  *reinterpret_cast<uint4 *>(rows + r0 * kRowP + 8 * seg) = g.a;
  *reinterpret_cast<uint4 *>(rows + r1 * kRowP + 8 * seg) = g.b;
  if (tr) {
    const uint32_t aw[4] = {g.a.x, g.a.y, g.a.z, g.a.w}, bw[4] = {g.b.x, g.b.y, g.b.z, g.b.w};
    const int col = tperm(r0);  // r0 even: r1 sits right after it
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<uint32_t *>(tr + (8 * seg + 2 * i) * kTRow + col) = (aw[i] & 0xffffu) | (bw[i] << 16);
      *reinterpret_cast<uint32_t *>(tr + (8 * seg + 2 * i + 1) * kTRow + col) = (aw[i] >> 16) | (bw[i] & 0xffff0000u);
    }
  }
}

// ------------------------------------------------------------------ dQ (+ Delta, parameter sums)
__global__ void __launch_bounds__(256) chord_bwd_dq_kernel(ChordBwdArgs a) {
  const int h = blockIdx.x, qb = a.nqb - 1 - static_cast<int>(blockIdx.y);  // heaviest blocks first
  const int b = blockIdx.z / a.nsq, chunk = blockIdx.z - b * a.nsq;
  const int ntiles = dq_tiles(qb, a.L, a.q_start);
  const int t_begin = chunk * a.cq, t_end = min(ntiles, t_begin + a.cq);
  if (t_begin >= t_end) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lc = lane & 31, hh = lane >> 5;
  const int kvh = h / (a.H / a.Hkv);
  const int q0 = qb * kBlk + 32 * w;
  const int my_q = q0 + lc;
  const bool qv = my_q < a.L;
  const int qr = min(my_q, a.L - 1);

  // this lane's query row: Q and dO as B operands (d = 16 ds + 8 hh .. +8), Delta
  const bf16_t *qrow = a.q + b * a.q_sb + h * a.q_sh + int64_t(qr) * a.q_st;
  const bf16_t *drow = a.dout + b * a.d_sb + h * a.d_sh + int64_t(qr) * a.d_st;
  const bf16_t *orow = a.o + b * a.o_sb + h * a.o_sh + int64_t(qr) * a.o_st;
  bf16x8 qreg[4], dreg[4];
  float dsum = 0.f;
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) {
    qreg[ds] = __builtin_bit_cast(bf16x8, ld16(qrow + 16 * ds + 8 * hh));
    dreg[ds] = __builtin_bit_cast(bf16x8, ld16(drow + 16 * ds + 8 * hh));
    const bf16x8 ov = __builtin_bit_cast(bf16x8, ld16(orow + 16 * ds + 8 * hh));
#pragma unroll
    for (int t = 0; t < 8; ++t) dsum = fmaf(static_cast<float>(dreg[ds][t]), static_cast<float>(ov[t]), dsum);
  }
  {
    const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(dsum), __float_as_uint(dsum), false, false);
    dsum = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
  }
  const float delta = dsum;
  const size_t ri = (static_cast<size_t>(b) * a.H + h) * a.L + my_q;
  if (chunk == 0 && qv && hh == 0) a.delta[ri] = delta;
  const float lse2 = qv ? a.lse[ri] : 0.f;
  const float lam = a.log_n[b * a.ln_sb + int64_t(qr) * a.ln_st];
  const float sig = a.ssmax[h], al = a.alpha[h], be = a.beta[h], mu = a.mu[h];
  const float s = a.scale, c = sig * lam, cl = c * kLog2e, cs = c * s;
  const int q_abs = a.q_start + my_q;
  const int wave_kv_end = a.q_start + min(a.L, q0 + 32);  // keys this wave sees: < wave_kv_end
  const int kv_end = min(a.S, a.q_start + min(a.L, qb * kBlk + kBlk));

  __shared__ __attribute__((aligned(16))) bf16_t sK[2][kT * kRowP];    // K rows of the tile
  __shared__ __attribute__((aligned(16))) bf16_t sV[2][kT * kRowP];    // V rows
  __shared__ __attribute__((aligned(16))) bf16_t sKT[2][kBD * kTRow];  // K^T, keys in tperm order
  __shared__ float4 sW[4][64];  // per wave: {b, d/d alpha, d/d beta, d/d mu} per distance
  __shared__ float sRed[4][4];

  const bf16_t *kbase = a.k + b * a.k_sb + kvh * a.k_sh;
  const bf16_t *vbase = a.v + b * a.v_sb + kvh * a.v_sh;
  f32x16 dqacc[2];
  dqacc[0] = f32x16{};
  dqacc[1] = f32x16{};
  float sa = 0.f, sb = 0.f, sm = 0.f, ss = 0.f;

  // threads 0-127 stage K (rows and K^T), 128-255 V (rows)
  const bool kside = tid < 128;
  const int st_t = tid & 127;
  auto load_kv = [&](int n0) {
    return kside ? stage_load(kbase + int64_t(n0) * a.k_st, a.k_st, kv_end - n0, st_t)
                 : stage_load(vbase + int64_t(n0) * a.v_st, a.v_st, kv_end - n0, st_t);
  };
  auto store_kv = [&](const Stage2 &g, int buf) { stage_store(g, st_t, kside ? sK[buf] : sV[buf], kside ? sKT[buf] : nullptr); };
  Stage2 stg = load_kv(t_begin * kT);
  store_kv(stg, 0);
  if (t_begin + 1 < t_end) stg = load_kv((t_begin + 1) * kT);
  __syncthreads();

  for (int kt = t_begin; kt < t_end; ++kt) {
    const int n0 = kt * kT, buf = (kt - t_begin) & 1;
    if (kt + 1 < t_end) {  // the next tile into the other buffer (free since the last barrier)
      store_kv(stg, buf ^ 1);
      if (kt + 2 < t_end) stg = load_kv(n0 + 2 * kT);
    }
    if (n0 < wave_kv_end) {
      // window entry j (lane j < 63): distance d = key - q_abs = n0 - q_start - q0 - 31 + j
      {
        const int d = n0 - a.q_start - q0 - 31 + lane;
        const float x = fabsf(static_cast<float>(d) - mu) + a.eps;
        const float l2 = fast_log2(x);
        const float xb = fast_exp2(be * l2);
        const float bias = -al * xb;
        const float sgn = static_cast<float>(d) > mu ? 1.f : (static_cast<float>(d) < mu ? -1.f : 0.f);
        sW[w][lane] = d <= 0 ? float4{bias, -xb, bias * l2 * 0.6931471805599453f, al * be * xb * rcp_fast(x) * sgn}
                             : float4{0.f, 0.f, 0.f, 0.f};
      }
      // The wave reads other lanes' window entries below: LDS operations of a wave complete
      // in order, and the wave barrier keeps the compiler from moving those reads above
      // this store.
      __builtin_amdgcn_wave_barrier();
      f32x16 sacc = {}, pacc = {};
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) {
        const bf16x8 ko = *reinterpret_cast<const bf16x8 *>(sK[buf] + lc * kRowP + 16 * ds + 8 * hh);
        const bf16x8 vo = *reinterpret_cast<const bf16x8 *>(sV[buf] + lc * kRowP + 16 * ds + 8 * hh);
        sacc = mma32(ko, qreg[ds], sacc);
        pacc = mma32(vo, dreg[ds], pacc);
      }
      float dz[16];
      auto body = [&](auto masked) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = 8 * (r >> 2) + 4 * hh + (r & 3);
          const float4 wv = sW[w][kk - lc + 31];
          const float rr = fmaf(s, sacc[r], wv.x);
          float p = fast_exp2(fmaf(cl, rr, -lse2));
          if constexpr (decltype(masked)::value) p = (qv && n0 + kk <= q_abs) ? p : 0.f;
          const float g = p * (pacc[r] - delta);
          ss = fmaf(g, rr, ss);
          sa = fmaf(g, wv.y, sa);
          sb = fmaf(g, wv.z, sb);
          sm = fmaf(g, wv.w, sm);
          dz[r] = g * cs;
        }
      };
      // every key of the tile at or before every query of the wave, all queries valid
      if (n0 + kT - 1 <= a.q_start + q0 && q0 + 32 <= a.L) body(std::false_type{});
      else body(std::true_type{});
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 zb = pack8(dz + 8 * ks);
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          const bf16x8 kto = *reinterpret_cast<const bf16x8 *>(sKT[buf] + (32 * dt + lc) * kTRow + 16 * ks + 8 * hh);
          dqacc[dt] = mma32(kto, zb, dqacc[dt]);
        }
      }
    }
    __syncthreads();  // this tile's reads done, the next tile's stores visible
  }

  if (qv) {
    if (a.nsq == 1) {
      bf16_t *dst = a.dq + b * a.dq_sb + h * a.dq_sh + int64_t(my_q) * a.dq_st;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          *reinterpret_cast<uint2 *>(dst + 32 * dt + 8 * q4 + 4 * hh) =
              uint2{pk2bf(dqacc[dt][4 * q4], dqacc[dt][4 * q4 + 1]), pk2bf(dqacc[dt][4 * q4 + 2], dqacc[dt][4 * q4 + 3])};
    } else {
      float *dst = a.pq + ((((static_cast<size_t>(chunk) * a.B + b) * a.H + h) * a.L) + my_q) * kBD;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          *reinterpret_cast<f32x4 *>(dst + 32 * dt + 8 * q4 + 4 * hh) =
              f32x4{dqacc[dt][4 * q4], dqacc[dt][4 * q4 + 1], dqacc[dt][4 * q4 + 2], dqacc[dt][4 * q4 + 3]};
    }
  }
  // parameter sums: d/d(bias) = c dZ, d/d ssmax = log_n dZ r
  float part[4] = {wave_sum(sa * c), wave_sum(sb * c), wave_sum(sm * c), wave_sum(ss * lam)};
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) sRed[w][i] = part[i];
  }
  __syncthreads();
  if (tid < 4) {
    const float tot = sRed[0][tid] + sRed[1][tid] + sRed[2][tid] + sRed[3][tid];
    a.pparam[(((static_cast<size_t>(chunk) * a.B + b) * a.nqb + qb) * a.H + h) * 4 + tid] = tot;
  }
}

// ------------------------------------------------------------------ dK, dV
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) chord_bwd_dkdv_kernel(ChordBwdArgs a) {
  const int h = blockIdx.x, kb = blockIdx.y;
  const int b = blockIdx.z / a.nskv, chunk = blockIdx.z - b * a.nskv;
  const int qt_end = (a.L + kT - 1) / kT;
  const int t_begin = kv_first_tile(kb, a.q_start) + chunk * a.ckv, t_end = min(qt_end, t_begin + a.ckv);
  // a chunk with no tiles writes nothing, except that direct writes must cover every key
  if (t_begin >= t_end && !(a.kv_direct && chunk == 0)) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lc = lane & 31, hh = lane >> 5;
  const int kvh = h / (a.H / a.Hkv);
  const int k0w = kb * kBlk + 32 * w;
  const int my_k = k0w + lc;
  const bool kvld = my_k < a.S;
  const int kr = min(my_k, a.S - 1);

  const bf16_t *krow = a.k + b * a.k_sb + kvh * a.k_sh + int64_t(kr) * a.k_st;
  const bf16_t *vrow = a.v + b * a.v_sb + kvh * a.v_sh + int64_t(kr) * a.v_st;
  bf16x8 kreg[4], vreg[4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) {
    kreg[ds] = __builtin_bit_cast(bf16x8, ld16(krow + 16 * ds + 8 * hh));
    vreg[ds] = __builtin_bit_cast(bf16x8, ld16(vrow + 16 * ds + 8 * hh));
  }

  __shared__ __attribute__((aligned(16))) bf16_t sQ[2][kT * kRowP];    // Q rows of the query tile
  __shared__ __attribute__((aligned(16))) bf16_t sD[2][kT * kRowP];    // dO rows
  __shared__ __attribute__((aligned(16))) bf16_t sQT[2][kBD * kTRow];  // Q^T, queries in tperm order
  __shared__ __attribute__((aligned(16))) bf16_t sDT[2][kBD * kTRow];  // dO^T
  __shared__ float4 sRow[2][kT];  // per query: {lse2, Delta, c log2 e, c s}
  __shared__ float sW[4][64];     // per wave: the bias window

  f32x16 dkacc[2], dvacc[2];
  dkacc[0] = dkacc[1] = dvacc[0] = dvacc[1] = f32x16{};
  const float s = a.scale;
  const float sig = a.ssmax[h], al = a.alpha[h], be = a.beta[h], mu = a.mu[h];
  const bf16_t *qbase = a.q + b * a.q_sb + h * a.q_sh;
  const bf16_t *dbase = a.dout + b * a.d_sb + h * a.d_sh;
  const size_t rbase = (static_cast<size_t>(b) * a.H + h) * a.L;

  // threads 0-127 stage Q, 128-255 dO (rows and transposed); threads 0-31 the row values
  const bool qside = tid < 128;
  const int st_t = tid & 127;
  auto load_q = [&](int i0) {
    return qside ? stage_load(qbase + int64_t(i0) * a.q_st, a.q_st, a.L - i0, st_t)
                 : stage_load(dbase + int64_t(i0) * a.d_st, a.d_st, a.L - i0, st_t);
  };
  auto load_row = [&](int i0) {
    const int i = i0 + (tid & (kT - 1));
    const bool iv = i < a.L;
    const size_t ri = rbase + (iv ? i : 0);
    const float c = iv ? sig * a.log_n[b * a.ln_sb + int64_t(i) * a.ln_st] : 0.f;
    return float4{iv ? a.lse[ri] : 0.f, iv ? a.delta[ri] : 0.f, c * kLog2e, c * s};
  };
  auto store_q = [&](const Stage2 &g, const float4 &rv, int buf) {
    stage_store(g, st_t, qside ? sQ[buf] : sD[buf], qside ? sQT[buf] : sDT[buf]);
    if (tid < kT) sRow[buf][tid] = rv;
  };
  Stage2 stg = {};
  float4 rowv = {};
  if (t_begin < t_end) {
    stg = load_q(t_begin * kT);
    if (tid < kT) rowv = load_row(t_begin * kT);
    store_q(stg, rowv, 0);
    if (t_begin + 1 < t_end) {
      stg = load_q((t_begin + 1) * kT);
      if (tid < kT) rowv = load_row((t_begin + 1) * kT);
    }
  }
  __syncthreads();

  for (int qt = t_begin; qt < t_end; ++qt) {
    const int i0 = qt * kT, buf = (qt - t_begin) & 1;
    if (qt + 1 < t_end) {  // the next tile into the other buffer (free since the last barrier)
      store_q(stg, rowv, buf ^ 1);
      if (qt + 2 < t_end) {
        stg = load_q(i0 + 2 * kT);
        if (tid < kT) rowv = load_row(i0 + 2 * kT);
      }
    }
    // a wave whose keys all lie past the tile's last query (or past S) skips it
    if (k0w < a.S && a.q_start + i0 + kT - 1 >= k0w) {
      {  // window entry j: distance key - q_abs = k0w - q_start - i0 - 31 + j
        const int d = k0w - a.q_start - i0 - 31 + lane;
        const float x = fabsf(static_cast<float>(d) - mu) + a.eps;
        sW[w][lane] = d <= 0 ? -al * fast_exp2(be * fast_log2(x)) : 0.f;
      }
      // The wave reads other lanes' window entries below: LDS operations of a wave complete
      // in order, and the wave barrier keeps the compiler from moving those reads above
      // this store.
      __builtin_amdgcn_wave_barrier();
      f32x16 sacc = {}, pacc = {};
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) {
        const bf16x8 qo = *reinterpret_cast<const bf16x8 *>(sQ[buf] + lc * kRowP + 16 * ds + 8 * hh);
        const bf16x8 dov = *reinterpret_cast<const bf16x8 *>(sD[buf] + lc * kRowP + 16 * ds + 8 * hh);
        sacc = mma32(qo, kreg[ds], sacc);
        pacc = mma32(dov, vreg[ds], pacc);
      }
      float pv[16], dz[16];
      auto body = [&](auto masked) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qq = 8 * (r >> 2) + 4 * hh + (r & 3);
          const float4 rw = sRow[buf][qq];
          const float rr = fmaf(s, sacc[r], sW[w][lc - qq + 31]);
          float p = fast_exp2(fmaf(rw.z, rr, -rw.x));
          if constexpr (decltype(masked)::value) p = (kvld && i0 + qq < a.L && my_k <= a.q_start + i0 + qq) ? p : 0.f;
          pv[r] = p;
          dz[r] = p * (pacc[r] - rw.y) * rw.w;
        }
      };
      // every key of the wave at or before every query of the tile, all queries valid
      if (k0w + 31 <= a.q_start + i0 && i0 + kT <= a.L) body(std::false_type{});
      else body(std::true_type{});
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 pb = pack8(pv + 8 * ks), zb = pack8(dz + 8 * ks);
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          const bf16x8 dto = *reinterpret_cast<const bf16x8 *>(sDT[buf] + (32 * dt + lc) * kTRow + 16 * ks + 8 * hh);
          const bf16x8 qto = *reinterpret_cast<const bf16x8 *>(sQT[buf] + (32 * dt + lc) * kTRow + 16 * ks + 8 * hh);
          dvacc[dt] = mma32(dto, pb, dvacc[dt]);
          dkacc[dt] = mma32(qto, zb, dkacc[dt]);
        }
      }
    }
    __syncthreads();  // this tile's reads done, the next tile's stores visible
  }

  if (!kvld) return;
  if (a.kv_direct) {
    bf16_t *dk = a.dk + b * a.dk_sb + kvh * a.dk_sh + int64_t(my_k) * a.dk_st;
    bf16_t *dv = a.dv + b * a.dv_sb + kvh * a.dv_sh + int64_t(my_k) * a.dv_st;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d0 = 32 * dt + 8 * q4 + 4 * hh;
        *reinterpret_cast<uint2 *>(dk + d0) =
            uint2{pk2bf(dkacc[dt][4 * q4], dkacc[dt][4 * q4 + 1]), pk2bf(dkacc[dt][4 * q4 + 2], dkacc[dt][4 * q4 + 3])};
        *reinterpret_cast<uint2 *>(dv + d0) =
            uint2{pk2bf(dvacc[dt][4 * q4], dvacc[dt][4 * q4 + 1]), pk2bf(dvacc[dt][4 * q4 + 2], dvacc[dt][4 * q4 + 3])};
      }
    return;
  }
  const size_t o = (((static_cast<size_t>(chunk) * a.H + h) * a.B + b) * a.S + my_k) * kBD;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d0 = 32 * dt + 8 * q4 + 4 * hh;
      *reinterpret_cast<f32x4 *>(a.pk + o + d0) =
          f32x4{dkacc[dt][4 * q4], dkacc[dt][4 * q4 + 1], dkacc[dt][4 * q4 + 2], dkacc[dt][4 * q4 + 3]};
      *reinterpret_cast<f32x4 *>(a.pv + o + d0) =
          f32x4{dvacc[dt][4 * q4], dvacc[dt][4 * q4 + 1], dvacc[dt][4 * q4 + 2], dvacc[dt][4 * q4 + 3]};
    }
}

// dK / dV of kv head kvh = the sum over its GQA group's query heads and the chunks of the
// key's block, in that order, rounded to bf16; one thread per 4 elements.
__global__ void __launch_bounds__(256) chord_bwd_reduce_kv_kernel(ChordBwdArgs a) {
  const int64_t n4 = static_cast<int64_t>(a.B) * a.Hkv * a.S * (kBD / 4);
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n4) return;
  const int d0 = 4 * static_cast<int>(e % (kBD / 4));
  const int64_t rest = e / (kBD / 4);
  const int sk = static_cast<int>(rest % a.S);
  const int kvh = static_cast<int>((rest / a.S) % a.Hkv), b = static_cast<int>(rest / (static_cast<int64_t>(a.S) * a.Hkv));
  const int G = a.H / a.Hkv;
  const int qt_end = (a.L + kT - 1) / kT;
  const int nqt = max(0, qt_end - kv_first_tile(sk / kBlk, a.q_start));
  const int ns = (nqt + a.ckv - 1) / a.ckv;
  f32x4 ks = {0.f, 0.f, 0.f, 0.f}, vs = {0.f, 0.f, 0.f, 0.f};
  for (int g = 0; g < G; ++g)
    for (int c = 0; c < ns; ++c) {
      const size_t o = (((static_cast<size_t>(c) * a.H + kvh * G + g) * a.B + b) * a.S + sk) * kBD + d0;
      const f32x4 pk = *reinterpret_cast<const f32x4 *>(a.pk + o), pv = *reinterpret_cast<const f32x4 *>(a.pv + o);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ks[i] += pk[i];
        vs[i] += pv[i];
      }
    }
  bf16_t *dk = a.dk + b * a.dk_sb + kvh * a.dk_sh + int64_t(sk) * a.dk_st + d0;
  bf16_t *dv = a.dv + b * a.dv_sb + kvh * a.dv_sh + int64_t(sk) * a.dv_st + d0;
  *reinterpret_cast<uint2 *>(dk) = uint2{pk2bf(ks[0], ks[1]), pk2bf(ks[2], ks[3])};
  *reinterpret_cast<uint2 *>(dv) = uint2{pk2bf(vs[0], vs[1]), pk2bf(vs[2], vs[3])};
}

// dQ = the sum over the chunks of the query's block, in order, rounded to bf16.
__global__ void __launch_bounds__(256) chord_bwd_reduce_q_kernel(ChordBwdArgs a) {
  const int64_t n4 = static_cast<int64_t>(a.B) * a.H * a.L * (kBD / 4);
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n4) return;
  const int d0 = 4 * static_cast<int>(e % (kBD / 4));
  const int64_t rest = e / (kBD / 4);
  const int i = static_cast<int>(rest % a.L);
  const int h = static_cast<int>((rest / a.L) % a.H), b = static_cast<int>(rest / (static_cast<int64_t>(a.L) * a.H));
  const int ns = (dq_tiles(i / kBlk, a.L, a.q_start) + a.cq - 1) / a.cq;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < ns; ++c) {
    const f32x4 p = *reinterpret_cast<const f32x4 *>(
        a.pq + (((static_cast<size_t>(c) * a.B + b) * a.H + h) * a.L + i) * kBD + d0);
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] += p[t];
  }
  bf16_t *dst = a.dq + b * a.dq_sb + h * a.dq_sh + int64_t(i) * a.dq_st + d0;
  *reinterpret_cast<uint2 *>(dst) = uint2{pk2bf(acc[0], acc[1]), pk2bf(acc[2], acc[3])};
}

// dparam[k][h] = the sum of the dQ workgroups' partials (batch rows, query blocks, chunks):
// one wave per (k, h), lanes over (batch row, query block) in a fixed order.
__global__ void __launch_bounds__(64) chord_bwd_reduce_param_kernel(ChordBwdArgs a) {
  const int t = blockIdx.x, h = t % a.H, k = t / a.H, lane = threadIdx.x;
  float acc = 0.f;
  for (int e = lane; e < a.B * a.nqb; e += 64) {
    const int b = e / a.nqb, qb = e - b * a.nqb;
    const int ns = (dq_tiles(qb, a.L, a.q_start) + a.cq - 1) / a.cq;
    for (int c = 0; c < ns; ++c) acc += a.pparam[(((static_cast<size_t>(c) * a.B + b) * a.nqb + qb) * a.H + h) * 4 + k];
  }
  acc = wave_sum(acc);
  if (lane == 0) a.dparam[k * a.H + h] = acc;
}

}  // namespace

// Chunk sizes: about 1024 chunks over the whole causal loop, at least 16 tiles each and at
// most 8 chunks per block.
struct BwdPlan {
  int nqb, nkb, cq, nsq, ckv, nskv;
  bool kv_direct;
  size_t off_param, off_pq, off_pk, off_pv, bytes;
};

static BwdPlan plan_bwd(int B, int H, int Hkv, int L, int S, int q_start) {
  BwdPlan p{};
  p.nqb = (L + kBlk - 1) / kBlk;
  p.nkb = (S + kBlk - 1) / kBlk;
  auto chunking = [](int64_t total, int maxt, int &csize, int &ns) {
    csize = static_cast<int>(std::max<int64_t>({16, (total + 1023) / 1024, (maxt + 7) / 8}));
    ns = std::max(1, (maxt + csize - 1) / csize);
  };
  int64_t tq = 0, tkv = 0;
  for (int qb = 0; qb < p.nqb; ++qb) tq += dq_tiles(qb, L, q_start);
  const int qt_end = (L + kT - 1) / kT;
  for (int kb = 0; kb < p.nkb; ++kb) tkv += std::max(0, qt_end - kv_first_tile(kb, q_start));
  chunking(tq * B * H, p.nqb ? dq_tiles(p.nqb - 1, L, q_start) : 0, p.cq, p.nsq);
  chunking(tkv * B * H, qt_end, p.ckv, p.nskv);
  p.kv_direct = H == Hkv && p.nskv == 1;
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  size_t off = al(static_cast<size_t>(B) * H * L * sizeof(float));  // Delta
  p.off_param = off;
  off += al(static_cast<size_t>(p.nsq) * B * p.nqb * H * 4 * sizeof(float));
  p.off_pq = off;
  if (p.nsq > 1) off += al(static_cast<size_t>(p.nsq) * B * H * L * kBD * sizeof(float));
  p.off_pk = p.off_pv = off;
  if (!p.kv_direct) {
    const size_t kvp = al(static_cast<size_t>(p.nskv) * H * B * S * kBD * sizeof(float));
    p.off_pv = off + kvp;
    off += 2 * kvp;
  }
  p.bytes = off;
  return p;
}

}  // namespace motif

extern "C" size_t motif_chord_bwd_workspace_bytes(int B, int H, int Hkv, int L, int S, int q_start) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || L < 0 || S < 0 || q_start < 0) return 0;
  return motif::plan_bwd(B, H, Hkv, L, S, q_start).bytes;
}

extern "C" int motif_chord_bwd(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    const void *out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    const void *dout, int64_t d_sb, int64_t d_sh, int64_t d_st,
    const float *lse, const float *alpha, const float *beta, const float *mu, const float *ssmax,
    const float *log_n, int64_t ln_sb, int64_t ln_st,
    void *dq, int64_t dq_sb, int64_t dq_sh, int64_t dq_st,
    void *dk, int64_t dk_sb, int64_t dk_sh, int64_t dk_st,
    void *dv, int64_t dv_sb, int64_t dv_sh, int64_t dv_st,
    float *dparam, int B, int H, int Hkv, int L, int S, int D, int q_start, float scale, float eps,
    void *workspace, size_t workspace_bytes, int dtype, void *stream) {
  using namespace motif;
  if (B < 0 || H <= 0 || Hkv <= 0 || L < 0 || S < 0 || H % Hkv != 0)
    return set_error(MOTIF_ERR_INVALID, "chord_bwd: bad sizes");
  if (dtype != MOTIF_BF16 || D != kBD)
    return set_error(MOTIF_ERR_UNSUPPORTED, "chord_bwd: bf16 with head_dim 64 only");
  if (q_start < 0 || static_cast<int64_t>(q_start) + L > S)
    return set_error(MOTIF_ERR_INVALID, "chord_bwd: need 0 <= q_start and q_start + L <= S");
  if (!dparam) return set_error(MOTIF_ERR_INVALID, "chord_bwd: NULL pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (B == 0 || S == 0) {  // (L <= S) nothing to differentiate: zero parameter gradients
    ChordBwdArgs z{};
    z.H = H;
    z.cq = 1;
    z.dparam = dparam;
    chord_bwd_reduce_param_kernel<<<dim3(4 * H), dim3(64), 0, s>>>(z);
    return check_launch("chord_bwd_reduce_param_kernel");
  }
  if (!q || !k || !v || !out || !dout || !lse || !alpha || !beta || !mu || !ssmax || !log_n || !dq || !dk || !dv)
    return set_error(MOTIF_ERR_INVALID, "chord_bwd: NULL pointer");
  const int64_t st = q_sb | q_sh | q_st | k_sb | k_sh | k_st | v_sb | v_sh | v_st | o_sb | o_sh | o_st | d_sb | d_sh |
                     d_st | dq_sb | dq_sh | dq_st | dk_sb | dk_sh | dk_st | dv_sb | dv_sh | dv_st;
  const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                       reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(dout) |
                       reinterpret_cast<uintptr_t>(dq) | reinterpret_cast<uintptr_t>(dk) | reinterpret_cast<uintptr_t>(dv);
  if ((st & 7) != 0 || (al & 15) != 0) return set_error(MOTIF_ERR_UNSUPPORTED, "chord_bwd: need 16-byte aligned rows");
  const BwdPlan pl = plan_bwd(B, H, Hkv, L, S, q_start);
  if (!workspace || workspace_bytes < pl.bytes)
    return set_error(MOTIF_ERR_INVALID, "chord_bwd: workspace too small (need " + std::to_string(pl.bytes) + " bytes)");
  ChordBwdArgs a;
  a.q = static_cast<const bf16_t *>(q); a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.k = static_cast<const bf16_t *>(k); a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v = static_cast<const bf16_t *>(v); a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.o = static_cast<const bf16_t *>(out); a.o_sb = o_sb; a.o_sh = o_sh; a.o_st = o_st;
  a.dout = static_cast<const bf16_t *>(dout); a.d_sb = d_sb; a.d_sh = d_sh; a.d_st = d_st;
  a.lse = lse; a.alpha = alpha; a.beta = beta; a.mu = mu; a.ssmax = ssmax;
  a.log_n = log_n; a.ln_sb = ln_sb; a.ln_st = ln_st;
  a.dq = static_cast<bf16_t *>(dq); a.dq_sb = dq_sb; a.dq_sh = dq_sh; a.dq_st = dq_st;
  a.dk = static_cast<bf16_t *>(dk); a.dk_sb = dk_sb; a.dk_sh = dk_sh; a.dk_st = dk_st;
  a.dv = static_cast<bf16_t *>(dv); a.dv_sb = dv_sb; a.dv_sh = dv_sh; a.dv_st = dv_st;
  a.dparam = dparam;
  char *ws = static_cast<char *>(workspace);
  a.delta = reinterpret_cast<float *>(ws);
  a.pparam = reinterpret_cast<float *>(ws + pl.off_param);
  a.pq = reinterpret_cast<float *>(ws + pl.off_pq);
  a.pk = reinterpret_cast<float *>(ws + pl.off_pk);
  a.pv = reinterpret_cast<float *>(ws + pl.off_pv);
  a.B = B; a.H = H; a.Hkv = Hkv; a.L = L; a.S = S; a.q_start = q_start;
  a.nqb = pl.nqb; a.nkb = pl.nkb;
  a.cq = pl.cq; a.nsq = pl.nsq; a.ckv = pl.ckv; a.nskv = pl.nskv; a.kv_direct = pl.kv_direct ? 1 : 0;
  a.scale = scale; a.eps = eps;
  int rc = MOTIF_OK;
  if (L > 0) {  // with no queries dK and dV are zero (the dK / dV pass below writes them)
    chord_bwd_dq_kernel<<<dim3(H, pl.nqb, B * pl.nsq), dim3(256), 0, s>>>(a);
    if ((rc = check_launch("chord_bwd_dq_kernel"))) return rc;
    if (pl.nsq > 1) {
      const int64_t n4 = static_cast<int64_t>(B) * H * L * (kBD / 4);
      chord_bwd_reduce_q_kernel<<<dim3(static_cast<unsigned>((n4 + 255) / 256)), dim3(256), 0, s>>>(a);
      if ((rc = check_launch("chord_bwd_reduce_q_kernel"))) return rc;
    }
  }
  chord_bwd_reduce_param_kernel<<<dim3(4 * H), dim3(64), 0, s>>>(a);
  if ((rc = check_launch("chord_bwd_reduce_param_kernel"))) return rc;
  chord_bwd_dkdv_kernel<<<dim3(H, pl.nkb, B * pl.nskv), dim3(256), 0, s>>>(a);
  if ((rc = check_launch("chord_bwd_dkdv_kernel"))) return rc;
  if (!pl.kv_direct) {
    const int64_t n4 = static_cast<int64_t>(B) * Hkv * S * (kBD / 4);
    chord_bwd_reduce_kv_kernel<<<dim3(static_cast<unsigned>((n4 + 255) / 256)), dim3(256), 0, s>>>(a);
    if ((rc = check_launch("chord_bwd_reduce_kv_kernel"))) return rc;
  }
  return MOTIF_OK;
}
