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
// chord_bwd_dq_kernel: one workgroup per (head, 128 queries, batch row), a wave per 32
// queries.  S^T = K Q^T and dP^T = V dO^T per 32-key tile on 32x32x16 MFMAs (lane l owns
// query column l % 32, so the row values -- Delta, the log-sum-exp, c -- are scalars per
// lane), dQ^T += K^T (s c dZ)^T from the same registers.  It also computes Delta (written
// for the second kernel) and per-workgroup partial sums of the four parameter gradients.
// chord_bwd_dkdv_kernel: one workgroup per (query head, 128 keys, batch row), a wave per
// 32 keys (lane l owns key column l % 32), looping over the query tiles that see its keys:
// S = Q K^T, dP = dO V^T, dV^T += dO^T P, dK^T += Q^T (s c dZ), into fp32 partials per
// query head that chord_bwd_reduce_kernel sums over each GQA group.  Both loops stage
// the next tile's global loads in registers while the current tile is computed.
// The GGD bias (and, in the dQ kernel, its three parameter derivatives) come from
// per-tile windows over the 63 distances a 32 x 32 tile meets, evaluated in registers.
#include <algorithm>

#include "capi_internal.h"
#include "common.h"

namespace motif {

namespace {

constexpr int kBD = 64;    // head dim
constexpr int kT = 32;     // keys (dQ kernel) or queries (dK / dV kernel) per tile
constexpr int kRowP = 72;  // padded LDS row of 64 bf16 (144 B)
constexpr int kTRow = 40;  // padded LDS row of a transposed 32-element tile (80 B)

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
  float *delta;   // [B][H][L] workspace
  float *pk, *pv; // [H][B][S][64] workspace: per query head dK / dV partials
  float *dparam;  // [B][nqb][H][4] partial sums (alpha, beta, mu, ssmax), summed by the caller
  int B, H, Hkv, L, S, q_start, nqb;
  float scale, eps;
};

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
  const int h = blockIdx.x, qb = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lc = lane & 31, hh = lane >> 5;
  const int kvh = h / (a.H / a.Hkv);
  const int q0 = qb * 128 + 32 * w;
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
  if (qv && hh == 0) a.delta[(static_cast<size_t>(b) * a.H + h) * a.L + my_q] = delta;
  const float lse2 = qv ? a.lse[(static_cast<size_t>(b) * a.H + h) * a.L + my_q] : 0.f;
  const float lam = a.log_n[b * a.ln_sb + int64_t(qr) * a.ln_st];
  const float sig = a.ssmax[h], al = a.alpha[h], be = a.beta[h], mu = a.mu[h];
  const float c = sig * lam, cl = c * kLog2e, s = a.scale;
  const int q_abs = a.q_start + my_q;

  const int wg_last = min(a.L, qb * 128 + 128) - 1;
  const int kv_end = min(a.S, a.q_start + wg_last + 1);
  const int ntiles = (kv_end + kT - 1) / kT;
  const int wave_kv_end = min(a.S, a.q_start + min(a.L, q0 + 32));

  __shared__ __attribute__((aligned(16))) bf16_t sK[kT * kRowP];   // K rows of the tile
  __shared__ __attribute__((aligned(16))) bf16_t sV[kT * kRowP];   // V rows
  __shared__ __attribute__((aligned(16))) bf16_t sKT[kBD * kTRow]; // K^T, keys in tperm order
  __shared__ float sW[4][4][64];                                   // per wave: b, d/dalpha, d/dbeta, d/dmu
  __shared__ float sRed[4][4];

  const bf16_t *kbase = a.k + b * a.k_sb + kvh * a.k_sh;
  const bf16_t *vbase = a.v + b * a.v_sb + kvh * a.v_sh;
  f32x16 dqacc[2];
  dqacc[0] = f32x16{};
  dqacc[1] = f32x16{};
  float sa = 0.f, sb = 0.f, sm = 0.f, ss = 0.f;
  float *win = &sW[w][0][0];

  // threads 0-127 stage K (rows and K^T), 128-255 V (rows)
  const bool kside = tid < 128;
  const int st_t = tid & 127;
  auto load_kv = [&](int n0) {
    return kside ? stage_load(kbase + int64_t(n0) * a.k_st, a.k_st, kv_end - n0, st_t)
                 : stage_load(vbase + int64_t(n0) * a.v_st, a.v_st, kv_end - n0, st_t);
  };
  Stage2 stg = load_kv(0);
  for (int kt = 0; kt < ntiles; ++kt) {
    const int n0 = kt * kT;
    __syncthreads();  // the previous tile's reads are done
    stage_store(stg, st_t, kside ? sK : sV, kside ? sKT : nullptr);
    if (kt + 1 < ntiles) stg = load_kv(n0 + kT);  // in flight during this tile's work
    const bool active = n0 < wave_kv_end;
    if (active) {
      // window entry j (lane j < 63): distance d = key - q_abs = n0 - q_start - q0 - 31 + j
      const int d = n0 - a.q_start - q0 - 31 + lane;
      const float x = fabsf(static_cast<float>(d) - mu) + a.eps;
      const float l2 = fast_log2(x);
      const float xb = fast_exp2(be * l2);
      const bool vis = d <= 0;
      const float bias = -al * xb;
      win[lane] = vis ? bias : 0.f;
      win[64 + lane] = vis ? -xb : 0.f;
      win[128 + lane] = vis ? bias * l2 * 0.6931471805599453f : 0.f;
      const float sgn = static_cast<float>(d) > mu ? 1.f : (static_cast<float>(d) < mu ? -1.f : 0.f);
      win[192 + lane] = vis ? al * be * xb * rcp_fast(x) * sgn : 0.f;
    }
    __syncthreads();
    if (!active) continue;

    f32x16 sacc = {}, pacc = {};
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      const bf16x8 ko = *reinterpret_cast<const bf16x8 *>(sK + lc * kRowP + 16 * ds + 8 * hh);
      const bf16x8 vo = *reinterpret_cast<const bf16x8 *>(sV + lc * kRowP + 16 * ds + 8 * hh);
      sacc = mma32(ko, qreg[ds], sacc);
      pacc = mma32(vo, dreg[ds], pacc);
    }
    float dz[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kk = 8 * (r >> 2) + 4 * hh + (r & 3);
      const int key = n0 + kk, j = kk - lc + 31;
      const bool vis = qv && key <= q_abs && key < a.S;
      const float rr = fmaf(s, sacc[r], win[j]);
      const float p = vis ? fast_exp2(fmaf(cl, rr, -lse2)) : 0.f;
      const float g = p * (pacc[r] - delta);
      ss = fmaf(g, vis ? rr : 0.f, ss);
      sa = fmaf(g, win[64 + j], sa);
      sb = fmaf(g, win[128 + j], sb);
      sm = fmaf(g, win[192 + j], sm);
      dz[r] = g * c * s;
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const bf16x8 zb = pack8(dz + 8 * ks);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const bf16x8 kto = *reinterpret_cast<const bf16x8 *>(sKT + (32 * dt + lc) * kTRow + 16 * ks + 8 * hh);
        dqacc[dt] = mma32(kto, zb, dqacc[dt]);
      }
    }
  }

  if (qv) {
    bf16_t *dst = a.dq + b * a.dq_sb + h * a.dq_sh + int64_t(my_q) * a.dq_st;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        *reinterpret_cast<uint2 *>(dst + 32 * dt + 8 * q4 + 4 * hh) =
            uint2{pk2bf(dqacc[dt][4 * q4], dqacc[dt][4 * q4 + 1]), pk2bf(dqacc[dt][4 * q4 + 2], dqacc[dt][4 * q4 + 3])};
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
    a.dparam[((static_cast<size_t>(b) * a.nqb + qb) * a.H + h) * 4 + tid] = tot;
  }
}

// ------------------------------------------------------------------ dK, dV
// One workgroup per (query head, 128 keys, batch row): the head's share of dK and dV in
// fp32 partials [H][B][S][64] (each query head of a GQA group separately, so the group's
// heads run in parallel); chord_bwd_reduce_kernel sums a group's partials.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) chord_bwd_dkdv_kernel(ChordBwdArgs a) {
  const int h = blockIdx.x, kb = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lc = lane & 31, hh = lane >> 5;
  const int kvh = h / (a.H / a.Hkv);
  const int k0w = kb * 128 + 32 * w;
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

  __shared__ __attribute__((aligned(16))) bf16_t sQ[kT * kRowP];    // Q rows of the query tile
  __shared__ __attribute__((aligned(16))) bf16_t sD[kT * kRowP];    // dO rows
  __shared__ __attribute__((aligned(16))) bf16_t sQT[kBD * kTRow];  // Q^T, queries in tperm order
  __shared__ __attribute__((aligned(16))) bf16_t sDT[kBD * kTRow];  // dO^T
  __shared__ float sRow[3][kT];                                      // per query: lse2, Delta, c
  __shared__ float sW[4][64];                                        // per wave: the bias window

  f32x16 dkacc[2], dvacc[2];
  dkacc[0] = dkacc[1] = dvacc[0] = dvacc[1] = f32x16{};
  const float s = a.scale;
  const float sig = a.ssmax[h], al = a.alpha[h], be = a.beta[h], mu = a.mu[h];
  const bf16_t *qbase = a.q + b * a.q_sb + h * a.q_sh;
  const bf16_t *dbase = a.dout + b * a.d_sb + h * a.d_sh;
  const size_t rbase = (static_cast<size_t>(b) * a.H + h) * a.L;
  // queries that see a key of this workgroup: i >= kb * 128 - q_start
  const int i_first = max(0, kb * 128 - a.q_start);
  const int qt_first = i_first / kT, qt_end = (a.L + kT - 1) / kT;

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
    return float4{iv ? a.lse[ri] : 0.f, iv ? a.delta[ri] : 0.f,
                  iv ? sig * a.log_n[b * a.ln_sb + int64_t(i) * a.ln_st] : 0.f, 0.f};
  };
  Stage2 stg = {};
  float4 rowv = {};
  if (qt_first < qt_end) {
    stg = load_q(qt_first * kT);
    if (tid < kT) rowv = load_row(qt_first * kT);
  }
  for (int qt = qt_first; qt < qt_end; ++qt) {
    const int i0 = qt * kT;
    __syncthreads();  // the previous tile's reads are done
    stage_store(stg, st_t, qside ? sQ : sD, qside ? sQT : sDT);
    if (tid < kT) {
      sRow[0][tid] = rowv.x;
      sRow[1][tid] = rowv.y;
      sRow[2][tid] = rowv.z;
    }
    if (qt + 1 < qt_end) {  // in flight during this tile's work
      stg = load_q(i0 + kT);
      if (tid < kT) rowv = load_row(i0 + kT);
    }
    // a wave whose keys all lie past the tile's last query skips it
    const bool active = a.q_start + i0 + kT - 1 >= k0w;
    if (active) {
      // window entry j: distance key - q_abs = k0w - q_start - i0 - 31 + j
      const int d = k0w - a.q_start - i0 - 31 + lane;
      const float x = fabsf(static_cast<float>(d) - mu) + a.eps;
      sW[w][lane] = d <= 0 ? -al * fast_exp2(be * fast_log2(x)) : 0.f;
    }
    __syncthreads();
    if (!active) continue;

    f32x16 sacc = {}, pacc = {};
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      const bf16x8 qo = *reinterpret_cast<const bf16x8 *>(sQ + lc * kRowP + 16 * ds + 8 * hh);
      const bf16x8 dov = *reinterpret_cast<const bf16x8 *>(sD + lc * kRowP + 16 * ds + 8 * hh);
      sacc = mma32(qo, kreg[ds], sacc);
      pacc = mma32(dov, vreg[ds], pacc);
    }
    float pv[16], dz[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qq = 8 * (r >> 2) + 4 * hh + (r & 3);
      const int i = i0 + qq;
      const bool vis = kvld && i < a.L && my_k <= a.q_start + i;
      const float cq = sRow[2][qq];
      const float rr = fmaf(s, sacc[r], sW[w][lc - qq + 31]);
      const float p = vis ? fast_exp2(fmaf(cq * kLog2e, rr, -sRow[0][qq])) : 0.f;
      pv[r] = p;
      dz[r] = p * (pacc[r] - sRow[1][qq]) * cq * s;
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const bf16x8 pb = pack8(pv + 8 * ks), zb = pack8(dz + 8 * ks);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const bf16x8 dto = *reinterpret_cast<const bf16x8 *>(sDT + (32 * dt + lc) * kTRow + 16 * ks + 8 * hh);
        const bf16x8 qto = *reinterpret_cast<const bf16x8 *>(sQT + (32 * dt + lc) * kTRow + 16 * ks + 8 * hh);
        dvacc[dt] = mma32(dto, pb, dvacc[dt]);
        dkacc[dt] = mma32(qto, zb, dkacc[dt]);
      }
    }
  }

  if (kvld) {
    const size_t o = ((static_cast<size_t>(h) * a.B + b) * a.S + my_k) * kBD;
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
}

// dK / dV of kv head kvh = the sum of its group's query-head partials, rounded to bf16;
// one thread per 4 elements.
__global__ void __launch_bounds__(256) chord_bwd_reduce_kernel(ChordBwdArgs a) {
  const int64_t n4 = static_cast<int64_t>(a.B) * a.Hkv * a.S * (kBD / 4);
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n4) return;
  const int d0 = 4 * static_cast<int>(e % (kBD / 4));
  const int64_t rest = e / (kBD / 4);
  const int sk = static_cast<int>(rest % a.S);
  const int kvh = static_cast<int>((rest / a.S) % a.Hkv), b = static_cast<int>(rest / (static_cast<int64_t>(a.S) * a.Hkv));
  const int G = a.H / a.Hkv;
  f32x4 ks = {0.f, 0.f, 0.f, 0.f}, vs = {0.f, 0.f, 0.f, 0.f};
  for (int g = 0; g < G; ++g) {
    const size_t o = ((static_cast<size_t>(kvh * G + g) * a.B + b) * a.S + sk) * kBD + d0;
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

}  // namespace

}  // namespace motif

extern "C" size_t motif_chord_bwd_workspace_bytes(int B, int H, int L, int S) {
  if (B <= 0 || H <= 0 || L < 0 || S < 0) return 0;
  const size_t delta = (static_cast<size_t>(B) * H * L * sizeof(float) + 255) / 256 * 256;
  return delta + 2 * static_cast<size_t>(H) * B * S * motif::kBD * sizeof(float);  // Delta, dK / dV partials
}

extern "C" size_t motif_chord_bwd_dparam_len(int B, int H, int L) {
  if (B <= 0 || H <= 0 || L <= 0) return 0;
  return static_cast<size_t>(B) * ((L + 127) / 128) * H * 4;
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
    float *dparam_partial, int B, int H, int Hkv, int L, int S, int D, int q_start, float scale, float eps,
    void *workspace, size_t workspace_bytes, int dtype, void *stream) {
  using namespace motif;
  if (B < 0 || H <= 0 || Hkv <= 0 || L < 0 || S < 0 || H % Hkv != 0)
    return set_error(MOTIF_ERR_INVALID, "chord_bwd: bad sizes");
  if (dtype != MOTIF_BF16 || D != kBD)
    return set_error(MOTIF_ERR_UNSUPPORTED, "chord_bwd: bf16 with head_dim 64 only");
  if (q_start < 0 || static_cast<int64_t>(q_start) + L > S)
    return set_error(MOTIF_ERR_INVALID, "chord_bwd: need 0 <= q_start and q_start + L <= S");
  if (B == 0 || S == 0) return MOTIF_OK;  // (L <= S) nothing to differentiate
  if (!q || !k || !v || !out || !dout || !lse || !alpha || !beta || !mu || !ssmax || !log_n || !dq || !dk || !dv ||
      !dparam_partial)
    return set_error(MOTIF_ERR_INVALID, "chord_bwd: NULL pointer");
  const int64_t st = q_sb | q_sh | q_st | k_sb | k_sh | k_st | v_sb | v_sh | v_st | o_sb | o_sh | o_st | d_sb | d_sh |
                     d_st | dq_sb | dq_sh | dq_st | dk_sb | dk_sh | dk_st | dv_sb | dv_sh | dv_st;
  const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                       reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(dout) |
                       reinterpret_cast<uintptr_t>(dq) | reinterpret_cast<uintptr_t>(dk) | reinterpret_cast<uintptr_t>(dv);
  if ((st & 7) != 0 || (al & 15) != 0) return set_error(MOTIF_ERR_UNSUPPORTED, "chord_bwd: need 16-byte aligned rows");
  const size_t need = motif_chord_bwd_workspace_bytes(B, H, L, S);
  if (!workspace || workspace_bytes < need)
    return set_error(MOTIF_ERR_INVALID, "chord_bwd: workspace too small (need " + std::to_string(need) + " bytes)");
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
  a.delta = static_cast<float *>(workspace);
  const size_t delta_bytes = (static_cast<size_t>(B) * H * L * sizeof(float) + 255) / 256 * 256;
  a.pk = reinterpret_cast<float *>(static_cast<char *>(workspace) + delta_bytes);
  a.pv = a.pk + static_cast<size_t>(H) * B * S * kBD;
  a.B = B; a.H = H; a.Hkv = Hkv; a.L = L; a.S = S; a.q_start = q_start;
  a.nqb = (L + 127) / 128;
  a.dparam = dparam_partial;
  a.scale = scale; a.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = MOTIF_OK;
  if (L > 0) {  // with no queries dK and dV are zero: the partials below stay zero
    chord_bwd_dq_kernel<<<dim3(H, a.nqb, B), dim3(256), 0, s>>>(a);
    if ((rc = check_launch("chord_bwd_dq_kernel"))) return rc;
  }
  chord_bwd_dkdv_kernel<<<dim3(H, (S + 127) / 128, B), dim3(256), 0, s>>>(a);
  if ((rc = check_launch("chord_bwd_dkdv_kernel"))) return rc;
  const int64_t n4 = static_cast<int64_t>(B) * Hkv * S * (kBD / 4);
  chord_bwd_reduce_kernel<<<dim3(static_cast<unsigned>((n4 + 255) / 256)), dim3(256), 0, s>>>(a);
  return check_launch("chord_bwd_reduce_kernel");
}
