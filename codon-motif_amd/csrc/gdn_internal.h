// Shared between the GDN translation units.
#pragma once

#include "capi_internal.h"
#include "common.h"

namespace motif {

struct GdnArgs {
  const void *q; int64_t q_sb, q_sh, q_st;
  const void *k; int64_t k_sb, k_sh, k_st;
  const void *v; int64_t v_sb, v_sh, v_st;
  const void *beta; int64_t b_sb, b_sh, b_st;
  const void *g; int64_t g_sb, g_sh, g_st;
  const float *s_in;
  float *s_out;
  void *o; int64_t o_sb, o_sh, o_st;
  int B, H, L, dk, dv;
  // Optional GatedRMSNorm epilogue of the bf16 MFMA chunk path (gate == nullptr: off):
  // y[b, t, h*dv + e] = T(T(T(o * rsqrt(mean_e o^2 + eps)) * w[e]) * T(silu(gate[b, t, h*dv + e])))
  // with o rounded to T first; o itself is stored only when non-null.
  const void *gate; int64_t gt_sb, gt_st;   // [B, L, H*dv]
  const void *nw; float neps;               // [dv]
  void *y; int64_t y_sb, y_st;              // [B, L, H*dv]
};

struct ChunkArgs {
  const int32_t *cu;    // packed-sequence boundaries or nullptr
  const int32_t *coff;  // cumulative chunk counts or nullptr
  int nseq;
  int nper;             // chunks per batch row (padded batches)
  int total_chunks;
  float *gam;           // [H][TC][C]
  float *W;             // [H][TC][C][DK]
  float *U;             // [H][TC][C][DV]
  float *attn;          // [H][TC][C][C]
};

// ------------------------------------------------------------------ chunk map
struct ChunkInfo {
  int batch, seq, t0, len;
};

__device__ __forceinline__ ChunkInfo resolve_chunk(int c, int C, int L, const ChunkArgs &ca) {
  ChunkInfo ci;
  int tok_end;
  if (ca.cu == nullptr) {
    ci.seq = c / ca.nper;
    ci.batch = ci.seq;
    ci.t0 = (c - ci.seq * ca.nper) * C;
    tok_end = L;
  } else {
    int lo = 0, hi = ca.nseq - 1;  // largest s with coff[s] <= c (skips empty sequences)
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (ca.coff[mid] <= c) lo = mid;
      else hi = mid - 1;
    }
    ci.seq = lo;
    ci.batch = 0;
    ci.t0 = ca.cu[lo] + (c - ca.coff[lo]) * C;
    tok_end = ca.cu[lo + 1];
  }
  ci.len = min(C, tok_end - ci.t0);
  return ci;
}

// MFMA chunk path (gdn_chunk.hip): chunk 64, dk in {32, 64}, dv % 16 == 0, dv <= 128.
bool chunk_mfma_supported(int dk, int dv, int chunk);
size_t chunk_mfma_workspace_bytes(int H, int dk, int dv, int total_chunks);
// bf16 in and out, supported shape, 16-byte aligned q / k / v rows.
bool chunk_mfma_eligible(const GdnArgs &a, int chunk, int in_dtype, int out_dtype);
int launch_chunk_mfma(const GdnArgs &a, const ChunkArgs &ca, void *workspace, hipStream_t s);

}  // namespace motif
