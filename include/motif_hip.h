/*
 * motif_hip.h - C ABI of the MI355X (gfx950) kernels for Motif Chord's
 * sequence-mixing hot path: the Gated DeltaNet (GDN) delta rule (token
 * recurrence and chunked prefill), its short causal conv front end, and Chord
 * GGD-biased softmax attention (prefill and split-K decode).
 *
 * Conventions
 *  - Every entry point is `extern "C"`, takes raw device pointers, element
 *    strides as int64 (the innermost/feature dimension must have stride 1),
 *    sizes as int, and a hipStream_t passed as `void *stream` (NULL = default
 *    stream).  Kernels are enqueued on that stream; nothing synchronises the
 *    host, nothing allocates device memory (scratch comes in as `workspace`).
 *  - Return value: MOTIF_OK (0) or a motif_status code; `motif_last_error()`
 *    returns a message for the last failure on the calling thread.
 *  - dtype codes: MOTIF_F32 = 0, MOTIF_BF16 = 1, MOTIF_F16 = 2 (fp16: the Chord attention
 *    entries only).
 *  - Recurrent state is always fp32, row-major [.., dk, dv], contiguous.
 */
#ifndef MOTIF_HIP_H
#define MOTIF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum motif_status {
  MOTIF_OK = 0,
  MOTIF_ERR_INVALID = 1,     /* bad argument (shape, pointer, size) */
  MOTIF_ERR_UNSUPPORTED = 2, /* valid but not implemented (head dim, dtype) */
  MOTIF_ERR_HIP = 3          /* a HIP runtime call failed */
};

enum motif_dtype { MOTIF_F32 = 0, MOTIF_BF16 = 1, MOTIF_F16 = 2 };

/* Version of this ABI (bumped on any signature change). */
int motif_abi_version(void);

/* Message describing the last non-zero status returned on this thread. */
const char *motif_last_error(void);

/*
 * Token-by-token gated delta rule.
 * Replaces motif/ops/gated_deltanet.py:26-59 `recurrent_gated_delta_rule`
 * (and the L == 1 decode dispatch at motif/block/attention/gdn_attn.py:198-199).
 *   q, k [B,H,L,dk]; v [B,H,L,dv]; beta, g [B,H,L]   (all `in_dtype`)
 *   state_in  [B,H,dk,dv] fp32 or NULL (zeros)
 *   state_out [B,H,dk,dv] fp32; may alias state_in (in-place update)
 *   o [B,H,L,dv] (`out_dtype`)
 * Supported: dk in {16,32,64,128}, any dv >= 1.
 */
int motif_gdn_recurrent_fwd(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    const void *beta, int64_t b_sb, int64_t b_sh, int64_t b_st,
    const void *g, int64_t g_sb, int64_t g_sh, int64_t g_st,
    const float *state_in, float *state_out,
    void *o, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int L, int dk, int dv, int in_dtype, int out_dtype, void *stream);

/*
 * Workspace bytes needed by motif_gdn_chunk_fwd for `total_chunks` chunks
 * (B * ceil(L / chunk) for padded batches, sum of ceil(len_i / chunk) for
 * packed sequences).
 */
size_t motif_gdn_chunk_workspace_bytes(int H, int dk, int dv, int chunk, int total_chunks);

/*
 * Chunked gated delta rule (WY / UT form).
 * Replaces motif/ops/gated_deltanet.py:287-321 `chunk_gated_delta_rule` and
 * :796-834 `chunk_gated_delta_rule_triton` (with the chunk preparation of
 * :118-177 and the inter-chunk scan of :326-422 / :614-641).
 *   Layouts as motif_gdn_recurrent_fwd.
 *   Padded batches: cu_seqlens = chunk_offsets = NULL, nseq = B.
 *   Packed sequences (new capability): B == 1, cu_seqlens[nseq+1] and
 *   chunk_offsets[nseq+1] (cumulative ceil(len_i / chunk)) are device int32;
 *   state_in / state_out are then [nseq,H,dk,dv] and every sequence starts
 *   from its own state (zeros when state_in is NULL).
 *   chunk in {16, 32, 64}; dk in {32, 64, 128}; dv % 32 == 0, dv <= 256.
 */
int motif_gdn_chunk_fwd(
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
    int in_dtype, int out_dtype, void *stream);

/*
 * GatedDeltaNet chunk scans in fp32 for the backward pass (all tensors contiguous fp32,
 * chunked as [BH, N, C, .], g the within-chunk cumulative log decay [BH, N, C]):
 * forward re-scan P [BH,N,Dk,Dv] (state entering each chunk), X [BH,N,C,Dv] = U - W P,
 * S_out [BH,Dk,Dv]; replaces the reference's _gdn_fused_scan_kernel
 * (motif/ops/gated_deltanet.py:327-408, host _fused_scan_triton :644-694).  S0 may be
 * NULL (zeros).
 * Needs C <= 64 and Dk <= 128, both multiples of 16, and Dv a multiple of 16.
 */
int motif_gdn_scan_fwd_f32(const float *k, const float *W, const float *U, const float *g, const float *S0,
                           float *P, float *X, float *S_out, int BH, int N, int C, int Dk, int Dv, void *stream);
/*
 * Reverse scan: dSn [BH,N,Dk,Dv] (gradient of the state leaving each chunk) and dS0 from
 * dS_final, with the upstream dX [BH,N,C,Dv] and dP [BH,N,Dk,Dv] (either may be NULL, as
 * may dS_final); replaces the reference's _gdn_bwd_scan_kernel (:428-520, host
 * _bwd_scan :558-612).  Same size limits.
 */
int motif_gdn_scan_bwd_f32(const float *k, const float *W, const float *g, const float *dX, const float *dP,
                           const float *dS_final, float *dSn, float *dS0, int BH, int N, int C, int Dk, int Dv,
                           void *stream);
/*
 * Both chunk scans of the backward in operator form (fp32): walks S <- M_n S + Q_n
 * (transpose != 0: S <- M_n^T S + Q_n) over the chunks (reverse != 0: last chunk first)
 * from S0 [BH,Dk,Dv] (NULL: zeros), writing S before each step to rec [BH,N,Dk,Dv] and the
 * final S to S_out.  M [BH,N,Dk,Dk] (16-byte aligned), Q [BH,N,Dk,Dv]; Dk in {16, 32, 64},
 * Dv a multiple of 16.  With M = A_n = e^{gamma_C} I - Kd^T W and Q = Kd^T U it is the
 * forward re-scan (rec = P), with the same M transposed and Q = dP - W^T dX the reverse
 * scan (rec = dSn): the reference's _gdn_fused_scan_kernel and _gdn_bwd_scan_kernel
 * (motif/ops/gated_deltanet.py:327-408, :428-520) with the per-chunk products folded into
 * one operator per chunk, formed beforehand for all chunks at once.
 */
int motif_gdn_opscan_f32(const float *M, const float *Q, const float *S0, float *rec, float *S_out, int BH, int N,
                         int Dk, int Dv, int reverse, int transpose, void *stream);
/*
 * Both operator-form scans of the backward in one launch (they are independent): the
 * forward re-scan S <- A_n S + Hn_n from S0 (NULL: zeros), writing P [BH,N,Dk,Dv] and
 * S_out, side by side with the reverse scan gS <- A_n^T gS + G_n from dS_final (NULL:
 * zeros), writing dSn [BH,N,Dk,Dv] and dS0 -- motif_gdn_opscan_f32 forward and reverse
 * (transpose) as one launch; same operands and limits.
 */
int motif_gdn_opscan_pair_f32(const float *A, const float *Hn, const float *S0, float *P, float *S_out, const float *G,
                              const float *dS_final, float *dSn, float *dS0, int BH, int N, int Dk, int Dv,
                              void *stream);
/*
 * Chunk backward, the per-chunk terms before the scans (fp32).  Inputs are chunked and
 * zero-padded: q, k [BH,N,C,Dk], v, dout [BH,N,C,Dv], beta, g [BH,N,C].  Writes
 * gam = cumsum(g) per chunk [BH,N,C], T = (I + strict(beta k k^T * D))^{-1} [BH,N,C,C],
 * W = T (beta e^gam k) [BH,N,C,Dk], U = T (beta v) [BH,N,C,Dv] (the forward re-scan's
 * inputs) and the output's upstream terms dP = (q e^gam)^T dout [BH,N,Dk,Dv],
 * dX = ((q k^T) * D)^T dout [BH,N,C,Dv] (the reverse scan's inputs).  With A non-NULL it
 * also writes the operators of motif_gdn_opscan_f32: A = e^{gam_C} I - Kd^T W [BH,N,Dk,Dk],
 * Hn = Kd^T U and G = dP - W^T dX [BH,N,Dk,Dv] (Kd = k e^{gam_C - gam}); dP may then be
 * NULL.  Replaces the
 * reference's chunk preparation forward recomputed for the backward
 * (motif/ops/gated_deltanet.py:118-177, the solve_triangular at :161-166) and the
 * autograd of the output combination (:830-832).  C == 64, Dk == 64, Dv in {64, 128};
 * q, k, v, dout 16-byte aligned.
 */
int motif_gdn_bwd_prep_f32(const float *q, const float *k, const float *v, const float *beta, const float *g,
                           const float *dout, float *W, float *U, float *gam, float *T, float *dP, float *dX,
                           float *A, float *Hn, float *G, int BH, int N, int C, int Dk, int Dv, void *stream);
/*
 * Chunk backward, the per-chunk gradients after the scans (fp32): from the prep's gam, T
 * and dX, the forward re-scan's P [BH,N,Dk,Dv] and X [BH,N,C,Dv] and the reverse scan's
 * dSn [BH,N,Dk,Dv], writes dq, dk [BH,N,C,Dk], dv [BH,N,C,Dv], dbeta, dg [BH,N,C]
 * (chunked, padded rows included).  With X NULL the residuals X = U - W P are formed in
 * the kernel from the prep's W [BH,N,C,Dk] and U [BH,N,C,Dv] (else W, U may be NULL).
 * Replaces the reference's
 * _PrepareChunksFunction.backward (motif/ops/gated_deltanet.py:180-260), the per-chunk
 * products of _FusedScanFunction.backward (:742-765) and the output combination's
 * gradient.  Same size limits.
 */
int motif_gdn_bwd_chunk_f32(const float *q, const float *k, const float *v, const float *beta, const float *gam,
                            const float *T, const float *P, const float *X, const float *dSn, const float *dout,
                            const float *dX, float *dq, float *dk, float *dv, float *dbeta, float *dg, const float *W,
                            const float *U, int BH, int N, int C, int Dk, int Dv, void *stream);

/*
 * motif_gdn_chunk_fwd with the layer's output norm fused into the output pass:
 *   y[b,t,h*dv+e] = GatedRMSNorm(o[b,h,t,:]; gate[b,t,h*dv:(h+1)*dv], norm_weight, norm_eps)
 * (o rounded to `dtype` first; y = T(T(T(o rsqrt(mean o^2 + eps)) w) T(silu(gate)))).
 * Replaces the chunk call and the GatedRMSNorm of motif/block/attention/gdn_attn.py:
 * 198-209 (motif/ops/rms_norm.py:530-553).  gate and y are [B,L,H*dv] (row strides
 * gate_st / y_st, batch strides gate_sb / y_sb); o may be NULL (not stored).
 * bf16 only, on the MFMA chunk path (chunk 64, dk in {32, 64}, dv % 16 == 0,
 * dv <= 128); other shapes return MOTIF_ERR_UNSUPPORTED and the caller runs the
 * two separate calls.
 */
int motif_gdn_chunk_fwd_gated(
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
    int dtype, void *stream);

/*
 * A GatedDeltaAttention prefill from its input projections to the o_proj input, fused
 * into three kernels: the chunk-preparation kernel reads the raw projection rows and
 * computes the q / k / v short causal conv + SiLU (q, k L2-normalised per head, q scaled
 * by q_scale), the gates beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias) and
 * the outgoing conv tails itself; the state scan and the output pass (with the
 * GatedRMSNorm by the gate columns) follow as in motif_gdn_chunk_fwd_gated.  Replaces
 * motif/block/attention/gdn_attn.py:183-209 (conv :116-136, gates :193-195, chunk rule
 * motif/ops/gated_deltanet.py:796-834, GatedRMSNorm motif/ops/rms_norm.py:530-553).
 *   proj [B, L, ncols] bf16 (strides p_sb, p_st) with the columns of q (H*dk), k (H*dk),
 *   v (H*dv), the norm gate (H*dv), a (H), b (H) at q_off .. b_off; wq, wk [H*dk, 4],
 *   wv [H*dv, 4]; tail_q/k/v [B, C, 3] incoming tails or NULL (zeros); tail_*_out
 *   [nseq, C, 3] or NULL; a_log, dt_bias [H]; norm_weight [dv]; state_in [nseq, H, dk, dv]
 *   fp32 or NULL, state_out the final states; y [B, L, H*dv].  Packed sequences as
 *   motif_gdn_chunk_fwd (B == 1, zero tails and states).  Workspace:
 *   motif_gdn_chunk_workspace_bytes(H, dk, dv, 64, total_chunks).
 *   dk in {32, 64}, dv in {64, 128}, conv_k == 4, bf16; other shapes return
 *   MOTIF_ERR_UNSUPPORTED and the caller runs the separate calls.
 */
int motif_gdn_prefill_fused(
    const void *proj, int64_t p_sb, int64_t p_st, int q_off, int k_off, int v_off, int g_off, int a_off, int b_off,
    const void *wq, const void *wk, const void *wv, int conv_k,
    const void *tail_q, const void *tail_k, const void *tail_v, void *tail_q_out, void *tail_k_out, void *tail_v_out,
    const void *a_log, const void *dt_bias, float q_scale, const void *norm_weight, float norm_eps,
    const float *state_in, float *state_out, void *y, int64_t y_sb, int64_t y_st,
    int B, int H, int L, int dk, int dv,
    const int32_t *cu_seqlens, const int32_t *chunk_offsets, int nseq, int total_chunks,
    void *workspace, size_t workspace_bytes, void *stream);

/*
 * Short causal depthwise conv (kernel K) followed by SiLU.
 * Replaces motif/block/attention/gdn_attn.py:116-136 `GatedDeltaAttention._conv`.
 *   x [B,L,D] (strides x_sb, x_st; channel stride 1), weight [D,K] contiguous,
 *   tail_in [B,D,K-1] contiguous or NULL (zeros), tail_out [B,D,K-1] or NULL
 *   (may alias tail_in), y [B,L,D].  All in `dtype`.
 *   y[t] = SiLU(sum_r w[r] * xc[t+r]) with xc = [tail || x];
 *   tail_out = last K-1 entries of xc (pre-activation inputs).
 *   Packed sequences: B == 1, cu_seqlens[nseq+1] device int32, max_seqlen =
 *   longest sequence; every sequence starts from a zero tail and tail_out is
 *   then [nseq,D,K-1].  Padded batches pass cu_seqlens = NULL, nseq = B,
 *   max_seqlen = L.  K in {2, 3, 4, 5}.
 */
int motif_short_conv_silu(
    const void *x, int64_t x_sb, int64_t x_st,
    const void *weight, const void *tail_in, void *tail_out,
    void *y, int64_t y_sb, int64_t y_st,
    int B, int L, int D, int K,
    const int32_t *cu_seqlens, int nseq, int max_seqlen,
    int dtype, void *stream);

/*
 * motif_short_conv_silu followed by the per-head L2 normalisation of the GDN
 * q / k inputs: every group of head_dim consecutive channels of each timestep is
 * divided by max(||y||_2, 1e-12) (F.normalize) and multiplied by `scale`
 * (dk^-1/2 for q, 1 for k).  Replaces the conv + `F.normalize(..) * scale` pair of
 * motif/block/attention/gdn_attn.py:120-121, :190-191.  head_dim in {16, 32, 64}.
 */
int motif_short_conv_silu_l2norm(
    const void *x, int64_t x_sb, int64_t x_st,
    const void *weight, const void *tail_in, void *tail_out,
    void *y, int64_t y_sb, int64_t y_st,
    int B, int L, int D, int K,
    const int32_t *cu_seqlens, int nseq, int max_seqlen,
    int head_dim, float scale, int dtype, void *stream);

/*
 * Up to three conv + SiLU problems in one launch (the GDN q, k and v front ends of
 * motif/block/attention/gdn_attn.py:116-136, :190-191): problem p is the call
 * motif_short_conv_silu_l2norm(x[p], x_sb[p], x_st[p], weight[p], tail_in[p],
 * tail_out[p], y[p], y_sb[p], y_st[p], B, L, D[p], K, ..., head_dim[p], scale[p])
 * with head_dim[p] == 0 meaning no normalisation.  All arrays hold n host values.
 * Served only where the 16-byte vector kernel applies (16-byte aligned rows and
 * tails, tail_out != tail_in, one head size among the normalised problems, L >= 1);
 * otherwise MOTIF_ERR_UNSUPPORTED and the caller makes the separate calls.
 */
int motif_short_conv_silu_multi(
    int n, const void *const *x, const int64_t *x_sb, const int64_t *x_st,
    const void *const *weight, const void *const *tail_in, void *const *tail_out,
    void *const *y, const int64_t *y_sb, const int64_t *y_st,
    const int *D, const int *head_dim, const float *scale,
    int B, int L, int K,
    const int32_t *cu_seqlens, int nseq, int max_seqlen,
    int dtype, void *stream);

/*
 * Workspace bytes needed by motif_chord_fwd (split-K partials); also returns
 * the split count the launcher will use in *splits (may be NULL).
 */
size_t motif_chord_workspace_bytes(int B, int H, int Hkv, int L, int S, int D, int *splits);

/*
 * Chord attention forward: causal softmax attention with the per-head gated
 * geometric-decay bias b = -alpha_h (|j - i_abs - mu_h| + eps)^beta_h, logits
 * (scale q.k + b) * ssmax_h * log_n[b,i], i_abs = q_start + i, keys j <= i_abs.
 * Replaces motif/ops/chord_attention.py:1557-1625 `apply_chord_attention`
 * (forward, split-K and merge: :74-507, :1128-1299).
 *   q [B,H,L,D]; k, v [B,Hkv,S,D]; out [B,H,L,D]   (dtype)
 *   alpha, beta, mu, ssmax [H] fp32; log_n [B,L] fp32 (strides ln_sb, ln_st)
 *   lse [B,H,L] fp32 (base-2 log-sum-exp) or NULL.
 *   Packed sequences (new capability): B == 1, cu_seqlens[nseq+1] device int32,
 *   max_seqlen = longest sequence; q/k/v packed on the sequence axis (L == S),
 *   positions restart at 0 per sequence and log_n is indexed with the packed
 *   row.  Padded batches pass cu_seqlens = NULL, nseq = B, max_seqlen = L.
 *   D == 64; bf16 only.
 */
int motif_chord_fwd(
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
    int dtype, void *stream);

/*
 * Chord attention backward: dq, dk, dv of the forward above and the gradients of the [H]
 * parameters alpha, beta, mu, ssmax.  Replaces the reference's custom backward
 * motif/ops/chord_attention.py:1348-1470 `_chord_backward_impl` (kernels :518-949,
 * called from `_TritonChordFunction.backward` :1520-1554).
 *   q, out, dout, dq [B,H,L,D]; k, v, dk, dv [B,Hkv,S,D] (bf16, D == 64, padded batch)
 *   lse [B,H,L] fp32: the forward's base-2 log-sum-exp.
 *   dparam [4][H] fp32 (written): d alpha, d beta, d mu, d ssmax.
 *   workspace: motif_chord_bwd_workspace_bytes(B, H, Hkv, L, S, q_start) bytes (row sums
 *   dout . out and the fp32 partials of the chunked causal loops).  Needs 0 <= q_start
 *   and q_start + L <= S.  Results do not depend on the run: partials are summed in a
 *   fixed order.
 */
size_t motif_chord_bwd_workspace_bytes(int B, int H, int Hkv, int L, int S, int q_start);
int motif_chord_bwd(
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
    void *workspace, size_t workspace_bytes, int dtype, void *stream);

/*
 * One decode step of a GatedDeltaAttention layer after its input projections, fused:
 * conv + SiLU of the new token (q, k, v), q / k L2 normalisation (q * dk^-1/2), gates
 * beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias), the delta-rule update of the
 * fp32 state and the GatedRMSNorm of the head outputs.  Replaces the L == 1 path of
 * motif/block/attention/gdn_attn.py:183-209 (conv :116-136, recurrent_gated_delta_rule
 * motif/ops/gated_deltanet.py:26-59, GatedRMSNorm motif/ops/rms_norm.py:530-553).
 *   proj [B, ncols] (row stride proj_sb) holds the projections at column offsets
 *   q_off (H*dk), k_off (H*dk), v_off (H*dv), g_off (H*dv, the norm gate), a_off (H),
 *   b_off (H); wq, wk [H*dk, K], wv [H*dv, K] conv weights; tail_q/k/v [B, C, K-1] in,
 *   tail_q/k/v_out [B, C, K-1] the shifted tails; a_log, dt_bias [H]; norm_weight [dv];
 *   state [B, H, dk, dv] fp32 in, state_out the new state; y [B, H*dv] (row stride
 *   y_sb).  Outputs may alias their inputs (an in-place step).  All but the states in
 *   `dtype`.  dk in {16, 32, 64}, dv <= 128.
 */
int motif_gdn_decode_fused(
    const void *proj, int64_t proj_sb, int q_off, int k_off, int v_off, int g_off, int a_off, int b_off,
    const void *wq, const void *wk, const void *wv, const void *tail_q, const void *tail_k, const void *tail_v,
    void *tail_q_out, void *tail_k_out, void *tail_v_out,
    const void *a_log, const void *dt_bias, const void *norm_weight, float norm_eps,
    const float *state, float *state_out, void *y, int64_t y_sb, int B, int H, int dk, int dv, int K, int dtype,
    void *stream);

/*
 * motif_chord_decode without a workspace argument, for callers that cannot allocate
 * device memory (code under graph capture that must not call hipMalloc, tight serving
 * loops, harnesses that forbid allocation).  No counterpart in the reference.  Same
 * arguments, kernels and results as motif_chord_decode; the split partials live in a
 * scratch array the library holds on every GPU it runs on until the process ends
 * (motif_chord_decode_noalloc_scratch_bytes() bytes, 16 MiB).  Sizes whose
 * motif_chord_decode_workspace_bytes exceeds it return MOTIF_ERR_INVALID.  Calls that
 * overlap in time on one GPU (other streams, other host threads) share that scratch
 * and race: serialise them.  Allocates nothing.
 */
size_t motif_chord_decode_noalloc_scratch_bytes(void);
int motif_chord_decode_noalloc(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int *length_dev, int capacity,
    const float *alpha, const float *beta, const float *mu, const float *ssmax,
    const float *log_n, int64_t ln_sb, int64_t ln_st, const float *log_table, int log_table_len,
    void *out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int Hkv, int L, int D, float scale, float eps, int dtype, void *stream);

/*
 * A ChordAttention decode step over a device cursor in one launch (bf16, head dim 64,
 * (H / Hkv) * L <= 16 query rows per kv head): what motif_chord_qkv_prep (with its
 * device cursor) followed by motif_chord_decode computes, with the same bits --
 * q = RMSNorm(q_h; q_norm_weight) and the new keys / values k_cache[b, g, pos + t] =
 * RMSNorm(k_g; k_norm_weight), v_cache[b, g, pos + t] = v_g from the projection rows
 * proj [B, L, ncols] (strides p_sb, p_st; q, k, v of head h / kv head g at columns
 * q_off + h*64, k_off + g*64, v_off + g*64), attention over *length_dev + L keys, out
 * [B, H, L, 64], then *length_dev += L.  Replaces motif/block/attention/chord_attn.py:
 * 255-265 (q / k norms, v), the cache append motif/model/cache.py:170-215 and the
 * decode call of apply_chord_attention (motif/ops/chord_attention.py:1128-1229).
 * workspace: motif_chord_decode_step_workspace_bytes(B, H, Hkv, L, capacity) bytes whose
 * last (B * Hkv + 1) ints are arrival counters that must be zero before the first call
 * (each call leaves them zero); calls that overlap in time on one workspace race.
 */
size_t motif_chord_decode_step_workspace_bytes(int B, int H, int Hkv, int L, int capacity);
int motif_chord_decode_step(
    const void *proj, int64_t p_sb, int64_t p_st, int q_off, int k_off, int v_off,
    const void *q_norm_weight, const void *k_norm_weight, float norm_eps,
    void *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st,
    void *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int *length_dev, int capacity,
    const float *alpha, const float *beta, const float *mu, const float *ssmax,
    const float *log_table, int log_table_len,
    void *out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int Hkv, int L, int D, float scale, float eps,
    void *workspace, size_t workspace_bytes, void *stream);

/*
 * ChordAttention input stage for a preallocated KV cache: from the fused q | k | v
 * projection rows proj [B, L, ncols] (strides p_sb, p_st; head h of q at column
 * q_off + h*D, of k at k_off + g*D, of v at v_off + g*D), per head
 *   q[b, h, t]               = RMSNorm(q_h; q_norm_weight)
 *   k_cache[b, g, pos + t]   = RMSNorm(k_g; k_norm_weight)
 *   v_cache[b, g, pos + t]   = v_g
 * RMSNorm as motif/ops/rms_norm.py:481-486 (T(x * rsqrt(mean(x^2) + eps)) * w).
 * Replaces motif/block/attention/chord_attn.py:255-265 and the KV append
 * (motif/model/cache.py:170-215).
 *   pos >= 0: a host position (pos + L <= capacity); length_dev, if given, is set to
 *             pos + L.
 *   pos < 0:  the position is read from the device cursor *length_dev (left as is:
 *             motif_chord_decode advances it); cache rows at or past `capacity` are
 *             not written.
 * All row starts 16-byte aligned; D * sizeof(T) in {64, 128, 256, 512} bytes.
 */
int motif_chord_qkv_prep(const void *proj, int64_t p_sb, int64_t p_st, int q_off, int k_off, int v_off,
                         const void *q_norm_weight, const void *k_norm_weight, float eps,
                         void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                         void *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st,
                         void *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_st,
                         int *length_dev, int pos, int capacity, int B, int L, int H, int Hkv, int D, int dtype,
                         void *stream);

/*
 * Workspace bytes of motif_chord_decode for a cache of `capacity` positions (the
 * split partials, plus the fp32 path's bias table); *splits (may be NULL) receives
 * the key-range split count.
 */
size_t motif_chord_decode_workspace_bytes(int B, int H, int Hkv, int L, int capacity, int D, int dtype,
                                          int *splits);

/*
 * Chord attention of L new queries over a fixed-capacity KV cache whose length lives
 * on the device: *length_dev positions are cached and the L new keys / values are
 * already at [*length_dev, *length_dev + L) (motif_chord_qkv_prep with pos < 0 puts
 * them there).  Attends over S = *length_dev + L keys with q_start = *length_dev (the
 * reference rule chord_attn.py:266-268, q_start = cached length), then advances
 * *length_dev by L, so one captured launch sequence serves token after token.
 * Replaces the decode call of motif/ops/chord_attention.py:1557-1625 (split-K and
 * merge :1128-1229) with the cached-length bookkeeping of motif/model/cache.py:170-215
 * and the log_n lookup of motif/block/attention/chord_attn.py:274-283 moved to the
 * device.
 *   q [B,H,L,D]; k_cache, v_cache [B,Hkv,capacity,D]; out [B,H,L,D]   (dtype)
 *   log_n [B,L] fp32, or NULL: log_n[b,i] = log_table[q_start + i] with log_table
 *   ln(1..log_table_len), log_table_len >= capacity.
 *   A cursor that would pass the capacity is clamped on the device (the window then
 *   ends at the capacity); callers check the length on the host.
 *   D == 64; bf16 or fp32.
 */
int motif_chord_decode(
    const void *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void *k_cache, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void *v_cache, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int *length_dev, int capacity,
    const float *alpha, const float *beta, const float *mu, const float *ssmax,
    const float *log_n, int64_t ln_sb, int64_t ln_st, const float *log_table, int log_table_len,
    void *out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    int B, int H, int Hkv, int L, int D, float scale, float eps,
    void *workspace, size_t workspace_bytes, int dtype, void *stream);

/*
 * Intra-block attention-residual read (one fused pass):
 *   r_n = 1/sqrt(mean(x_n^2) + eps), s_n = sum_d query_d * weight_d * x_nd * r_n,
 *   alpha = softmax_n(s), out = sum_n alpha_n * x_n      (fp32 arithmetic)
 * Replaces motif/ops/attn_res.py:588-593 (the eager read of `_read_sources`) and
 * the fused Triton read it falls back from (motif/ops/attn_res.py:94-186).
 *   sources: host array of nsrc (1..8) device pointers, each [B,T,D] with strides
 *   src_sb[n], src_st[n] (host arrays); query, norm_weight [D]; out [B,T,D].
 *   All tensors in `dtype`; rows 16-byte aligned, D a multiple of 16 bytes and at
 *   most 4096 bytes (D <= 2048 bf16 / 1024 fp32).
 */
int motif_attn_res_read(const void *const *sources, const int64_t *src_sb, const int64_t *src_st,
                        int nsrc, const void *query, const void *norm_weight, float eps, void *out,
                        int64_t out_sb, int64_t out_st, int B, int T, int D, int dtype, void *stream);

/*
 * The attention-residual read above followed by up to two RMSNorms of its result h
 * (the decoder's attn_norm and mlp_norm), in the same pass: norm_outs[i] =
 * T(h * rsqrt(mean(h^2) + norm_eps)) * norm_weights[i], h first rounded to T as the
 * reference stores it.  Replaces motif/block/decoder.py:195-206 (apply_block_attn_res,
 * then attn_norm / mlp_norm; RMSNorm motif/ops/rms_norm.py:461-486).
 *   out may be NULL (h not stored); nnorm in 0..2; norm_weights[i] [D],
 *   norm_outs[i] [B,T,D] with strides norm_sb[i], norm_st[i] (host arrays).
 */
int motif_attn_res_read_norms(const void *const *sources, const int64_t *src_sb, const int64_t *src_st,
                              int nsrc, const void *query, const void *norm_weight, float eps, void *out,
                              int64_t out_sb, int64_t out_st, int nnorm, const void *const *norm_weights,
                              void *const *norm_outs, const int64_t *norm_sb, const int64_t *norm_st,
                              float norm_eps, int B, int T, int D, int dtype, void *stream);

/*
 * y = x W^T for a few activation rows (the projections of a decode step), bf16 with
 * fp32 accumulation, with the elementwise op that follows the projection fused in.
 * Replaces nn.Linear (cuBLAS / hipBLASLt) at decode sizes plus, per epilogue:
 *   0 none
 *   1 gate    y = (x W^T) * sigmoid(aux)      motif/block/attention/chord_attn.py:254, :313
 *   2 resid   y = (x W^T) + aux; y2 = aux2 + y (when y2 != NULL)
 *                                             motif/block/decoder.py:208 (f_h = attn + mlp),
 *                                             motif/model/cache.py:514-526 (partial block fold)
 *   3 swiglu  y = (x W[:N/2]^T) * SiLU(x W[N/2:]^T)
 *                                             motif/block/mlp.py:53-63, motif/ops/swiglu.py:252-253
 * Intermediates are rounded to bf16 where the reference's separate ops round.
 *   x [M, K] (row stride x_rs), W [N, K] (row stride w_rs), y / aux / aux2 / y2
 *   [M, Nout] with their row strides; Nout = N (N/2 for swiglu).  K a multiple of 32;
 *   x and W rows 16-byte aligned; any M.
 */
int motif_linear_rows(const void *x, int64_t x_rs, const void *w, int64_t w_rs, void *y, int64_t y_rs,
                      int M, int N, int K, int epilogue, const void *aux, int64_t aux_rs,
                      const void *aux2, int64_t aux2_rs, void *y2, int64_t y2_rs, void *stream);

/*
 * Two independent decode projections in one launch: the decoder's attention input
 * projection (epilogue1 0 none or 3 swiglu) and its MLP gate/up projection (SwiGLU
 * epilogue), whose inputs -- attn_norm(h) and mlp_norm(h) -- are ready together.
 * Replaces the projections at motif/block/attention/gdn_attn.py:183-207 (q/k/v/g/a/b
 * of the new token) or motif/block/attention/chord_attn.py:252-256 (g/q/k/v), together
 * with motif/block/mlp.py:63 (gate_up_proj + SwiGLU), as two motif_linear_rows calls
 * would: each output equals that call's bit for bit.
 *   problem 1: x1 [M, K1] W1 [N1, K1] -> y1 [M, N1] (N1/2 for swiglu)
 *   problem 2: x2 [M, K2] W2 [N2, K2] -> y2 [M, N2/2]
 * K1 == K2, a multiple of 64; M <= 64; rows 16-byte aligned.
 */
int motif_linear_rows_pair(const void *x1, int64_t x1_rs, const void *w1, int64_t w1_rs, void *y1, int64_t y1_rs,
                           int N1, int K1, int epilogue1, const void *x2, int64_t x2_rs, const void *w2,
                           int64_t w2_rs, void *y2, int64_t y2_rs, int N2, int K2, int M, void *stream);

/*
 * The decoder's two output projections and the residual fold in one launch:
 *   u = T(x1 W1^T), or with a gate  u = T(T(x1 W1^T) * T(sigmoid(gate)))   (o_proj)
 *   y = T(u + T(x2 W2^T))                                                   (f_h = attn + down_proj)
 *   y2 = T(aux2 + y)  when y2 != NULL                                       (the block's running sum)
 * Replaces motif/block/attention/gdn_attn.py:210 or motif/block/attention/chord_attn.py:313, :361
 * (o_proj, gated), motif/block/mlp.py:63 (down_proj) and motif/block/decoder.py:207-213
 * (f_h, update_increment) -- what motif_linear_rows with the gate epilogue followed by
 * one with the resid epilogue computes, bit for bit.
 *   x1 [M, K1], W1 [N, K1], x2 [M, K2], W2 [N, K2], gate / aux2 / y / y2 [M, N];
 *   K1, K2 multiples of 64; M <= 64; rows 16-byte aligned.
 */
int motif_linear_rows_dual(const void *x1, int64_t x1_rs, const void *w1, int64_t w1_rs, int K1, const void *x2,
                           int64_t x2_rs, const void *w2, int64_t w2_rs, int K2, const void *gate, int64_t gate_rs,
                           const void *aux2, int64_t aux2_rs, void *y, int64_t y_rs, void *y2, int64_t y2_rs, int M,
                           int N, void *stream);

/*
 * GatedRMSNorm of the GDN layer output per head without the concatenation:
 *   y[b, t, h*dv + e] = T(T(T(o * rsqrt(mean_e o^2 + eps)) * weight[e]) * T(SiLU(gate[b, t, h*dv + e])))
 * for o = o[b, h, t, :].  Replaces motif/block/attention/gdn_attn.py:206-209 (cat + o_norm,
 * motif/ops/rms_norm.py:530-553).  o [B, H, L, dv] (strides o_sb, o_sh, o_st), gate / y
 * [B, L, H*dv] (strides g_sb, g_st / y_sb, y_st), weight [dv]; rows 16-byte aligned.
 */
int motif_gated_rms_norm(const void *o, int64_t o_sb, int64_t o_sh, int64_t o_st, const void *gate,
                         int64_t g_sb, int64_t g_st, const void *weight, float eps, void *y,
                         int64_t y_sb, int64_t y_st, int B, int L, int H, int dv, int dtype, void *stream);

/*
 * y[m, :] = x[m, :I] * SiLU(x[m, I:]) (SiLU rounded to T first) -- the SwiGLU activation
 * (motif/ops/swiglu.py:252-253).  x [M, 2I] (row stride x_rs), y [M, I].
 */
int motif_swiglu(const void *x, int64_t x_rs, void *y, int64_t y_rs, int M, int I, int dtype, void *stream);

/*
 * f = a + b and p_out = p + f (p may be NULL), all [M, N] row-major with their row
 * strides: the decoder's f_h = attn + mlp and the block's running sum
 * (motif/block/decoder.py:208-213, motif/model/cache.py:514-526).
 */
int motif_add_fold(const void *a, int64_t a_rs, const void *b, int64_t b_rs, const void *p, int64_t p_rs,
                   void *f, int64_t f_rs, void *p_out, int64_t po_rs, int M, int N, int dtype, void *stream);

/*
 * A decoder's output and the block's running sum in one pass, with the adds of the
 * running sum that were put off since it was last stored:
 *   f = T(T(a * T(sigmoid(g))) + b)        (f = T(a + b) when g is NULL)
 *   p = T(..T(T(c_0 + c_1) + c_2) .. + f)  over the addends chain[0 .. nchain)
 * one add and one rounding to T each, in the order of the reference's adds
 * (motif/block/decoder.py:205-213: f_h = attn + mlp, then partial_block + f_h per
 * decoder; motif/block/attention/chord_attn.py:254: the Chord output gate).  nchain = 0:
 * no p.  With a, g, b and f NULL: p = the sum of the nchain >= 2 addends only.  All
 * [M, N] row-major with their row strides, 16-byte aligned; at most 8 addends.
 */
int motif_residual_fold(const void *a, int64_t a_rs, const void *g, int64_t g_rs, const void *b, int64_t b_rs,
                        const void *const *chain, const int64_t *chain_rs, int nchain, void *f, int64_t f_rs,
                        void *p, int64_t p_rs, int M, int N, int dtype, void *stream);

/*
 * GDN gates in one pass: beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias)
 * (softplus threshold 20), each step rounded to T as the reference's separate ops
 * round (motif/block/attention/gdn_attn.py:193-195).  a, b [B, L, H] (strides a_sb,
 * a_st / b_sb, b_st; unit head stride); a_log, dt_bias [H]; beta, g [B, H, L] with
 * strides o_sb, o_sh, o_st.
 */
int motif_gdn_gates(const void *a, int64_t a_sb, int64_t a_st, const void *b, int64_t b_sb, int64_t b_st,
                    const void *a_log, const void *dt_bias, void *beta, void *g, int64_t o_sb, int64_t o_sh,
                    int64_t o_st, int B, int L, int H, int dtype, void *stream);

/*
 * y = x * sigmoid(g) (sigmoid rounded to T), [M, N] row-major: the Chord output gate
 * o_proj(out) * G (motif/block/attention/chord_attn.py:254, :313).
 */
int motif_mul_sigmoid(const void *x, int64_t x_rs, const void *g, int64_t g_rs, void *y, int64_t y_rs,
                      int M, int N, int dtype, void *stream);

/*
 * Measurement probes (no reference counterpart): the measured denominators of the
 * roofline fractions bench.py reports beside the published MI355X peaks.
 *   motif_probe_copy       dst = src over `bytes` (a multiple of 16): each byte read
 *                          once and written once;
 *   motif_probe_read       a reduction of src (`bytes`, a multiple of 16) to one word
 *                          per workgroup in out [grid];
 *   motif_probe_mfma_bf16  `iters` rounds per wave of eight independent
 *                          v_mfma_f32_16x16x32_bf16 (shape 16) or four independent
 *                          v_mfma_f32_32x32x16_bf16 (shape 32), 16384 / 32768 flops each,
 *                          256-thread workgroups; out [grid * 256] fp32 receives one value
 *                          per thread.
 */
int motif_probe_copy(const void *src, void *dst, size_t bytes, int grid, void *stream);
int motif_probe_read(const void *src, void *out, size_t bytes, int grid, void *stream);
int motif_probe_mfma_bf16(void *out, int grid, int iters, int shape, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MOTIF_HIP_H */
