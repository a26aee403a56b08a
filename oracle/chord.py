'''CPU restatement of Chord attention (GGD-biased causal softmax).  Test infrastructure only.'''
import math

import torch

GGD_EPS = 1e-5


def ggd_bias(alpha, beta, mu, q_len, kv_len, q_start, eps=GGD_EPS, dtype=torch.float64):
    '''Materialised GGD bias [H, q_len, kv_len].

    Follows motif/block/attention/chord_attn.py:140-176: d = k_pos - q_pos with
    q_pos = q_start + i; bias = -alpha * (|d - mu| + eps) ** beta.
    '''
    a, b, m = (t.to(dtype) for t in (alpha, beta, mu))
    q_pos = torch.arange(q_len, dtype=dtype) + float(q_start)
    k_pos = torch.arange(kv_len, dtype=dtype)
    d = k_pos[None, :] - q_pos[:, None]
    base = torch.abs(d[None] - m[:, None, None]) + eps
    return -a[:, None, None] * base ** b[:, None, None]


def chord_attention(q, k, v, alpha, beta, mu, ssmax, log_n, q_start=None,
                    softmax_scale=None, eps=GGD_EPS, compute_dtype=torch.float64):
    '''Chord attention forward with the bias materialised (the eager path).

    Follows motif/block/attention/chord_attn.py:316-361 and the semantics of
    motif/ops/chord_attention.py:1557-1625 (defaults q_start = S - L,
    scale = D^-1/2) and :145-244 (GQA head map h // (H / Hkv), causal rule
    key <= q_start + i, keys >= S invisible):
      logits = (scale * q.k + bias) * ssmax_h * log_n[b, i]
      logits = clamp_min(logits, finfo.min / 4); masked -> -inf; softmax; @ v.
    Computed entirely in `compute_dtype` (no rounding of the probabilities).

    Args:
        q: [B, H, L, D];  k, v: [B, Hkv, S, D];  alpha, beta, mu, ssmax: [H];
        log_n: [B, L] (or [L]).

    Returns:
        [B, H, L, D] in compute_dtype.
    '''
    B, H, L, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    if q_start is None:
        q_start = S - L
    cd = compute_dtype
    qf, kf, vf = (t.to(cd) for t in (q, k, v))
    if Hkv != H:
        rep = H // Hkv
        kf = kf.repeat_interleave(rep, dim=1)
        vf = vf.repeat_interleave(rep, dim=1)
    scores = (qf @ kf.transpose(-1, -2)) * softmax_scale
    bias = ggd_bias(alpha, beta, mu, L, S, q_start, eps, cd)
    logits = scores + bias[None]
    ln = log_n.to(cd)
    ln = ln.view(1, 1, L, 1) if ln.dim() == 1 else ln.view(B, 1, L, 1)
    logits = logits * (ssmax.to(cd).view(1, H, 1, 1) * ln)
    logits = logits.clamp_min(torch.finfo(cd).min / 4)
    q_pos = torch.arange(L) + int(q_start)
    k_pos = torch.arange(S)
    logits = logits.masked_fill(k_pos[None, :] > q_pos[:, None], float('-inf'))
    attn = torch.softmax(logits, dim=-1)
    return attn @ vf


def chord_attention_bruteforce(q, k, v, alpha, beta, mu, ssmax, log_n, q_start,
                               softmax_scale, eps=GGD_EPS):
    '''Pure-Python scalar loops over (b, h, i, j) in float64; tiny inputs only.

    An independent statement of the same definition used to pin
    `chord_attention` (no tensor broadcasting, explicit max-shifted softmax).
    '''
    B, H, L, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    Q, K, V = q.double().tolist(), k.double().tolist(), v.double().tolist()
    al, be, mu_, ss = (t.double().tolist() for t in (alpha, beta, mu, ssmax))
    ln = log_n.double().tolist()
    out = [[[[0.0] * D for _ in range(L)] for _ in range(H)] for _ in range(B)]
    for b in range(B):
        for h in range(H):
            kh = h // (H // Hkv)
            for i in range(L):
                qa = q_start + i
                row = []
                for j in range(min(S, qa + 1)):
                    dot = sum(Q[b][h][i][t] * K[b][kh][j][t] for t in range(D))
                    dist = j - qa
                    bias = -al[h] * (abs(dist - mu_[h]) + eps) ** be[h]
                    row.append((softmax_scale * dot + bias) * ss[h] * ln[b][i])
                if not row:
                    continue
                mx = max(row)
                w = [math.exp(x - mx) for x in row]
                tot = sum(w)
                for t in range(D):
                    out[b][h][i][t] = sum(w[j] * V[b][kh][j][t] for j in range(len(w))) / tot
    return torch.tensor(out, dtype=torch.float64)


def log_n_table(q_start, q_len):
    '''log(q_start + 1 .. q_start + q_len): motif/block/attention/chord_attn.py:21-43, :282-283.'''
    return torch.log(torch.arange(q_start + 1, q_start + q_len + 1, dtype=torch.float64))


def chord_attention_varlen(q, k, v, alpha, beta, mu, ssmax, cu_seqlens,
                           softmax_scale=None, eps=GGD_EPS, compute_dtype=torch.float64):
    '''Packed-sequence Chord attention (B == 1): new capability.

    Defined as an independent causal run per sequence with positions restarting
    at 0 and log_n = log(1 .. len) per sequence, outputs concatenated on L.
    '''
    cu = [int(c) for c in cu_seqlens]
    outs = []
    for i in range(len(cu) - 1):
        s, e = cu[i], cu[i + 1]
        qs, ks, vs = q[:, :, s:e], k[:, :, s:e], v[:, :, s:e]
        ln = log_n_table(0, e - s)[None]
        outs.append(chord_attention(qs, ks, vs, alpha, beta, mu, ssmax, ln, 0,
                                    softmax_scale, eps, compute_dtype))
    return torch.cat(outs, dim=2)


def ggd_parameters(p):
    '''alpha = exp(theta_alpha), beta = theta_beta, mu = 2 sinh(theta_mu).

    Follows motif/block/attention/chord_attn.py:126-138.
    '''
    tm = p['theta_mu'].double()
    return p['theta_alpha'].double().exp(), p['theta_beta'].double(), tm.exp() - (-tm).exp()


def chord_layer(hidden, p, num_heads, num_kv_heads, k_cache=None, v_cache=None,
                q_start=0, eps_norm=1e-6, cu_seqlens=None):
    '''ChordAttention.forward, restated: motif/block/attention/chord_attn.py:204-361.

    G = sigmoid(g_proj h) (:254); q/k/v projections and per-head RMSNorm on q, k
    (:256-261); K/V appended to the cache (:263-270; q_start = cached length when
    the position is 0); log_n = log(q_start + 1 ..) (:274-283); attention
    (:316-359); o_proj(out) * G (:361).

    Returns:
        (output [B, L, hidden], k_all [B, Hkv, S, D], v_all [B, Hkv, S, D])
    '''
    B, L, hid = hidden.shape
    D = hid // num_heads
    G = torch.sigmoid(hidden @ p['g_proj.weight'].t())
    q = (hidden @ p['q_proj.weight'].t()).view(B, L, num_heads, D).transpose(1, 2)
    k = (hidden @ p['k_proj.weight'].t()).view(B, L, num_kv_heads, D).transpose(1, 2)
    v = (hidden @ p['v_proj.weight'].t()).view(B, L, num_kv_heads, D).transpose(1, 2)
    from oracle.gdn import rms_norm
    q = rms_norm(q, p['q_norm.weight'], eps_norm)
    k = rms_norm(k, p['k_norm.weight'], eps_norm)
    alpha, beta, mu = ggd_parameters(p)
    ssmax = p['ssmax_s'].double()
    cd = torch.float64 if hidden.dtype == torch.float64 else torch.float32
    if cu_seqlens is not None:
        out = chord_attention_varlen(q, k, v, alpha, beta, mu, ssmax, cu_seqlens,
                                     softmax_scale=D ** -0.5, compute_dtype=cd)
        k_all, v_all = k, v
    else:
        if k_cache is not None and k_cache.shape[2] > 0:
            if q_start == 0:
                q_start = k_cache.shape[2]
            k_all = torch.cat([k_cache, k], dim=2)
            v_all = torch.cat([v_cache, v], dim=2)
        else:
            k_all, v_all = k, v
        ln = log_n_table(q_start, L)[None].expand(B, L)
        out = chord_attention(q, k_all, v_all, alpha, beta, mu, ssmax, ln, q_start,
                              softmax_scale=D ** -0.5, compute_dtype=cd)
    out = out.to(hidden.dtype).transpose(1, 2).reshape(B, L, hid)
    return (out @ p['o_proj.weight'].t()) * G, k_all, v_all


def chord_prefill_flops(B, H, D, L, S=None, q_start=None):
    '''B*H*4*D*sum_i(visible keys of query i): QK^T + PV over the causal triangle.'''
    S = L if S is None else S
    q_start = S - L if q_start is None else q_start
    vis = sum(min(S, q_start + i + 1) for i in range(L))
    return 4.0 * B * H * D * vis
