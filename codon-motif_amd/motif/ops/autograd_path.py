'''Differentiable torch forms of the hot-path ops, for calls that need gradients.

The HIP kernels are forward-only.  When an input requires grad (training), the op
entry points route here, as the reference's layers fall back to their torch paths
(motif/ops/gated_deltanet.py:287-321, motif/block/attention/gdn_attn.py:116-136,
motif/block/attention/chord_attn.py:316-361): the same arithmetic written with torch
ops in float32, so autograd supplies the backward.  Inference never takes this path.
'''
import math

import torch
import torch.nn.functional as F


def wants_grad(*items) -> bool:
    '''True when autograd is recording and any of `items` needs a gradient: a tensor
    that requires grad, a module with such a parameter, or a sequence holding either.
    Every kernel dispatch asks this of all its tensor inputs and parameters, since the
    kernels are forward-only.'''
    if not torch.is_grad_enabled():
        return False
    for it in items:
        if it is None:
            continue
        if isinstance(it, torch.Tensor):
            if it.requires_grad:
                return True
        elif isinstance(it, torch.nn.Module):
            if any(p.requires_grad for p in it.parameters()):
                return True
        elif isinstance(it, (list, tuple)):
            if wants_grad(*it):
                return True
    return False


def _cdt(t):
    '''Compute dtype: float32, or float64 for float64 inputs.'''
    return torch.float64 if t.dtype == torch.float64 else torch.float32


def gdn_chunk_torch(q, k, v, beta, g, S=None, chunk=64):
    '''Chunked gated delta rule (gated_deltanet.py:287-321 with :118-177).

    q, k [B, H, L, dk]; v [B, H, L, dv]; beta, g [B, H, L]; S [B, H, dk, dv] or None.
    Returns (o [B, H, L, dv] in q's dtype, S [B, H, dk, dv] in the compute dtype: float32,
    or float64 for float64 inputs).
    '''
    B, H, L, dk = q.shape
    dv = v.shape[-1]
    C = max(1, min(int(chunk), 64))
    n = (L + C - 1) // C
    pad = n * C - L
    cdt = _cdt(q)
    odt = q.dtype
    q, k, v, beta, g = (t.to(cdt) for t in (q, k, v, beta, g))
    if pad:  # zero tokens leave the state unchanged (k = 0, g = 0)
        q, k, v = (F.pad(t, (0, 0, 0, pad)) for t in (q, k, v))
        beta, g = (F.pad(t, (0, pad)) for t in (beta, g))
    q, k, v = (t.reshape(B, H, n, C, -1) for t in (q, k, v))
    beta, g = beta.reshape(B, H, n, C), g.reshape(B, H, n, C)
    gam = g.cumsum(-1)                                            # gamma within each chunk
    lower = torch.ones(C, C, dtype=torch.bool, device=q.device).tril()
    strict = lower.clone().fill_diagonal_(False)
    diff = gam[..., :, None] - gam[..., None, :]
    D = torch.where(lower, diff, torch.full_like(diff, -math.inf)).exp()        # e^{g_i - g_j}, j <= i
    Gk = (beta[..., None] * k) @ k.transpose(-1, -2)
    A = -(Gk * D).masked_fill(~strict, 0.0)
    eye = torch.eye(C, device=q.device, dtype=q.dtype)
    T = torch.linalg.solve_triangular(eye - A, eye.expand_as(A), upper=False, unitriangular=True)
    W = T @ (beta[..., None] * k * gam[..., None].exp())
    U = T @ (beta[..., None] * v)
    attn = (q @ k.transpose(-1, -2)) * D                          # causal incl. the diagonal
    qg = q * gam[..., None].exp()
    kd = k * (gam[..., -1:] - gam).exp()[..., None]
    St = torch.zeros(B, H, dk, dv, device=q.device, dtype=cdt) if S is None else S.to(cdt)
    outs = []
    for c in range(n):
        u = U[:, :, c] - W[:, :, c] @ St
        outs.append(qg[:, :, c] @ St + attn[:, :, c] @ u)
        St = St * gam[:, :, c, -1, None, None].exp() + kd[:, :, c].transpose(-1, -2) @ u
    o = torch.stack(outs, 2).reshape(B, H, n * C, dv)[:, :, :L]
    return o.to(odt), St


def short_conv_silu_torch(x, weight, cache=None, head_dim=None, scale=1.0):
    '''[cache || x] -> depthwise causal conv -> SiLU (gdn_attn.py:116-136), then the
    optional per-head L2 norm times `scale` (gdn_attn.py:190-191).  x [B, L, D],
    weight [D, 1, K], cache [B, D, K-1].  Returns (y [B, L, D], new cache).'''
    B, L, D = x.shape
    K = weight.shape[-1]
    xt = x.transpose(1, 2)
    head = cache.to(x.dtype) if cache is not None else xt.new_zeros(B, D, K - 1)
    xc = torch.cat([head, xt], -1)
    cdt = _cdt(x)
    y = F.silu(F.conv1d(xc.to(cdt), weight.reshape(D, 1, K).to(cdt), groups=D)).transpose(1, 2)
    if head_dim:
        y = F.normalize(y.reshape(B, L, D // head_dim, head_dim), dim=-1).reshape(B, L, D) * scale
    return y.to(x.dtype), xc[..., xc.shape[-1] - (K - 1):]


def chord_attention_torch(q, k, v, alpha, beta, mu, ssmax, log_n, q_start=None, softmax_scale=None, eps=1e-5):
    '''Chord attention with the gated geometric-decay bias (chord_attention.py:74-244):
    logit = (s q_i.k_j - alpha_h (|j - i_abs - mu_h| + eps)^beta_h) ssmax_h log_n[b, i],
    keys j <= i_abs = q_start + i, softmax over keys.  q [B, H, L, D], k / v
    [B, Hkv, S, D]; returns [B, H, L, D] in q's dtype.'''
    B, H, L, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    scale = D ** -0.5 if softmax_scale is None else softmax_scale
    q_start = S - L if q_start is None else int(q_start)
    cdt = _cdt(q)
    c = lambda t: t.to(cdt)
    kf = c(k).repeat_interleave(H // Hkv, dim=1)
    vf = c(v).repeat_interleave(H // Hkv, dim=1)
    i_abs = q_start + torch.arange(L, device=q.device)
    dist = c(torch.arange(S, device=q.device)[None, :] - i_abs[:, None])                 # [L, S]
    bias = -c(alpha)[:, None, None] * ((dist[None] - c(mu)[:, None, None]).abs() + eps) ** c(beta)[:, None, None]
    logits = (scale * (c(q) @ kf.transpose(-1, -2)) + bias[None]) * c(ssmax)[None, :, None, None] \
        * c(log_n)[:, None, :, None]
    visible = torch.arange(S, device=q.device)[None, :] <= i_abs[:, None]
    logits = logits.masked_fill(~visible, -math.inf)
    return (logits.softmax(-1) @ vf).to(q.dtype)


def chord_attention_varlen_torch(q, k, v, alpha, beta, mu, ssmax, log_n, cu_seqlens, softmax_scale=None, eps=1e-5):
    '''Packed-sequence Chord attention as separate differentiable runs: sequence i
    (rows cu[i]:cu[i+1] of q [1, H, T, D] / k, v [1, Hkv, T, D]) attends causally within
    itself from position 0 with its slice of log_n [1, T].'''
    cu = [int(x) for x in cu_seqlens.detach().to('cpu')]
    outs = [chord_attention_torch(q[:, :, a:b], k[:, :, a:b], v[:, :, a:b], alpha, beta, mu, ssmax,
                                  log_n[:, a:b], 0, softmax_scale, eps)
            for a, b in zip(cu[:-1], cu[1:]) if b > a]
    if not outs:
        return q.new_empty(q.shape)
    return torch.cat(outs, dim=2)
