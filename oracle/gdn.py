'''CPU restatement of the gated delta rule (GDN) path.  Test infrastructure only.

All functions take CPU tensors and compute in the dtype they are given (use
float64 to pin, float32 to time the CPU baseline).
'''
import torch
import torch.nn.functional as F


def recurrent(q, k, v, beta, g, S=None):
    '''Token-by-token gated delta rule.

    Follows motif/ops/gated_deltanet.py:26-59: per step S <- S * exp(g_t);
    v_old = k_t^T S; S <- S + k_t (beta_t (v_t - v_old))^T; o_t = S^T q_t.

    Args:
        q, k: [B, H, L, Dk];  v: [B, H, L, Dv];  beta, g: [B, H, L].
        S: optional [B, H, Dk, Dv] initial state (zeros when None).

    Returns:
        (o [B, H, L, Dv], S [B, H, Dk, Dv])
    '''
    B, H, L, Dk = q.shape
    Dv = v.shape[-1]
    if S is None:
        S = q.new_zeros(B, H, Dk, Dv)
    S = S.clone()
    outs = []
    for t in range(L):
        S = S * torch.exp(g[:, :, t])[..., None, None]
        kt = k[:, :, t]
        v_old = torch.einsum('bhk,bhkv->bhv', kt, S)
        delta = beta[:, :, t, None] * (v[:, :, t] - v_old)
        S = S + kt[..., :, None] * delta[..., None, :]
        outs.append(torch.einsum('bhk,bhkv->bhv', q[:, :, t], S))
    if L == 0:
        return q.new_zeros(B, H, 0, Dv), S
    return torch.stack(outs, dim=2), S


def chunk_factors(k, v, beta, g, C):
    '''Per-chunk WY factors of the chunked delta rule.

    Follows motif/ops/gated_deltanet.py:137-170: zero-pad L to a multiple of C,
    gamma = cumsum(g) per chunk, D_ij = exp(gamma_i - gamma_j) (j <= i, else 0),
    A = -strict_lower((beta*K) K^T * D), T = (I - A)^{-1} (unit lower),
    W = T (beta * K * exp(gamma)), U = T (beta * V).

    Returns:
        dict with gamma [B,H,N,C], D [B,H,N,C,C], T, W [B,H,N,C,Dk],
        U [B,H,N,C,Dv], kc [B,H,N,C,Dk], pad, N.
    '''
    B, H, L, Dk = k.shape
    Dv = v.shape[-1]
    pad = (C - L % C) % C
    if pad:
        k = F.pad(k, (0, 0, 0, pad))
        v = F.pad(v, (0, 0, 0, pad))
        beta = F.pad(beta, (0, pad))
        g = F.pad(g, (0, pad))
    N = (L + pad) // C
    kc = k.reshape(B, H, N, C, Dk)
    vc = v.reshape(B, H, N, C, Dv)
    bc = beta.reshape(B, H, N, C)
    gamma = g.reshape(B, H, N, C).cumsum(-1)
    tril = torch.ones(C, C, dtype=torch.bool).tril()
    strict = torch.ones(C, C, dtype=torch.bool).tril(-1)
    D = (gamma[..., :, None] - gamma[..., None, :]).masked_fill(~tril, float('-inf')).exp()
    G1 = (kc * bc[..., None]) @ kc.transpose(-1, -2)
    A = (-G1 * D).masked_fill(~strict, 0.0)
    eye = torch.eye(C, dtype=k.dtype)
    T = torch.linalg.solve_triangular(eye - A, eye.expand_as(A).contiguous(),
                                      upper=False, unitriangular=True)
    W = T @ (kc * bc[..., None] * gamma.exp()[..., None])
    U = T @ (vc * bc[..., None])
    return dict(gamma=gamma, D=D, A=A, T=T, W=W, U=U, kc=kc, pad=pad, N=N)


def chunked(q, k, v, beta, g, S=None, chunk_size=64):
    '''Chunked gated delta rule (the reference's pure-torch CPU path).

    Follows motif/ops/gated_deltanet.py:287-321 (loop over chunks:
    u = U_n - W_n S; o = (q*e^gamma) S + ((q k^T) * D) u;
    S <- S e^{gamma_C} + (k * e^{gamma_C - gamma})^T u), output sliced to L.
    '''
    B, H, L, Dk = q.shape
    Dv = v.shape[-1]
    C = chunk_size
    f = chunk_factors(k, v, beta, g, C)
    N, pad = f['N'], f['pad']
    qp = F.pad(q, (0, 0, 0, pad)) if pad else q
    qc = qp.reshape(B, H, N, C, Dk)
    if S is None:
        S = q.new_zeros(B, H, Dk, Dv)
    o = q.new_empty(B, H, N, C, Dv)
    for n in range(N):
        qi, ki, gi = qc[:, :, n], f['kc'][:, :, n], f['gamma'][:, :, n]
        attn = (qi @ ki.transpose(-1, -2)) * f['D'][:, :, n]
        u = f['U'][:, :, n] - f['W'][:, :, n] @ S
        o[:, :, n] = (qi * gi.exp()[..., None]) @ S + attn @ u
        S = S * gi[:, :, -1].exp()[..., None, None] + \
            (ki * (gi[:, :, -1:] - gi).exp()[..., None]).transpose(-1, -2) @ u
    return o.reshape(B, H, N * C, Dv)[:, :, :L], S


def _split_varlen(x, cu_seqlens, dim):
    cu = [int(c) for c in cu_seqlens]
    return [x.narrow(dim, cu[i], cu[i + 1] - cu[i]) for i in range(len(cu) - 1)]


def chunked_varlen(q, k, v, beta, g, cu_seqlens, S=None, chunk_size=64):
    '''Packed-sequence gated delta rule: B == 1, sequences concatenated on L.

    New capability (no reference counterpart): defined as an independent
    `chunked` run per sequence from its own initial state (zeros, or S[i]),
    outputs concatenated on L; final states stacked as [nseq, H, Dk, Dv].
    '''
    nseq = len(cu_seqlens) - 1
    outs, states = [], []
    qs, ks, vs = (_split_varlen(t, cu_seqlens, 2) for t in (q, k, v))
    bs, gs = (_split_varlen(t, cu_seqlens, 2) for t in (beta, g))
    for i in range(nseq):
        s0 = None if S is None else S[i:i + 1]
        o, s = chunked(qs[i], ks[i], vs[i], bs[i], gs[i], s0, chunk_size)
        outs.append(o)
        states.append(s[0])
    return torch.cat(outs, dim=2), torch.stack(states, 0)


def short_conv_silu(x, weight, cache=None):
    '''Short causal depthwise conv followed by SiLU.

    Follows motif/block/attention/gdn_attn.py:116-136: xc = [cache || x] along
    time (cache = zeros when None), y = SiLU(conv1d(xc, groups=D)), new cache =
    the last K-1 *pre-activation inputs* of xc.

    Args:
        x: [B, L, D];  weight: [D, 1, K] (nn.Conv1d layout);  cache: [B, D, K-1].

    Returns:
        (y [B, L, D], new_cache [B, D, K-1])
    '''
    B, L, D = x.shape
    K = weight.shape[-1]
    xt = x.transpose(1, 2)
    if cache is None:
        cache = xt.new_zeros(B, D, K - 1)
    xc = torch.cat([cache, xt], dim=-1)
    new_cache = xc[..., -(K - 1):]
    if L == 0:
        return x.new_zeros(B, 0, D), new_cache
    y = F.silu(F.conv1d(xc, weight, groups=D))
    return y.transpose(1, 2), new_cache


def short_conv_silu_varlen(x, weight, cu_seqlens):
    '''Packed short conv: every sequence starts from a zero tail (B == 1).'''
    ys, tails = [], []
    for xs in _split_varlen(x, cu_seqlens, 1):
        y, t = short_conv_silu(xs, weight, None)
        ys.append(y)
        tails.append(t[0])
    return torch.cat(ys, dim=1), torch.stack(tails, 0)


def rms_norm(x, weight, eps=1e-6):
    '''Eager RMSNorm: motif/ops/rms_norm.py:481-486 (normalise in fp32, cast, scale).'''
    xf = x.float() if x.dtype in (torch.float16, torch.bfloat16) else x
    y = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)
    return y * weight if weight is not None else y


def gated_rms_norm(x, weight, dim, eps=1e-6):
    '''Eager GatedRMSNorm: motif/ops/rms_norm.py:548-553 (values || gate halves).'''
    x_in, gate = x.split(dim, dim=-1)
    return rms_norm(x_in, weight, eps) * F.silu(gate)


def gdn_gates(hidden, p):
    '''beta and log-decay g of a GDN layer: motif/block/attention/gdn_attn.py:193-195.

    beta = sigmoid(b_proj h);  g = -exp(A_log) * softplus(a_proj h + dt_bias).
    Returns [B, H, L] tensors.
    '''
    beta = torch.sigmoid(hidden @ p['b_proj.weight'].t()).transpose(1, 2)
    g = -p['A_log'].exp() * F.softplus(hidden @ p['a_proj.weight'].t() + p['dt_bias'])
    return beta, g.transpose(1, 2)


def gdn_layer(hidden, p, num_heads, dk, dv, state=None, conv_state=None,
              chunk_size=64, cu_seqlens=None):
    '''GatedDeltaAttention.forward, restated: motif/block/attention/gdn_attn.py:138-219.

    q/k/v projections -> short conv + SiLU (:183-185) -> per-head L2 normalise,
    q scaled by dk^-1/2 (:187-191) -> beta, g (:193-195) -> delta rule in fp32
    (:197-204; the recurrence for L == 1, chunked otherwise) -> cast back
    (:206) -> GatedRMSNorm over [o || g_proj h] per head (:207-209) -> o_proj.

    Args:
        hidden: [B, L, hidden] (any float dtype; the recurrence runs in fp32 or
            fp64 when hidden is fp64).
        p: dict of parameters named like the reference module's state_dict.
        cu_seqlens: optional packed-sequence boundaries (B == 1); every sequence
            then starts from zero state and zero conv tails.

    Returns:
        (output [B, L, hidden], state [B|nseq, H, dk, dv], (cq, ck, cv))
    '''
    B, L, _ = hidden.shape
    cdt = torch.float64 if hidden.dtype == torch.float64 else torch.float32
    tails = conv_state if conv_state is not None else (None, None, None)
    xs = [hidden @ p[f'{n}_proj.weight'].t() for n in ('q', 'k', 'v')]
    ws = [p[f'{n}_conv.weight'] for n in ('q', 'k', 'v')]
    if cu_seqlens is None:
        outs = [short_conv_silu(x, w, c) for x, w, c in zip(xs, ws, tails)]
    else:
        outs = [short_conv_silu_varlen(x, w, cu_seqlens) for x, w in zip(xs, ws)]
    (q, cq), (k, ck), (v, cv) = outs
    q = q.view(B, L, num_heads, dk).transpose(1, 2)
    k = k.view(B, L, num_heads, dk).transpose(1, 2)
    v = v.view(B, L, num_heads, dv).transpose(1, 2)
    q = F.normalize(q, dim=-1) * (dk ** -0.5)
    k = F.normalize(k, dim=-1)
    beta, g = gdn_gates(hidden, p)
    qf, kf, vf, bf, gf = (t.to(cdt) for t in (q, k, v, beta, g))
    S0 = None if state is None else state.to(cdt)
    if cu_seqlens is not None:
        o, S = chunked_varlen(qf, kf, vf, bf, gf, cu_seqlens, S0, chunk_size)
    elif L == 1:
        o, S = recurrent(qf, kf, vf, bf, gf, S0)
    else:
        o, S = chunked(qf, kf, vf, bf, gf, S0, chunk_size)
    o = o.to(hidden.dtype).transpose(1, 2)
    gate = (hidden @ p['g_proj.weight'].t()).view(B, L, num_heads, dv)
    o = gated_rms_norm(torch.cat([o, gate.to(o.dtype)], dim=-1), p['o_norm.weight'], dv)
    return o.reshape(B, L, -1) @ p['o_proj.weight'].t(), S, (cq, ck, cv)


def gdn_prefill_flops(B, T, H, dk, dv, C=64):
    '''Algorithmic flop count of a GDN prefill (the measurement convention).

    B*T*H*[2C(3dk+2dv) + 6*dk*dv + C^2/3]: K K^T, Q K^T, T Z (2C*dk each),
    T (beta V) and attn X (2C*dv each), W S, Q S, K~^T X (2 dk dv each) and the
    triangular inverse (C^2/3).
    '''
    return B * T * H * (2 * C * (3 * dk + 2 * dv) + 6 * dk * dv + C * C / 3.0)

