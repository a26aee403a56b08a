'''Backward of the chunked gated delta rule: the HIP forward for the output and the fp32
backward of the reference's training path.

The reference differentiates its chunk rule in three pieces
(motif/ops/gated_deltanet.py): the chunk preparation `_PrepareChunksFunction.backward`
(:180-260, the triangular solve differentiated in closed form), the scan
`_FusedScanFunction.backward` (:727-765, a reverse scan kernel plus batched products) and
the per-chunk output combination (autograd through :851-855).  `GDNChunkFunction` runs
the same pieces: the two sequential scans are the HIP kernels `motif_gdn_scan_fwd_f32`
(re-scan for the per-chunk states P and residuals X) and `motif_gdn_scan_bwd_f32` (the
reverse scan), the per-chunk terms are the HIP kernels `motif_gdn_bwd_prep_f32` (the chunk factors, the
inverse by blocked substitution and the output's upstream terms) and
`motif_gdn_bwd_chunk_f32` (every gradient of the preparation, the scan products and the
output combination) for chunk 64, dk 64 and dv 64 / 128; other shapes take the same
formulas as batched fp32 torch products (`_backward_torch`).

Per chunk, with gamma the within-chunk cumulative log decay, D[i, j] = e^{gamma_i -
gamma_j} (j <= i), Kb = beta k, Vb = beta v, A = -(Kb k^T * D) strictly lower,
T = (I - A)^{-1}, W = T (Kb e^gamma), U = T Vb:
    X = U - W P,   S' = e^{gamma_C} P + (k e^{gamma_C - gamma})^T X,
    o = (q e^gamma) P + ((q k^T) * D) X.
'''
import torch
import torch.nn.functional as F

from . import _lib


def scans_serve(Dk: int, Dv: int, C: int) -> bool:
    '''True when both the HIP chunk forward (dk 32 / 64 / 128) and the two fp32 scans
    (C 16 / 32 / 64, Dv a multiple of 16) take this shape; other shapes differentiate
    through the torch form.'''
    return C in (16, 32, 64) and Dk in (32, 64, 128) and Dv % 16 == 0


def fused_scan(k, W, U, g, S0):
    '''The forward chunk scan on the HIP kernel: (P [B,H,N,Dk,Dv], S [B,H,Dk,Dv],
    X [B,H,N,C,Dv]) from chunked fp32 k, W [B,H,N,C,Dk], U [B,H,N,C,Dv], cumulative g
    [B,H,N,C] and S0 [B,H,Dk,Dv] (or None); the reference's `_fused_scan_triton`
    (motif/ops/gated_deltanet.py:644-694).'''
    B, H, N, C, Dk = k.shape
    Dv = U.shape[-1]
    k, W, U, g = (t.float().contiguous() for t in (k, W, U, g))
    S0 = None if S0 is None else S0.float().contiguous()
    P = torch.empty(B, H, N, Dk, Dv, dtype=torch.float32, device=k.device)
    X = torch.empty(B, H, N, C, Dv, dtype=torch.float32, device=k.device)
    S = torch.empty(B, H, Dk, Dv, dtype=torch.float32, device=k.device)
    rc = _lib.lib().motif_gdn_scan_fwd_f32(k.data_ptr(), W.data_ptr(), U.data_ptr(), g.data_ptr(), _lib.ptr(S0),
                                           P.data_ptr(), X.data_ptr(), S.data_ptr(), B * H, N, C, Dk, Dv,
                                           _lib.stream_ptr(k.device))
    _lib.check(rc, 'motif_gdn_scan_fwd_f32')
    return P, S, X


def bwd_scan(k, W, g, dX, dP, dS_final):
    '''The reverse chunk scan on the HIP kernel: (dSn [B,H,N,Dk,Dv], dS0 [B,H,Dk,Dv]);
    dX, dP and dS_final may be None.  The reference's `_bwd_scan`
    (motif/ops/gated_deltanet.py:558-612).'''
    B, H, N, C, Dk = k.shape
    Dv = (dS_final if dS_final is not None else dX if dX is not None else dP).shape[-1]
    k, W, g = (t.float().contiguous() for t in (k, W, g))
    dX, dP, dS_final = (None if t is None else t.float().contiguous() for t in (dX, dP, dS_final))
    dSn = torch.empty(B, H, N, Dk, Dv, dtype=torch.float32, device=k.device)
    dS0 = torch.empty(B, H, Dk, Dv, dtype=torch.float32, device=k.device)
    rc = _lib.lib().motif_gdn_scan_bwd_f32(k.data_ptr(), W.data_ptr(), g.data_ptr(), _lib.ptr(dX), _lib.ptr(dP),
                                           _lib.ptr(dS_final), dSn.data_ptr(), dS0.data_ptr(), B * H, N, C, Dk, Dv,
                                           _lib.stream_ptr(k.device))
    _lib.check(rc, 'motif_gdn_scan_bwd_f32')
    return dSn, dS0


def opscan(M, Q, S0, reverse, transpose=False):
    '''S <- M_n S + Q_n (transpose: M_n^T S + Q_n) over the chunks on the HIP kernel
    (reverse: last chunk first), recording S before each step: (rec [B,H,N,Dk,Dv],
    S_final [B,H,Dk,Dv]) from fp32 M [B,H,N,Dk,Dk], Q [B,H,N,Dk,Dv] and S0 [B,H,Dk,Dv]
    (or None: zeros).  The two scans of the reference's backward
    (motif/ops/gated_deltanet.py:327-408, :428-520) in operator form: M = A_n =
    e^{gamma_C} I - Kd_n^T W_n with Q = H_n = Kd_n^T U_n (forward, records P), M^T = A_n^T
    with Q = G_n = dP_n - W_n^T dX_n (reverse, records dSn).'''
    B, H, N, Dk, Dv = Q.shape
    M, Q = M.float().contiguous(), Q.float().contiguous()
    S0 = None if S0 is None else S0.float().contiguous()
    rec = torch.empty(B, H, N, Dk, Dv, dtype=torch.float32, device=Q.device)
    S = torch.empty(B, H, Dk, Dv, dtype=torch.float32, device=Q.device)
    rc = _lib.lib().motif_gdn_opscan_f32(M.data_ptr(), Q.data_ptr(), _lib.ptr(S0), rec.data_ptr(), S.data_ptr(),
                                         B * H, N, Dk, Dv, int(bool(reverse)), int(bool(transpose)),
                                         _lib.stream_ptr(Q.device))
    _lib.check(rc, 'motif_gdn_opscan_f32')
    return rec, S


def opscan_pair(A, Hn, S0, G, dS_final):
    '''Both operator-form scans in one HIP launch (independent of each other):
    (P, S_final) of the forward re-scan S <- A_n S + Hn_n from S0 and (dSn, dS0) of the
    reverse scan gS <- A_n^T gS + G_n from dS_final (either may be None: zeros).'''
    B, H, N, Dk, Dv = Hn.shape
    A, Hn, G = (t.float().contiguous() for t in (A, Hn, G))
    S0, dS_final = (None if t is None else t.float().contiguous() for t in (S0, dS_final))
    f = lambda *shape: torch.empty(B, H, *shape, dtype=torch.float32, device=Hn.device)
    P, S, dSn, dS0 = f(N, Dk, Dv), f(Dk, Dv), f(N, Dk, Dv), f(Dk, Dv)
    rc = _lib.lib().motif_gdn_opscan_pair_f32(A.data_ptr(), Hn.data_ptr(), _lib.ptr(S0), P.data_ptr(), S.data_ptr(),
                                              G.data_ptr(), _lib.ptr(dS_final), dSn.data_ptr(), dS0.data_ptr(),
                                              B * H, N, Dk, Dv, _lib.stream_ptr(Hn.device))
    _lib.check(rc, 'motif_gdn_opscan_pair_f32')
    return P, S, dSn, dS0


def scan_operators(kc, W, U, gam, dP, dX):
    '''The per-chunk affine operators of both scans, for all chunks at once (fp32 batched
    products): A = e^{gamma_C} I - Kd^T W, H = Kd^T U, G = dP - W^T dX, Kd = k e^{gamma_C - gamma}.'''
    gl = gam[..., -1:]
    kdT = (kc * (gl - gam).exp()[..., None]).transpose(-1, -2)
    A = torch.matmul(kdT, W).neg_()
    A.diagonal(dim1=-2, dim2=-1).add_(gl.exp())
    return A, torch.matmul(kdT, U), dP - torch.matmul(W.transpose(-1, -2), dX)


def chunk_kernels_serve(Dk: int, Dv: int, C: int) -> bool:
    '''True when the per-chunk backward kernels take this shape (chunk 64, dk 64, dv 64 or
    128); other shapes run the per-chunk terms as torch products.'''
    return C == 64 and Dk == 64 and Dv in (64, 128)


def bwd_prep(qc, kc, vc, bc, gc, doc, operators=False):
    '''Per-chunk terms before the scans on the HIP kernel, from chunked fp32 inputs
    q, k [B,H,N,C,Dk], v, do [B,H,N,C,Dv], beta, g [B,H,N,C]: (W, U, gamma, T, dP, dX), or
    with `operators` (W, U, gamma, T, dX, A, Hn, G), the scans' per-chunk operators
    A = e^{gamma_C} I - Kd^T W [B,H,N,Dk,Dk], Hn = Kd^T U and G = dP - W^T dX
    [B,H,N,Dk,Dv] in place of dP.'''
    B, H, N, C, Dk = kc.shape
    Dv = vc.shape[-1]
    dev = kc.device
    f = lambda *shape: torch.empty(B, H, N, *shape, dtype=torch.float32, device=dev)
    W, U, gam, T, dX = f(C, Dk), f(C, Dv), f(C), f(C, C), f(C, Dv)
    if operators:
        dP, A, Hn, G = None, f(Dk, Dk), f(Dk, Dv), f(Dk, Dv)
    else:
        dP, A, Hn, G = f(Dk, Dv), None, None, None
    rc = _lib.lib().motif_gdn_bwd_prep_f32(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), bc.data_ptr(),
                                           gc.data_ptr(), doc.data_ptr(), W.data_ptr(), U.data_ptr(),
                                           gam.data_ptr(), T.data_ptr(), _lib.ptr(dP), dX.data_ptr(),
                                           _lib.ptr(A), _lib.ptr(Hn), _lib.ptr(G),
                                           B * H, N, C, Dk, Dv, _lib.stream_ptr(dev))
    _lib.check(rc, 'motif_gdn_bwd_prep_f32')
    if operators:
        return W, U, gam, T, dX, A, Hn, G
    return W, U, gam, T, dP, dX


def bwd_chunk(qc, kc, vc, bc, gam, T, P, X, dSn, doc, dX, W=None, U=None):
    '''Per-chunk gradients after the scans on the HIP kernel: (dq, dk, dv, dbeta, dg),
    chunked [B,H,N,C,...] fp32.  With X None the residuals X = U - W P are formed in the
    kernel from the prep's W and U.'''
    B, H, N, C, Dk = kc.shape
    Dv = vc.shape[-1]
    dq, dk, dv = torch.empty_like(qc), torch.empty_like(kc), torch.empty_like(vc)
    dbeta, dg = torch.empty_like(bc), torch.empty_like(bc)
    rc = _lib.lib().motif_gdn_bwd_chunk_f32(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), bc.data_ptr(),
                                            gam.data_ptr(), T.data_ptr(), P.data_ptr(), _lib.ptr(X),
                                            dSn.data_ptr(), doc.data_ptr(), dX.data_ptr(), dq.data_ptr(),
                                            dk.data_ptr(), dv.data_ptr(), dbeta.data_ptr(), dg.data_ptr(),
                                            _lib.ptr(W), _lib.ptr(U), B * H, N, C, Dk, Dv, _lib.stream_ptr(kc.device))
    _lib.check(rc, 'motif_gdn_bwd_chunk_f32')
    return dq, dk, dv, dbeta, dg


def _chunks(t, C, pad):
    '''[B, H, L, ...] fp32, zero-padded to N * C steps, as [B, H, N, C, ...].'''
    t = t.float()
    if pad:
        t = F.pad(t, (0, 0, 0, pad)) if t.dim() == 4 else F.pad(t, (0, pad))
    B, H, Lp = t.shape[:3]
    return t.reshape(B, H, Lp // C, C, *t.shape[3:])


def _factors(q, k, v, beta, g, C):
    '''The chunk factors of the forward, recomputed in fp32 (the reference's
    `_PrepareChunksFunction.forward`, motif/ops/gated_deltanet.py:116-176).'''
    L = q.shape[2]
    pad = (C - L % C) % C
    qc, kc, vc = (_chunks(t, C, pad) for t in (q, k, v))
    bc, gc = _chunks(beta, C, pad), _chunks(g, C, pad).cumsum(-1)
    dev = q.device
    lower = torch.ones(C, C, dtype=torch.bool, device=dev).tril()
    strict = lower.tril(-1)
    D = (gc[..., :, None] - gc[..., None, :]).masked_fill(~lower, float('-inf')).exp()
    kb, vb = kc * bc[..., None], vc * bc[..., None]
    G1 = kb @ kc.transpose(-1, -2)
    A = (-G1 * D).masked_fill(~strict, 0.0)
    eye = torch.eye(C, device=dev, dtype=torch.float32)
    T = torch.linalg.solve_triangular(eye - A, eye.expand_as(A), upper=False, unitriangular=True)
    E = gc.exp()
    Z = kb * E[..., None]
    return dict(qc=qc, kc=kc, vc=vc, bc=bc, gc=gc, D=D, kb=kb, vb=vb, G1=G1, T=T, E=E, Z=Z,
                W=T @ Z, U=T @ vb, strict=strict, pad=pad)


class GDNChunkFunction(torch.autograd.Function):
    '''Chunked gated delta rule: HIP forward (`chunk_gated_delta_rule`'s kernels), fp32
    backward with the HIP scans.  Gradients for q, k, v, beta, g and the initial state.'''

    @staticmethod
    def forward(ctx, q, k, v, beta, g, S, C, fwd):
        o, S_out = fwd(q.detach(), k.detach(), v.detach(), beta.detach(), g.detach(),
                       None if S is None else S.detach())
        ctx.save_for_backward(q, k, v, beta, g, S)
        ctx.C = C
        return o, S_out

    @staticmethod
    def backward(ctx, do, dS_fin):
        q, k, v, beta, g, S0 = ctx.saved_tensors
        C = ctx.C
        B, H, L, Dk = q.shape
        Dv = v.shape[-1]
        if do is None:
            do = torch.zeros(B, H, L, Dv, device=q.device)
        if chunk_kernels_serve(Dk, Dv, C):
            grads = _backward_kernels(q, k, v, beta, g, S0, do, dS_fin, C)
        else:
            grads = _backward_torch(q, k, v, beta, g, S0, do, dS_fin, C)
        needs = ctx.needs_input_grad
        return tuple(gr if needs[i] else None for i, gr in enumerate(grads)) + (None, None)


def _back(t, like, L):
    '''Chunked [B, H, N, C, ...] back to [B, H, L, ...] in `like`'s dtype.'''
    B, H, N, C = t.shape[:4]
    return t.reshape(B, H, N * C, *t.shape[4:])[:, :, :L].to(like.dtype)


def _backward_kernels(q, k, v, beta, g, S0, do, dS_fin, C):
    '''The backward on the HIP kernels: per-chunk terms, forward re-scan, reverse scan,
    per-chunk gradients (four launches plus the input chunking).'''
    L = q.shape[2]
    pad = (C - L % C) % C
    qc, kc, vc, doc = (_chunks(t, C, pad).contiguous() for t in (q, k, v, do))
    bc, gc = (_chunks(t, C, pad).contiguous() for t in (beta, g))
    W, U, gam, T, dX, A, Hn, G = bwd_prep(qc, kc, vc, bc, gc, doc, operators=True)
    P, _, dSn, dS0 = opscan_pair(A, Hn, S0, G, dS_fin)
    # (the residuals X_n = U_n - W_n P_n are formed inside the per-chunk kernel)
    dq, dk, dv, dbeta, dg = bwd_chunk(qc, kc, vc, bc, gam, T, P, None, dSn, doc, dX, W=W, U=U)
    return (_back(dq, q, L), _back(dk, k, L), _back(dv, v, L), _back(dbeta, beta, L), _back(dg, g, L),
            None if S0 is None else dS0.to(S0.dtype))


def _backward_torch(q, k, v, beta, g, S0, do, dS_fin, C):
    '''The same backward with the per-chunk terms as batched fp32 torch products (shapes
    the per-chunk kernels do not take); the scans still run on the HIP kernels.'''
    B, H, L, Dk = q.shape
    f = _factors(q, k, v, beta, g, C)
    qc, kc, vc, bc, gc, D, E = f['qc'], f['kc'], f['vc'], f['bc'], f['gc'], f['D'], f['E']
    W, U, T, Z, kb, vb, G1 = f['W'], f['U'], f['T'], f['Z'], f['kb'], f['vb'], f['G1']
    N = qc.shape[2]

    # forward states and residuals
    P, _, X = fused_scan(kc, W, U, gc, S0)

    # output o = (q e^gamma) P + ((q k^T) * D) X
    doc = _chunks(do, C, f['pad'])
    qg = qc * E[..., None]
    qk = qc @ kc.transpose(-1, -2)
    attn = qk * D
    dP_out = qg.transpose(-1, -2) @ doc
    dX_out = attn.transpose(-1, -2) @ doc
    dattn = (doc @ X.transpose(-1, -2)) * D                   # zero above the diagonal
    dqg = doc @ P.transpose(-1, -2)
    dq = dqg * E[..., None] + dattn @ kc
    dk = dattn.transpose(-1, -2) @ qc
    dgam = (dqg * qg).sum(-1)                                  # d/d gamma through q e^gamma
    ddec = dattn * qk                                          # d/d D (times D already in dattn)

    # the scan: X = U - W P, S' = e^{gamma_C} P + Kd^T X
    dSn, dS0 = bwd_scan(kc, W, gc, dX_out, dP_out, dS_fin)
    gl = gc[..., -1:]
    dec = (gl - gc).exp()                                      # e^{gamma_C - gamma_c}
    dxt = dX_out + (kc @ dSn) * dec[..., None]                 # total d/dX
    dU = dxt
    dW = -(dxt @ P.transpose(-1, -2))
    dKd = X @ dSn.transpose(-1, -2)                            # [C, Dk]
    dk = dk + dKd * dec[..., None]
    kdk = (dKd * kc * dec[..., None]).sum(-1)                  # per row: dKd . Kd
    dgam = dgam - kdk
    last = kdk.sum(-1) + gl.squeeze(-1).exp() * (dSn * P).sum((-1, -2))
    dgam[..., -1] += last

    # the preparation: W = T Z, U = T Vb, T = (I - A)^{-1}, A = -(Kb k^T * D) strict
    Tt = T.transpose(-1, -2)
    dT = dW @ Z.transpose(-1, -2) + dU @ vb.transpose(-1, -2)
    dZ = Tt @ dW
    dvb = Tt @ dU
    dA = (Tt @ dT @ Tt).masked_fill(~f['strict'], 0.0)
    dG1 = -dA * D
    ddec = ddec - dA * G1 * D                                  # d/d D, times D
    dkb = dG1 @ kc + dZ * E[..., None]
    dk = dk + dG1.transpose(-1, -2) @ kb
    dgam = dgam + (dZ * Z).sum(-1) + ddec.sum(-1) - ddec.sum(-2)
    dbeta = (dkb * kc).sum(-1) + (dvb * vc).sum(-1)
    dk = dk + dkb * bc[..., None]
    dv = dvb * bc[..., None]
    dg = dgam.flip(-1).cumsum(-1).flip(-1)                     # gamma = cumsum(g)

    return (_back(dq, q, L), _back(dk, k, L), _back(dv, v, L), _back(dbeta, beta, L), _back(dg, g, L),
            None if S0 is None else dS0.to(S0.dtype))
