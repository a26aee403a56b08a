'''GPU parity of the GDN backward: the fp32 chunk scans (motif_gdn_scan_fwd_f32 /
motif_gdn_scan_bwd_f32 through the C ABI) against their defining loops in float64 on
the CPU, and the gradients of `chunk_gated_delta_rule` (GDNChunkFunction) against
autograd through the differentiable torch form (motif/ops/autograd_path.py, whose
gradients tests/test_autograd_path.py pins with gradcheck) in float64.

Bars: the scans are fp32 products of 64..128 terms: max-abs within 1e-4 of the largest
reference entry.  Gradients: the backward computes in fp32 from the same inputs, so
max-abs within 2e-3 of the largest reference entry and mean-relative 1e-3 (the
triangular solve and the per-chunk sums of the decay gradient cancel, which costs a
few fp32 ulps of the largest terms); for bf16 inputs the gradients come back in bf16
(one rounding of 2^-9 relative), so 1e-2 and 5e-3.'''
import pytest
import torch

from support import gdn_inputs

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _scan_fwd_ref(k, W, U, g, S0):
    B, H, N, C, Dk = k.shape
    P, X, S = [], [], S0.clone()
    for n in range(N):
        P.append(S)
        gl = g[:, :, n, -1:]
        kd = k[:, :, n] * (gl - g[:, :, n]).exp()[..., None]
        x = U[:, :, n] - W[:, :, n] @ S
        X.append(x)
        S = gl.exp()[..., None] * S + kd.transpose(-1, -2) @ x
    return torch.stack(P, 2), S, torch.stack(X, 2)


def _scan_bwd_ref(k, W, g, dX, dP, dS):
    B, H, N, C, Dk = k.shape
    dSn = [None] * N
    for n in range(N - 1, -1, -1):
        dSn[n] = dS
        gl = g[:, :, n, -1:]
        kd = k[:, :, n] * (gl - g[:, :, n]).exp()[..., None]
        dx = kd @ dS + dX[:, :, n]
        dS = gl.exp()[..., None] * dS - W[:, :, n].transpose(-1, -2) @ dx + dP[:, :, n]
    return torch.stack(dSn, 2), dS


def _close(got, ref, what, rel=1e-4, mean_rel=None):
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    d = (got - ref).abs()
    scale = ref.abs().max().item()
    mr = d.sum().item() / max(ref.abs().sum().item(), 1e-30)
    print(f'{what}: max_abs={d.max().item():.3e} (of {scale:.3e}) mean_rel={mr:.3e}', flush=True)
    assert d.max().item() <= rel * max(scale, 1e-6), what
    if mean_rel is not None:
        assert mr <= mean_rel, what


@pytest.mark.parametrize('N,C,Dk,Dv', [(5, 64, 64, 128), (3, 32, 128, 32), (4, 16, 16, 16)])
def test_scans_match_loops(N, C, Dk, Dv):
    from motif.ops.gdn_grad import bwd_scan, fused_scan
    g0 = torch.Generator().manual_seed(N * 7 + C)
    B, H = 2, 3
    k = torch.nn.functional.normalize(torch.randn(B, H, N, C, Dk, generator=g0), dim=-1)
    W = torch.randn(B, H, N, C, Dk, generator=g0) * 0.2
    U = torch.randn(B, H, N, C, Dv, generator=g0)
    g = torch.nn.functional.logsigmoid(torch.randn(B, H, N, C, generator=g0)).cumsum(-1) * 0.2
    S0 = torch.randn(B, H, Dk, Dv, generator=g0) * 0.3
    P, S, X = fused_scan(*(t.to(DEV) for t in (k, W, U, g, S0)))
    rP, rS, rX = _scan_fwd_ref(*(t.double() for t in (k, W, U, g, S0)))
    _close(P, rP, 'P')
    _close(S, rS, 'S')
    _close(X, rX, 'X')
    dX = torch.randn(B, H, N, C, Dv, generator=g0)
    dP = torch.randn(B, H, N, Dk, Dv, generator=g0) * 0.1
    dS = torch.randn(B, H, Dk, Dv, generator=g0)
    dSn, dS0 = bwd_scan(*(t.to(DEV) for t in (k, W, g, dX, dP, dS)))
    rdSn, rdS0 = _scan_bwd_ref(*(t.double() for t in (k, W, g, dX, dP, dS)))
    _close(dSn, rdSn, 'dSn')
    _close(dS0, rdS0, 'dS0')


@pytest.mark.parametrize('N,Dk,Dv', [(5, 64, 128), (64, 64, 128), (1, 64, 64), (3, 32, 48), (2, 16, 16)])
def test_operator_scans_match_loops(N, Dk, Dv):
    '''The operator-form scans (motif_gdn_opscan_f32 with the per-chunk operators formed
    beforehand) against the same defining loops as the direct scans.'''
    from motif.ops.gdn_grad import opscan, opscan_pair, scan_operators
    g0 = torch.Generator().manual_seed(N * 11 + Dv)
    B, H, C = 2, 3, 64
    k = torch.nn.functional.normalize(torch.randn(B, H, N, C, Dk, generator=g0), dim=-1)
    W = torch.randn(B, H, N, C, Dk, generator=g0) * 0.2
    U = torch.randn(B, H, N, C, Dv, generator=g0)
    g = torch.nn.functional.logsigmoid(torch.randn(B, H, N, C, generator=g0)).cumsum(-1) * 0.2
    S0 = torch.randn(B, H, Dk, Dv, generator=g0) * 0.3
    dX = torch.randn(B, H, N, C, Dv, generator=g0)
    dP = torch.randn(B, H, N, Dk, Dv, generator=g0) * 0.1
    dS = torch.randn(B, H, Dk, Dv, generator=g0)
    kd, Wd, Ud, gd, dPd, dXd = (t.to(DEV) for t in (k, W, U, g, dP, dX))
    A, Hn, G = scan_operators(kd, Wd, Ud, gd, dPd, dXd)
    P, S = opscan(A, Hn, S0.to(DEV), reverse=False)
    X = Ud - torch.matmul(Wd, P)
    rP, rS, rX = _scan_fwd_ref(*(t.double() for t in (k, W, U, g, S0)))
    _close(P, rP, 'P')
    _close(S, rS, 'S')
    _close(X, rX, 'X')
    dSn, dS0 = opscan(A, G, dS.to(DEV), reverse=True, transpose=True)
    dSn2, _ = opscan(A.transpose(-1, -2), G, dS.to(DEV), reverse=True)
    _close(dSn2, dSn, 'dSn (transposed operand handed in)')
    rdSn, rdS0 = _scan_bwd_ref(*(t.double() for t in (k, W, g, dX, dP, dS)))
    _close(dSn, rdSn, 'dSn')
    _close(dS0, rdS0, 'dS0')
    P2, S2, dSn3, dS03 = opscan_pair(A, Hn, S0.to(DEV), G, dS.to(DEV))   # both scans in one launch
    for name, x, y in (('P', P2, P), ('S', S2, S), ('dSn', dSn3, dSn), ('dS0', dS03, dS0)):
        assert torch.equal(x, y), name
    P0, S00 = opscan(A, Hn, None, reverse=False)   # zero initial state
    rP0, rS00, _ = _scan_fwd_ref(*(t.double() for t in (k, W, U, g, torch.zeros_like(S0))))
    _close(P0, rP0, 'P (S0 = 0)')
    _close(S00, rS00, 'S (S0 = 0)')



def _grads(fn, q, k, v, b, g, S0, do, dS, dev, dtype):
    ts = [t.to(dev, dtype).requires_grad_(True) for t in (q, k, v, b, g)]
    s0 = S0.to(dev, torch.float64 if dtype == torch.float64 else torch.float32).requires_grad_(True)
    o, S = fn(*ts, s0)
    loss = (o.to(do.dtype) * do.to(dev)).sum() + (S.to(dS.dtype) * dS.to(dev)).sum()
    loss.backward()
    return o.detach(), S.detach(), [t.grad for t in ts] + [s0.grad]


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
# dk = 16 / 48: head sizes the HIP chunk forward does not take, differentiated through the
# torch form on the device
@pytest.mark.parametrize('B,H,L,dk,dv,C', [(2, 3, 200, 64, 128, 64), (1, 2, 77, 32, 64, 32),
                                           (1, 2, 90, 16, 32, 64), (1, 1, 70, 48, 16, 16)])
def test_chunk_rule_gradients_match_torch_form(dtype, B, H, L, dk, dv, C):
    from motif.ops import chunk_gated_delta_rule
    from motif.ops.autograd_path import gdn_chunk_torch
    q, k, v, b, g = gdn_inputs(B, H, L, dk, dv, seed=L + dk, dtype=dtype)
    g0 = torch.Generator().manual_seed(L)
    S0 = torch.randn(B, H, dk, dv, generator=g0) * 0.1
    do = torch.randn(B, H, L, dv, generator=g0, dtype=torch.float64)
    dS = torch.randn(B, H, dk, dv, generator=g0, dtype=torch.float64) * 0.1
    ro, rS, rg = _grads(lambda *a: gdn_chunk_torch(*a, chunk=C), q, k, v, b, g, S0, do, dS, 'cpu', torch.float64)
    go, gS, gg = _grads(lambda *a: chunk_gated_delta_rule(*a, chunk_size=C), q, k, v, b, g, S0, do, dS, DEV, dtype)
    _close(go, ro, 'o', 2e-2 if dtype == torch.bfloat16 else 1e-4)
    bars = (1e-2, 5e-3) if dtype == torch.bfloat16 else (2e-3, 1e-3)   # bf16: gradients rounded to bf16
    for name, got, ref in zip(('dq', 'dk', 'dv', 'dbeta', 'dg', 'dS0'), gg, rg):
        _close(got, ref, name, *bars)


def test_only_state_output_used():
    '''A loss on the final state alone (no output gradient) still reaches every input.'''
    from motif.ops import chunk_gated_delta_rule
    q, k, v, b, g = (t.to(DEV).requires_grad_(True) for t in gdn_inputs(1, 2, 70, 64, 64, seed=4))
    _, S = chunk_gated_delta_rule(q, k, v, b, g)
    S.square().sum().backward()
    for t in (q, k, v, b, g):
        assert t.grad is not None and torch.isfinite(t.grad).all()
    assert q.grad.abs().max().item() == 0.0   # the state does not depend on q


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_varlen_gradients_match_torch_form(dtype):
    '''Packed sequences with gradients (each non-empty sequence through
    GDNChunkFunction) against the per-sequence torch form in float64.'''
    from motif.ops import chunk_gated_delta_rule_varlen
    from motif.ops.autograd_path import gdn_chunk_torch
    lens = [70, 0, 5, 130]
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    T = sum(lens)
    q, k, v, b, g = gdn_inputs(1, 2, T, 64, 64, seed=31, dtype=dtype)
    g0 = torch.Generator().manual_seed(5)
    S0 = torch.randn(len(lens), 2, 64, 64, generator=g0) * 0.1
    do = torch.randn(1, 2, T, 64, generator=g0, dtype=torch.float64)
    dS = torch.randn(len(lens), 2, 64, 64, generator=g0, dtype=torch.float64) * 0.1

    def ref_fn(q_, k_, v_, b_, g_, s_):
        outs, sts = [], []
        for i in range(len(lens)):
            sl = slice(int(cu[i]), int(cu[i + 1]))
            if sl.stop == sl.start:   # an empty sequence keeps its state
                o_i, s_i = q_.new_empty(1, 2, 0, 64), s_[i:i + 1]
            else:
                o_i, s_i = gdn_chunk_torch(q_[:, :, sl], k_[:, :, sl], v_[:, :, sl], b_[:, :, sl], g_[:, :, sl],
                                           s_[i:i + 1], 64)
            outs.append(o_i)
            sts.append(s_i)
        return torch.cat(outs, 2), torch.cat(sts, 0)

    ro, rS, rg = _grads(ref_fn, q, k, v, b, g, S0, do, dS, 'cpu', torch.float64)
    go, gS, gg = _grads(lambda *a: chunk_gated_delta_rule_varlen(*a[:5], cu.to(DEV), S=a[5]),
                        q, k, v, b, g, S0, do, dS, DEV, dtype)
    _close(go, ro, 'o', 2e-2 if dtype == torch.bfloat16 else 1e-4)
    bars = (1e-2, 5e-3) if dtype == torch.bfloat16 else (2e-3, 1e-3)
    for name, got, ref in zip(('dq', 'dk', 'dv', 'dbeta', 'dg', 'dS0'), gg, rg):
        _close(got, ref, name, *bars)


def test_varlen_gradient_branch_validates_cu_seqlens():
    '''The packed form checks B, S and cu_seqlens before choosing its gradient or
    no-gradient branch, with the same errors either way.'''
    from motif.ops import chunk_gated_delta_rule_varlen
    q, k, v, b, g = (t.to(DEV) for t in gdn_inputs(1, 2, 50, 64, 64, seed=9))
    for grad in (False, True):
        ts = [t.clone().requires_grad_(grad) for t in (q, k, v, b, g)]
        for cu in ([0, 20, 40], [5, 20, 50], [0, 30, 20, 50]):
            with pytest.raises(ValueError, match='cu_seqlens'):
                chunk_gated_delta_rule_varlen(*ts, torch.tensor(cu, dtype=torch.int32, device=DEV))
        with pytest.raises(ValueError, match='S must be'):
            chunk_gated_delta_rule_varlen(*ts, torch.tensor([0, 50], dtype=torch.int32, device=DEV),
                                          S=torch.zeros(2, 2, 64, 64, device=DEV))
        q2 = torch.cat([ts[0]] * 2)
        with pytest.raises(ValueError, match='B == 1'):
            chunk_gated_delta_rule_varlen(q2, torch.cat([ts[1]] * 2), torch.cat([ts[2]] * 2),
                                          torch.cat([ts[3]] * 2), torch.cat([ts[4]] * 2),
                                          torch.tensor([0, 50], dtype=torch.int32, device=DEV))


@pytest.mark.parametrize('B,H,L,dv', [(1, 2, 64, 64), (2, 3, 200, 128), (1, 12, 1000, 128)])
def test_chunk_kernels_equal_torch_products(B, H, L, dv):
    '''The per-chunk backward kernels (motif_gdn_bwd_prep_f32 / motif_gdn_bwd_chunk_f32)
    against the same backward with the per-chunk terms as fp32 torch products, on the
    same inputs: both fp32, so within 1e-4 of the largest entry.'''
    from motif.ops.gdn_grad import _backward_kernels, _backward_torch, chunk_kernels_serve
    assert chunk_kernels_serve(64, dv, 64)
    q, k, v, b, g = (t.to(DEV) for t in gdn_inputs(B, H, L, 64, dv, seed=L + dv))
    g0 = torch.Generator().manual_seed(L)
    S0 = (torch.randn(B, H, 64, dv, generator=g0) * 0.1).to(DEV)
    do = torch.randn(B, H, L, dv, generator=g0).to(DEV)
    dS = (torch.randn(B, H, 64, dv, generator=g0) * 0.1).to(DEV)
    got = _backward_kernels(q, k, v, b, g, S0, do, dS, 64)
    ref = _backward_torch(q, k, v, b, g, S0, do, dS, 64)
    for name, x, y in zip(('dq', 'dk', 'dv', 'dbeta', 'dg', 'dS0'), got, ref):
        assert x.shape == y.shape, name
        _close(x, y, f'{name} (B={B} H={H} L={L} dv={dv})', 1e-4)


@pytest.mark.parametrize('dv', [64, 128])
def test_prep_scan_operators_equal_torch_products(dv):
    '''The backward prep kernel's scan operators (A, Hn, G) against the same operators
    formed from its other outputs by fp32 torch products (scan_operators), and its W, U,
    gamma, T, dX unchanged by asking for them.'''
    from motif.ops.gdn_grad import _chunks, bwd_prep, scan_operators
    B, H, L = 1, 3, 300
    q, k, v, b, g = (t.to(DEV) for t in gdn_inputs(B, H, L, 64, dv, seed=dv))
    do = torch.randn(B, H, L, dv, generator=torch.Generator().manual_seed(dv)).to(DEV)
    pad = (64 - L % 64) % 64
    qc, kc, vc, doc = (_chunks(t, 64, pad).contiguous() for t in (q, k, v, do))
    bc, gc = (_chunks(t, 64, pad).contiguous() for t in (b, g))
    W, U, gam, T, dP, dX = bwd_prep(qc, kc, vc, bc, gc, doc)
    W2, U2, gam2, T2, dX2, A, Hn, G = bwd_prep(qc, kc, vc, bc, gc, doc, operators=True)
    for name, x, y in (('W', W2, W), ('U', U2, U), ('gam', gam2, gam), ('T', T2, T), ('dX', dX2, dX)):
        assert torch.equal(x, y), name
    rA, rH, rG = scan_operators(kc, W, U, gam, dP, dX)
    _close(A, rA, 'A', 1e-5)
    _close(Hn, rH, 'Hn', 1e-5)
    _close(G, rG, 'G', 1e-5)


def test_chunk_kernel_forms_residuals_itself():
    '''The per-chunk gradient kernel given the residuals X = U - W P against the same kernel
    forming them from W, U and P itself: equal up to the fp32 rounding of X.'''
    from motif.ops.gdn_grad import _chunks, bwd_chunk, bwd_prep, opscan_pair
    B, H, L, dv = 1, 2, 250, 128
    q, k, v, b, g = (t.to(DEV) for t in gdn_inputs(B, H, L, 64, dv, seed=5))
    g0 = torch.Generator().manual_seed(5)
    do = torch.randn(B, H, L, dv, generator=g0).to(DEV)
    S0 = (torch.randn(B, H, 64, dv, generator=g0) * 0.1).to(DEV)
    dS = (torch.randn(B, H, 64, dv, generator=g0) * 0.1).to(DEV)
    pad = (64 - L % 64) % 64
    qc, kc, vc, doc = (_chunks(t, 64, pad).contiguous() for t in (q, k, v, do))
    bc, gc = (_chunks(t, 64, pad).contiguous() for t in (b, g))
    W, U, gam, T, dX, A, Hn, G = bwd_prep(qc, kc, vc, bc, gc, doc, operators=True)
    P, _, dSn, _ = opscan_pair(A, Hn, S0, G, dS)
    X = U - torch.matmul(W, P)
    given = bwd_chunk(qc, kc, vc, bc, gam, T, P, X, dSn, doc, dX)
    formed = bwd_chunk(qc, kc, vc, bc, gam, T, P, None, dSn, doc, dX, W=W, U=U)
    for name, x, y in zip(('dq', 'dk', 'dv', 'dbeta', 'dg'), formed, given):
        _close(x, y, name, 1e-5)
