'''Pins for the GDN oracle (CPU, float64).

Each check is chosen so that a plausible mistake in the restatement fails it:
closed-form special cases of the recurrence, an independent matrix-product
statement of one step, chunked == recurrent for several chunk lengths and
ragged lengths (different algorithms), the triangular inverse against SciPy,
and the conv against a scalar loop.
'''
import math

import pytest
import scipy.linalg
import torch
import torch.nn.functional as F

from oracle import gdn
from support import gdn_inputs

D64 = torch.float64


def _inputs(B=2, H=3, T=37, dk=16, dv=24, seed=0):
    return [t.double() for t in gdn_inputs(B, H, T, dk, dv, seed=seed)]


def test_beta_zero_keeps_state_decayed():
    '''beta = 0: S_t = exp(sum g) S0 and o_t = q_t^T S_t (no writes).'''
    q, k, v, b, g = _inputs()
    S0 = torch.randn(2, 3, 16, 24, dtype=D64)
    o, S = gdn.recurrent(q, k, v, torch.zeros_like(b), g, S0)
    cum = g.cumsum(-1)
    expect_o = torch.einsum('bhtk,bhkv->bhtv', q, S0) * cum.exp()[..., None]
    assert torch.allclose(o, expect_o, atol=1e-12)
    assert torch.allclose(S, S0 * cum[..., -1].exp()[..., None, None], atol=1e-12)


def test_reset_with_very_negative_gate():
    '''g_t = -inf (exp -> 0) erases the history: the run restarts at step t.'''
    q, k, v, b, g = _inputs(T=20)
    g2 = g.clone()
    g2[:, :, 9] = -1e4
    o, S = gdn.recurrent(q, k, v, b, g2)
    o_tail, S_tail = gdn.recurrent(q[:, :, 9:], k[:, :, 9:], v[:, :, 9:], b[:, :, 9:],
                                   torch.cat([torch.zeros_like(g2[:, :, 9:10]), g2[:, :, 10:]], -1))
    assert torch.allclose(o[:, :, 9:], o_tail, atol=1e-12)
    assert torch.allclose(S, S_tail, atol=1e-12)


def test_single_token_outer_product():
    '''One token from zero state with g = 0, beta = 1: S = k v^T and o = (q.k) v.'''
    q, k, v, b, g = _inputs(T=1)
    o, S = gdn.recurrent(q, k, v, torch.ones_like(b), torch.zeros_like(g))
    assert torch.allclose(S, k[:, :, 0, :, None] * v[:, :, 0, None, :], atol=1e-14)
    assert torch.allclose(o[:, :, 0], (q[:, :, 0] * k[:, :, 0]).sum(-1, keepdim=True) * v[:, :, 0], atol=1e-14)


def test_orthonormal_keys_overwrite_exactly():
    '''beta = 1, g = 0 and orthonormal keys: after the run S^T k_t = v_t for every t.'''
    dk, dv, T = 16, 8, 10
    Q, _ = torch.linalg.qr(torch.randn(dk, dk, dtype=D64))
    k = Q[:T].reshape(1, 1, T, dk)
    v = torch.randn(1, 1, T, dv, dtype=D64)
    q = torch.randn(1, 1, T, dk, dtype=D64)
    _, S = gdn.recurrent(q, k, v, torch.ones(1, 1, T, dtype=D64), torch.zeros(1, 1, T, dtype=D64))
    assert torch.allclose(torch.einsum('tk,kv->tv', k[0, 0], S[0, 0]), v[0, 0], atol=1e-12)


def test_step_as_householder_like_product():
    '''Independent statement of one step: S_t = (I - b k k^T) e^g S_{t-1} + b k v^T.'''
    q, k, v, b, g = _inputs(B=1, H=1, T=6)
    S = torch.randn(16, 24, dtype=D64)
    S_ref = S.clone()
    for t in range(6):
        kt, vt, bt, gt = k[0, 0, t], v[0, 0, t], b[0, 0, t], g[0, 0, t]
        S_ref = (torch.eye(16, dtype=D64) - bt * torch.outer(kt, kt)) @ (gt.exp() * S_ref) + bt * torch.outer(kt, vt)
    _, S_out = gdn.recurrent(q, k, v, b, g, S[None, None])
    assert torch.allclose(S_out[0, 0], S_ref, atol=1e-12)


@pytest.mark.parametrize('C', [16, 32, 64])
@pytest.mark.parametrize('T', [1, 15, 64, 100, 200])
def test_chunked_equals_recurrent(C, T):
    q, k, v, b, g = _inputs(T=T, dk=32, dv=48, seed=T)
    S0 = torch.randn(2, 3, 32, 48, dtype=D64) * 0.3
    o_r, S_r = gdn.recurrent(q, k, v, b, g, S0)
    o_c, S_c = gdn.chunked(q, k, v, b, g, S0, C)
    assert torch.allclose(o_c, o_r, atol=1e-10)
    assert torch.allclose(S_c, S_r, atol=1e-10)


def test_chunk_inverse_matches_scipy():
    q, k, v, b, g = _inputs(B=1, H=1, T=64, dk=32, dv=8)
    f = gdn.chunk_factors(k, v, b, g, 64)
    M = (torch.eye(64, dtype=D64) - f['A'][0, 0, 0]).numpy()
    T_ref = scipy.linalg.solve_triangular(M, torch.eye(64, dtype=D64).numpy(), lower=True, unit_diagonal=True)
    assert torch.allclose(f['T'][0, 0, 0], torch.from_numpy(T_ref), atol=1e-12)
    assert torch.count_nonzero(torch.triu(f['A'][0, 0, 0])) == 0


def test_varlen_equals_separate_runs():
    lens = [5, 0, 70, 1]
    cu = torch.tensor([0, 5, 5, 75, 76])
    q, k, v, b, g = _inputs(B=1, H=2, T=76, dk=16, dv=16)
    o, S = gdn.chunked_varlen(q, k, v, b, g, cu, None, 32)
    start = 0
    for i, n in enumerate(lens):
        sl = slice(start, start + n)
        o_i, S_i = gdn.recurrent(q[:, :, sl], k[:, :, sl], v[:, :, sl], b[:, :, sl], g[:, :, sl])
        assert torch.allclose(o[:, :, sl], o_i, atol=1e-10)
        assert torch.allclose(S[i], S_i[0], atol=1e-10)
        start += n


@pytest.mark.parametrize('with_cache', [False, True])
def test_short_conv_against_scalar_loop(with_cache):
    B, L, D, K = 2, 9, 5, 4
    x = torch.randn(B, L, D, dtype=D64)
    w = torch.randn(D, 1, K, dtype=D64)
    cache = torch.randn(B, D, K - 1, dtype=D64) if with_cache else None
    y, nc = gdn.short_conv_silu(x, w, cache)
    for bb in range(B):
        for d in range(D):
            seq = ([0.0] * (K - 1) if cache is None else cache[bb, d].tolist()) + x[bb, :, d].tolist()
            for t in range(L):
                acc = sum(w[d, 0, r].item() * seq[t + r] for r in range(K))
                assert abs(y[bb, t, d].item() - acc / (1 + math.exp(-acc))) < 1e-12
            assert nc[bb, d].tolist() == seq[-(K - 1):]


def test_layer_gates_formula():
    '''g = -exp(A_log) softplus(a h + dt_bias), beta = sigmoid(b h), per head.'''
    h = torch.randn(2, 3, 8, dtype=D64)
    p = {'a_proj.weight': torch.randn(4, 8, dtype=D64), 'b_proj.weight': torch.randn(4, 8, dtype=D64),
         'A_log': torch.randn(4, dtype=D64), 'dt_bias': torch.randn(4, dtype=D64)}
    beta, g = gdn.gdn_gates(h, p)
    for hh in range(4):
        a = h @ p['a_proj.weight'][hh] + p['dt_bias'][hh]
        assert torch.allclose(g[:, hh], -p['A_log'][hh].exp() * torch.log1p(a.exp()), atol=1e-12)
        assert torch.allclose(beta[:, hh], 1 / (1 + (-(h @ p['b_proj.weight'][hh])).exp()), atol=1e-12)


def test_flop_formula_config1():
    assert gdn.gdn_prefill_flops(1, 256, 4, 64, 64) == pytest.approx(6.85e7, rel=2e-3)
    assert gdn.gdn_prefill_flops(1, 4096, 12, 64, 128) == pytest.approx(5.30e9, rel=2e-3)


def test_normalize_matches_reference_eps():
    x = torch.zeros(1, 1, 1, 4, dtype=D64)
    assert torch.equal(F.normalize(x, dim=-1), x)
