'''GPU parity of the Chord backward kernels (motif_chord_bwd through ChordFunction)
against the differentiable torch form (motif/ops/autograd_path.py, gradcheck-pinned in
tests/test_autograd_path.py) run in float64 on the CPU with the same bf16 inputs.

Bars: dq / dk / dv within max-abs 2.5e-2 of the largest reference entry and mean-relative
1e-2 (the kernels round P and dZ to bf16 as MFMA operands, as the reference's bf16
backward does); the [H] parameter gradients within 3e-2 relative (Frobenius) error: each
is a sum over every (query, key) pair of terms that cancel row by row (the entries of a
row of dZ sum to zero), and the row sums Delta = dO . O use the bf16 output, as the
reference's backward does, which leaves ~1e-2 of the sum.'''
import math

import pytest
import torch

from support import gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _inputs(B, H, Hkv, L, S, seed):
    g = gen(seed)
    q = (torch.randn(B, H, L, 64, generator=g) * 0.5).to(torch.bfloat16)
    k = (torch.randn(B, Hkv, S, 64, generator=g) * 0.5).to(torch.bfloat16)
    v = (torch.randn(B, Hkv, S, 64, generator=g) * 0.5).to(torch.bfloat16)
    alpha = torch.randn(H, generator=g) * 0.1 + 0.05
    beta = torch.randn(H, generator=g) * 0.1 + 0.3
    mu = torch.randn(H, generator=g) * 0.5
    ssmax = 1.0 + torch.randn(H, generator=g) * 0.1
    dout = torch.randn(B, H, L, 64, generator=g).to(torch.bfloat16)
    return q, k, v, alpha, beta, mu, ssmax, dout


def _grads_torch64(q, k, v, alpha, beta, mu, ssmax, log_n, q_start, dout):
    from motif.ops.autograd_path import chord_attention_torch
    ts = [t.double().requires_grad_(True) for t in (q, k, v, alpha, beta, mu, ssmax)]
    out = chord_attention_torch(*ts, log_n.double(), q_start, 64 ** -0.5, 1e-5)
    (out * dout.double()).sum().backward()
    return out.detach(), [t.grad for t in ts]


def _grads_gpu(q, k, v, alpha, beta, mu, ssmax, log_n, q_start, dout):
    from motif.ops import apply_chord_attention
    ts = [t.to(DEV).requires_grad_(True) for t in (q, k, v, alpha, beta, mu, ssmax)]
    out = apply_chord_attention(*ts, log_n.to(DEV), q_start=q_start, softmax_scale=64 ** -0.5, eps=1e-5)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    return out.detach().cpu(), [t.grad.detach().cpu() for t in ts]


def _close(got, ref, what, max_rel=2.5e-2, mean_rel=1e-2):
    got, ref = got.double(), ref.double()
    d = (got - ref).abs()
    scale = ref.abs().max().item()
    mr = d.sum().item() / max(ref.abs().sum().item(), 1e-30)
    print(f'{what}: max_abs={d.max().item():.3e} (of {scale:.3e}) mean_rel={mr:.3e}', flush=True)
    assert d.max().item() <= max_rel * max(scale, 1e-6) and mr <= mean_rel, what


@pytest.mark.parametrize('B,H,Hkv,L,S,q_start', [
    (2, 4, 2, 160, 160, 0),      # GQA group 2, ragged last tiles
    (1, 4, 4, 96, 300, 204),     # MHA, queries after a cached prefix
    (1, 12, 3, 512, 512, 0),     # the model's grouping (4 heads per kv head)
    (1, 4, 2, 1024, 1024, 0),    # causal loops cut into chunks (fp32 partials summed)
    (1, 2, 1, 700, 1500, 800),   # chunks after a cached prefix, ragged tiles
])
def test_chord_backward_matches_torch_form(B, H, Hkv, L, S, q_start):
    q, k, v, alpha, beta, mu, ssmax, dout = _inputs(B, H, Hkv, L, S, seed=L + S + H)
    log_n = torch.log(torch.arange(q_start + 1, q_start + L + 1, dtype=torch.float32))[None].expand(B, L).contiguous()
    ro, rg = _grads_torch64(q, k, v, alpha, beta, mu, ssmax, log_n, q_start, dout)
    go, gg = _grads_gpu(q, k, v, alpha, beta, mu, ssmax, log_n, q_start, dout)
    _close(go, ro, 'out', 2e-2, 5e-3)
    for name, got, ref in zip(('dq', 'dk', 'dv'), gg[:3], rg[:3]):
        _close(got, ref, name)
    for name, got, ref in zip(('d_alpha', 'd_beta', 'd_mu', 'd_ssmax'), gg[3:], rg[3:]):
        err = ((got.double() - ref).norm() / ref.norm().clamp_min(1e-30)).item()
        print(f'{name}: rel={err:.3e} ref_norm={ref.norm().item():.3e}', flush=True)
        assert err <= 3e-2, name


def test_chord_backward_only_some_inputs_need_grad():
    '''Gradients flow only where asked; the parameters' slots stay None otherwise.'''
    from motif.ops import apply_chord_attention
    q, k, v, alpha, beta, mu, ssmax, dout = _inputs(1, 4, 2, 64, 64, seed=3)
    log_n = torch.log(torch.arange(1, 65, dtype=torch.float32))[None].contiguous()
    qd = q.to(DEV).requires_grad_(True)
    out = apply_chord_attention(qd, k.to(DEV), v.to(DEV), alpha.to(DEV), beta.to(DEV), mu.to(DEV), ssmax.to(DEV),
                                log_n.to(DEV), q_start=0)
    out.backward(dout.to(DEV))
    assert qd.grad is not None and qd.grad.shape == q.shape
    assert math.isfinite(qd.grad.float().abs().sum().item())


def test_varlen_backward_matches_torch_form():
    '''Packed sequences with gradients: each sequence through the HIP forward / backward
    pair, against the per-sequence torch form in float64 (same bars as above).'''
    from motif.ops import apply_chord_attention_varlen
    from motif.ops.autograd_path import chord_attention_varlen_torch
    lens = [1, 70, 130, 5, 64]
    T = sum(lens)
    q, k, v, alpha, beta, mu, ssmax, dout = _inputs(1, 4, 2, T, T, seed=11)
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    log_n = torch.cat([torch.log(torch.arange(1, n + 1, dtype=torch.float32)) for n in lens])[None].contiguous()
    ts = [t.double().requires_grad_(True) for t in (q, k, v, alpha, beta, mu, ssmax)]
    ro = chord_attention_varlen_torch(*ts, log_n.double(), cu, 64 ** -0.5, 1e-5)
    (ro * dout.double()).sum().backward()
    rg = [t.grad for t in ts]
    gs = [t.to(DEV).requires_grad_(True) for t in (q, k, v, alpha, beta, mu, ssmax)]
    go = apply_chord_attention_varlen(*gs, log_n.to(DEV), cu.to(DEV), softmax_scale=64 ** -0.5, eps=1e-5)
    go.backward(dout.to(DEV))
    torch.cuda.synchronize()
    _close(go.detach().cpu(), ro.detach(), 'out', 2e-2, 5e-3)
    for name, got, ref in zip(('dq', 'dk', 'dv'), gs[:3], rg[:3]):
        _close(got.grad.detach().cpu(), ref, name)
    for name, got, ref in zip(('d_alpha', 'd_beta', 'd_mu', 'd_ssmax'), gs[3:], rg[3:]):
        err = ((got.grad.detach().cpu().double() - ref).norm() / ref.norm().clamp_min(1e-30)).item()
        print(f'{name}: rel={err:.3e}', flush=True)
        assert err <= 3e-2, name
