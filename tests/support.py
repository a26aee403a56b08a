'''Shared helpers: seeded inputs and the tolerance checks used by the parity tests.'''
import torch
import torch.nn.functional as F


def gen(seed=0):
    return torch.Generator().manual_seed(seed)


def gdn_inputs(B, H, T, dk, dv, seed=0, dtype=torch.float32):
    '''Config-1 style GDN inputs: q, k ~ N(0,1) L2-normalised; v ~ N(0,1);
    beta = sigmoid(N(0,1)); g = logsigmoid(N(0,1)).  Built on the CPU.'''
    gg = gen(seed)
    q = F.normalize(torch.randn(B, H, T, dk, generator=gg), dim=-1)
    k = F.normalize(torch.randn(B, H, T, dk, generator=gg), dim=-1)
    v = torch.randn(B, H, T, dv, generator=gg)
    beta = torch.sigmoid(torch.randn(B, H, T, generator=gg))
    g = F.logsigmoid(torch.randn(B, H, T, generator=gg))
    return [t.to(dtype) for t in (q, k, v, beta, g)]


def chord_inputs(B, H, Hkv, L, S, seed=0, D=64):
    '''Config-2 style Chord inputs (bf16 q/k/v ~ 0.5 N(0,1); alpha, beta ~ 0.1 N(0,1);
    mu = 0; ssmax = 1).'''
    gg = gen(seed)
    q = (torch.randn(B, H, L, D, generator=gg) * 0.5).to(torch.bfloat16)
    k = (torch.randn(B, Hkv, S, D, generator=gg) * 0.5).to(torch.bfloat16)
    v = (torch.randn(B, Hkv, S, D, generator=gg) * 0.5).to(torch.bfloat16)
    alpha = torch.randn(H, generator=gg) * 0.1
    beta = torch.randn(H, generator=gg) * 0.1
    mu = torch.zeros(H)
    ssmax = torch.ones(H)
    return q, k, v, alpha, beta, mu, ssmax


def assert_bf16_close(out, ref, max_abs=2e-2, mean_rel=5e-3, what=''):
    '''The bf16 bar: max-abs <= 2e-2 and mean-relative (sum|d| / sum|ref|) <= 5e-3.'''
    out = out.detach().double().cpu()
    ref = ref.detach().double().cpu()
    d = (out - ref).abs()
    ma = d.max().item() if d.numel() else 0.0
    mr = (d.sum() / ref.abs().sum().clamp_min(1e-30)).item() if d.numel() else 0.0
    assert ma <= max_abs and mr <= mean_rel, f'{what}: max_abs={ma:.3e} mean_rel={mr:.3e}'
    return ma, mr


def assert_fp32_close(out, ref, tol=1e-4, what=''):
    '''The fp32 bar: max |out - ref| <= tol * max(1, max|ref|).'''
    out = out.detach().double().cpu()
    ref = ref.detach().double().cpu()
    d = (out - ref).abs().max().item() if out.numel() else 0.0
    scale = max(1.0, ref.abs().max().item() if ref.numel() else 0.0)
    assert d <= tol * scale, f'{what}: max_abs={d:.3e} (tol {tol * scale:.3e})'
    return d


def assert_state_close(out, ref, rel=1e-2, what=''):
    '''Final recurrent state within relative Frobenius error `rel`.'''
    out = out.detach().double().cpu()
    ref = ref.detach().double().cpu()
    e = ((out - ref).norm() / ref.norm().clamp_min(1e-30)).item()
    assert e <= rel, f'{what}: rel_err={e:.3e}'
    return e


def bf16_gap(out, ref):
    '''(max |out - ref|, mean-relative sum|out - ref| / sum|ref|) in float64.'''
    out = out.detach().double().cpu()
    ref = ref.detach().double().cpu()
    d = (out - ref).abs()
    if not d.numel():
        return 0.0, 0.0
    return d.max().item(), (d.sum() / ref.abs().sum().clamp_min(1e-30)).item()


def assert_bf16_layer_close(out, ref64, ref16, what='', max_abs=2e-2, mean_rel=5e-3, slack=1.25):
    '''A bf16 layer output against the exact (float64) result of the same layer on the
    same inputs: within the bf16 bar (max-abs 2e-2, mean-rel 5e-3), or no further from
    the exact result than the reference's own bf16 arithmetic (`ref16`, the oracle run
    in bf16) is, times `slack`.  A whole layer rounds its projections, gates and norms
    to bf16, which alone moves it ~7e-3 (mean-rel) from the exact result at the model
    shapes; the bar of the ops themselves applies where that gap is smaller.'''
    g_max, g_mr = bf16_gap(out, ref64)
    r_max, r_mr = bf16_gap(ref16, ref64)
    lim_max, lim_mr = max(max_abs, slack * r_max), max(mean_rel, slack * r_mr)
    msg = (f'{what}: vs exact max_abs={g_max:.3e} mean_rel={g_mr:.3e}; reference bf16 arithmetic '
           f'max_abs={r_max:.3e} mean_rel={r_mr:.3e}')
    print(msg, flush=True)
    assert g_max <= lim_max and g_mr <= lim_mr, msg
    return g_max, g_mr
