'''The differentiable torch forms that calls needing gradients take (the HIP kernels
are forward-only): their forwards against the fp64 oracle, their backwards against
finite differences (gradcheck), the op entry points routing grad calls to them, a tiny
model training step on the CPU, and -- on the GPU -- training-mode logits equal to the
kernels' inference logits.'''
import pytest
import torch

from motif.ops.autograd_path import chord_attention_torch, gdn_chunk_torch, short_conv_silu_torch
from oracle import chord as ochord
from oracle import gdn as ogdn
from support import gdn_inputs


@pytest.mark.parametrize('L,C,init', [(70, 64, False), (37, 16, True), (5, 64, True)])
def test_gdn_torch_equals_oracle_recurrence(L, C, init):
    q, k, v, b, g = (t.double() for t in gdn_inputs(2, 3, L, 16, 24, seed=L))
    S0 = torch.randn(2, 3, 16, 24, dtype=torch.float64) * 0.1 if init else None
    o, S = gdn_chunk_torch(q, k, v, b, g, S0, C)
    ro, rS = ogdn.recurrent(q, k, v, b, g, S0)
    assert (o - ro).abs().max().item() < 1e-10 and (S - rS).abs().max().item() < 1e-10


def test_gdn_torch_gradcheck():
    q, k, v, b, g = (t.double().requires_grad_() for t in gdn_inputs(1, 1, 6, 3, 2, seed=2))
    S0 = (torch.randn(1, 1, 3, 2, dtype=torch.float64) * 0.3).requires_grad_()

    def f(q, k, v, b, g, S0):
        o, S = gdn_chunk_torch(q, k, v, b, g, S0, 4)
        return o, S
    assert torch.autograd.gradcheck(f, (q, k, v, b, g, S0))


def test_conv_torch_equals_oracle():
    g_ = torch.Generator().manual_seed(3)
    x = torch.randn(2, 9, 12, generator=g_, dtype=torch.float64)
    w = torch.randn(12, 1, 4, generator=g_, dtype=torch.float64) * 0.5
    cache = torch.randn(2, 12, 3, generator=g_, dtype=torch.float64)
    y, tail = short_conv_silu_torch(x, w, cache)
    ry, rtail = ogdn.short_conv_silu(x, w, cache)
    assert (y - ry).abs().max().item() < 1e-12 and torch.equal(tail, rtail)
    yn, _ = short_conv_silu_torch(x, w, cache, head_dim=4, scale=0.5)
    ref = torch.nn.functional.normalize(ry.view(2, 9, 3, 4), dim=-1).view(2, 9, 12) * 0.5
    assert (yn - ref).abs().max().item() < 1e-12


@pytest.mark.parametrize('Hkv,L,S,q_start', [(2, 7, 7, None), (1, 3, 10, 7), (4, 5, 9, 2)])
def test_chord_torch_equals_oracle(Hkv, L, S, q_start):
    g_ = torch.Generator().manual_seed(L + S)
    H, D = 4, 16
    q = torch.randn(2, H, L, D, generator=g_, dtype=torch.float64)
    k = torch.randn(2, Hkv, S, D, generator=g_, dtype=torch.float64)
    v = torch.randn(2, Hkv, S, D, generator=g_, dtype=torch.float64)
    alpha, beta = (torch.randn(H, generator=g_, dtype=torch.float64) * 0.3 for _ in range(2))
    alpha = alpha.abs()
    mu = torch.randn(H, generator=g_, dtype=torch.float64) * 0.5
    ssmax = 1 + 0.2 * torch.randn(H, generator=g_, dtype=torch.float64)
    qs = S - L if q_start is None else q_start
    log_n = torch.log(torch.arange(qs + 1, qs + L + 1, dtype=torch.float64)).expand(2, L).contiguous()
    out = chord_attention_torch(q, k, v, alpha, beta, mu, ssmax, log_n, q_start)
    ref = ochord.chord_attention(q, k, v, alpha, beta, mu, ssmax, log_n, q_start)
    assert (out - ref).abs().max().item() < 1e-10


def test_chord_torch_gradcheck():
    g_ = torch.Generator().manual_seed(9)
    mk = lambda *s: (torch.randn(*s, generator=g_, dtype=torch.float64) * 0.5).requires_grad_()
    q, k, v = mk(1, 2, 3, 4), mk(1, 1, 5, 4), mk(1, 1, 5, 4)
    alpha = (torch.rand(2, generator=g_, dtype=torch.float64) * 0.3 + 0.1).requires_grad_()
    beta, mu, ssmax = mk(2), mk(2), (1 + mk(2).detach() * 0.2).requires_grad_()
    log_n = torch.log(torch.arange(3, 6, dtype=torch.float64))[None]
    f = lambda *a: chord_attention_torch(*a, log_n)
    assert torch.autograd.gradcheck(f, (q, k, v, alpha, beta, mu, ssmax))


def test_op_entry_points_route_grad_calls():
    '''Grad-requiring calls no longer raise: they run the torch forms (on any device).'''
    import motif.ops as ops
    q, k, v, b, g = (t.requires_grad_() for t in gdn_inputs(1, 2, 20, 16, 16, seed=5))
    o, S = ops.chunk_gated_delta_rule(q, k, v, b, g)
    (o.sum() + S.sum()).backward()
    assert q.grad is not None and torch.isfinite(q.grad).all()
    o2, _ = ops.recurrent_gated_delta_rule(q, k, v, b, g)
    assert torch.allclose(o2, o, atol=1e-5)


def _identity_read(name):
    '''The first decoder of a block reads one source, which the attention-residual read
    returns unchanged (motif/ops/attn_res.py:619-620): its pseudo-query and norm weight
    never enter the graph, in the reference as here.'''
    import re
    return re.fullmatch(r'blocks\.\d+\.(pseudo_queries\.0|attn_res_norms\.0\.weight)', name) is not None


def test_tiny_model_backward_on_cpu():
    from motif.model.config import MotifChordConfig
    from motif.model.motif import MotifChordModel
    cfg = MotifChordConfig(vocab_size=97, model_dim=64, num_heads=4, num_kv_heads=2, head_k_dim=16,
                           block=('gdn', 'chord'), block_n=2)
    torch.manual_seed(0)
    m = MotifChordModel(cfg).train()
    ids = torch.randint(0, 97, (2, 70), generator=torch.Generator().manual_seed(1))
    out = m(ids, labels=ids)
    out.loss.backward()
    for name, p in m.named_parameters():
        if p.requires_grad and not _identity_read(name):
            assert p.grad is not None, f'{name} got no gradient'
            assert torch.isfinite(p.grad).all(), name


@pytest.mark.gpu
def test_training_forward_matches_kernel_inference():
    '''fp32 tiny model on the GPU: logits with gradients enabled (torch forms) equal
    the logits of the same forward under no_grad (HIP kernels).'''
    from motif.model.config import MotifChordConfig
    from motif.model.motif import MotifChordModel
    import motif.ops as ops
    assert ops.HAS_TRITON
    cfg = MotifChordConfig(vocab_size=128, model_dim=256, num_heads=4, num_kv_heads=2, head_k_dim=64,
                           block=('gdn', 'chord'), block_n=2)
    torch.manual_seed(0)
    m = MotifChordModel(cfg)
    with torch.no_grad():
        for p in m.parameters():
            p.add_(torch.randn_like(p) * 0.02)
    m = m.cuda().eval()
    ids = torch.randint(0, 128, (2, 150), generator=torch.Generator().manual_seed(1)).cuda()
    with torch.no_grad():
        ref = m(ids).logits
    out = m(ids).logits
    assert out.requires_grad
    err = (out - ref).abs().max().item()
    assert err <= 1e-4 * max(1.0, ref.abs().max().item()), err
    out.float().pow(2).mean().backward()
    assert all(torch.isfinite(p.grad).all() for p in m.parameters() if p.grad is not None)


def _train_grads(model, ids, cu=None):
    model.zero_grad(set_to_none=True)
    logits = model(ids, cu_seqlens=cu).logits
    logits.float().pow(2).mean().backward()
    return {n: p.grad.detach().cpu().clone() for n, p in model.named_parameters() if p.grad is not None}


@pytest.mark.gpu
@pytest.mark.parametrize('case', ['plain', 'packed', 'frozen_conv', 'frozen_embed'])
def test_gpu_gradients_match_cpu(case):
    '''Training on the GPU (fp32 tiny model with head_dim 64, so the kernels would serve
    its inference calls): every parameter that requires grad gets a gradient, and every
    gradient equals the same model's gradient on the CPU within 1e-3 of its scale.
    Cases: a padded batch, packed sequences (cu_seqlens), frozen conv weights (the
    layer's other parameters still train), a frozen embedding (the first layer's input
    needs no gradient, its weights do).'''
    import copy

    from motif.model.config import MotifChordConfig
    from motif.model.motif import MotifChordModel
    cfg = MotifChordConfig(vocab_size=128, model_dim=256, num_heads=4, num_kv_heads=2, head_k_dim=64,
                           block=('gdn', 'chord'), block_n=2, tied_weight=False)
    torch.manual_seed(0)
    m = MotifChordModel(cfg)
    with torch.no_grad():
        for p in m.parameters():
            p.add_(torch.randn_like(p) * 0.02)
    if case == 'frozen_conv':
        for blk in m.blocks:
            for dec in blk.features:
                if dec.attn_type == 'gdn':
                    for c in (dec.attn.q_conv, dec.attn.k_conv, dec.attn.v_conv):
                        c.weight.requires_grad_(False)
    if case == 'frozen_embed':
        m.embed.weight.requires_grad_(False)
    m = m.train()
    g_ = torch.Generator().manual_seed(1)
    cu = None
    if case == 'packed':
        ids = torch.randint(0, 128, (1, 150), generator=g_)
        cu = torch.tensor([0, 40, 41, 110, 150], dtype=torch.int32)
    else:
        ids = torch.randint(0, 128, (2, 90), generator=g_)
    ref = _train_grads(m, ids, cu)
    gm = copy.deepcopy(m).cuda()
    got = _train_grads(gm, ids.cuda(), None if cu is None else cu.cuda())
    want = {n for n, p in m.named_parameters() if p.requires_grad and not _identity_read(n)}
    assert set(ref) == want and set(got) == want, (sorted(want - set(got)), sorted(want - set(ref)))
    for n in sorted(want):
        scale = ref[n].abs().max().item()
        err = (got[n] - ref[n]).abs().max().item()
        assert err <= 1e-3 * scale + 1e-7, f'{case}: {n} gradient differs by {err:.3e} (scale {scale:.3e})'
