'''GPU parity of the fused GDN decode step (motif_gdn_decode_fused inside
GatedDeltaAttention.forward for L == 1 with a cache) against the CPU oracle's
layer restatement (oracle/gdn.py gdn_layer, the recurrence for L == 1).

- fp32 layers: within 1e-4 of the fp64 oracle for every supported head size
  (dk 16 / 32 / 64, dv up to 128, odd dv, conv kernels 2..5), over several steps
  from a random state and random conv tails; state and tails within 1e-4 too.
- An empty cache starts from zero state and zero tails (the oracle's defaults).
- bf16: against the fp64 oracle on the same bf16 weights / inputs (the bf16 bar, or no
  further than the reference's own bf16 arithmetic is), and within the bf16 bar of that
  arithmetic (the oracle run in bf16).
- Unsupported layouts (a bf16 state, dk 128) fall back to the unfused ops and still
  match.
'''
import pytest
import torch

from golden.weights import fill_params
from oracle.gdn import gdn_layer
from support import assert_bf16_close, assert_bf16_layer_close, assert_fp32_close, gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _layer(hidden, H, dk, dv, K, dtype, seed=11):
    from motif.block.attention.gdn_attn import GatedDeltaAttention
    layer = GatedDeltaAttention(hidden_size=hidden, num_heads=H, head_k_dim=dk, expand_v=dv / dk, conv_size=K)
    assert layer.dv == dv
    fill_params(layer, seed)
    return layer.to(DEV, dtype).eval()


def _random_cache(layer, B, dtype, seed):
    from motif.model.cache import GatedDeltaAttentionLayerCache
    g = gen(seed)
    H, dk, dv, K = layer.num_heads, layer.dk, layer.dv, layer.conv_size
    c = GatedDeltaAttentionLayerCache()
    c.state = (torch.randn(B, H, dk, dv, generator=g) * 0.1).to(DEV)
    c.conv_state = tuple((torch.randn(B, n, K - 1, generator=g) * 0.5).to(DEV, dtype)
                         for n in (H * dk, H * dk, H * dv))
    c.length = 7
    return c


def _run_steps(layer, cache, xs, p, ref_dtype=torch.float64):
    '''Decode every token of xs [B, n, hidden] through the layer and the oracle.'''
    H, dk, dv = layer.num_heads, layer.dk, layer.dv
    S = None if cache.state is None else cache.state.detach().cpu().to(ref_dtype)
    tails = None if cache.conv_state is None else tuple(t.detach().cpu().to(ref_dtype) for t in cache.conv_state)
    outs, refs = [], []
    for i in range(xs.shape[1]):
        x = xs[:, i:i + 1]
        outs.append(layer(x.to(DEV), past_key_value=cache).output)
        r, S, tails = gdn_layer(x.to(ref_dtype), p, H, dk, dv, state=S, conv_state=tails)
        refs.append(r)
    return torch.cat(outs, 1), torch.cat(refs, 1), S, tails


SHAPES = [  # (B, hidden, H, dk, dv, K)
    (3, 64, 2, 16, 32, 2),
    (2, 96, 3, 32, 64, 3),
    (5, 128, 2, 64, 128, 4),
    (1, 64, 1, 64, 96, 5),
    (4, 64, 4, 16, 16, 4),
]


@pytest.mark.parametrize('B,hidden,H,dk,dv,K', SHAPES)
@torch.no_grad()
def test_fused_decode_fp32_matches_oracle(B, hidden, H, dk, dv, K):
    layer = _layer(hidden, H, dk, dv, K, torch.float32)
    cache = _random_cache(layer, B, torch.float32, seed=dk + dv + K)
    assert layer._decode_fusable(torch.empty(B, 1, hidden, device=DEV), cache)
    p = {k: v.detach().double().cpu() for k, v in layer.state_dict().items()}
    xs = torch.randn(B, 4, hidden, generator=gen(3))
    out, ref, S_ref, tails_ref = _run_steps(layer, cache, xs, p)
    what = f'B={B} H={H} dk={dk} dv={dv} K={K}'
    assert_fp32_close(out, ref, 1e-4, f'out {what}')
    assert_fp32_close(cache.state, S_ref, 1e-4, f'state {what}')
    for t, r in zip(cache.conv_state, tails_ref):
        assert_fp32_close(t, r, 1e-6, f'tails {what}')
    assert cache.seq_length == 11


@torch.no_grad()
def test_fused_decode_from_empty_cache():
    from motif.model.cache import GatedDeltaAttentionLayerCache
    layer = _layer(128, 2, 64, 128, 4, torch.float32)
    p = {k: v.detach().double().cpu() for k, v in layer.state_dict().items()}
    cache = GatedDeltaAttentionLayerCache()
    xs = torch.randn(2, 3, 128, generator=gen(4))
    out, ref, S_ref, _ = _run_steps(layer, cache, xs, p)
    assert_fp32_close(out, ref, 1e-4, 'out')
    assert_fp32_close(cache.state, S_ref, 1e-4, 'state')
    assert cache.seq_length == 3


@torch.no_grad()
def test_fused_decode_bf16_matches_oracle():
    B, hidden, H, dk, dv, K = 8, 256, 4, 64, 128, 4
    layer = _layer(hidden, H, dk, dv, K, torch.bfloat16)
    cache = _random_cache(layer, B, torch.bfloat16, seed=5)
    p = {k: v.detach().double().cpu() for k, v in layer.state_dict().items()}
    p16 = {k: v.detach().cpu() for k, v in layer.state_dict().items()}
    xs = torch.randn(B, 3, hidden, generator=gen(6)).to(torch.bfloat16)
    # the reference's own bf16 arithmetic: the oracle layer in bf16 from the same cache
    S16, tails16 = cache.state.detach().cpu(), tuple(t.detach().cpu() for t in cache.conv_state)
    r16 = []
    for i in range(xs.shape[1]):
        r, S16, tails16 = gdn_layer(xs[:, i:i + 1], p16, H, dk, dv, state=S16, conv_state=tails16)
        r16.append(r)
    r16 = torch.cat(r16, 1)
    out, ref, S_ref, _ = _run_steps(layer, cache, xs, p)
    # within the bf16 bar of the exact result, or no further than the reference's bf16
    # arithmetic is; and within the bf16 bar of that arithmetic itself
    assert_bf16_layer_close(out, ref, r16, 'bf16 fused decode')
    assert_bf16_close(out, r16, 2e-2, 5e-3, 'bf16 fused decode vs the reference bf16 arithmetic')
    e = ((cache.state.double().cpu() - S_ref).norm() / S_ref.norm()).item()
    assert e < 1e-2, e


@torch.no_grad()
def test_unfusable_layouts_fall_back_and_match():
    layer = _layer(128, 2, 64, 128, 4, torch.float32)
    B = 2
    p = {k: v.detach().double().cpu() for k, v in layer.state_dict().items()}
    xs = torch.randn(B, 2, 128, generator=gen(7))
    # non-contiguous state: not the kernel's layout -> the unfused ops
    cache = _random_cache(layer, B, torch.float32, seed=8)
    cache.state = cache.state.transpose(2, 3).contiguous().transpose(2, 3)
    assert not layer._decode_fusable(xs[:, :1].to(DEV), cache)
    out, ref, S_ref, _ = _run_steps(layer, cache, xs, p)
    assert_fp32_close(out, ref, 1e-4, 'fallback out')
    assert_fp32_close(cache.state, S_ref, 1e-4, 'fallback state')
    # dk = 128 has no fused decode kernel
    wide = _layer(256, 2, 128, 128, 4, torch.float32)
    cw = _random_cache(wide, B, torch.float32, seed=9)
    assert not wide._decode_fusable(torch.empty(B, 1, 256, device=DEV), cw)
    pw = {k: v.detach().double().cpu() for k, v in wide.state_dict().items()}
    out, ref, _, _ = _run_steps(wide, cw, torch.randn(B, 2, 256, generator=gen(10)), pw)
    assert_fp32_close(out, ref, 1e-4, 'dk128 out')
