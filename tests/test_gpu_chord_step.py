'''The fused Chord decode step (motif_chord_decode_step: q / k norms, the cache append,
split-K attention, the merge and the cursor advance in one launch) against the three
launches it replaces (motif_chord_qkv_prep at the device cursor, then
motif_chord_decode's decode and merge kernels), through ChordAttention's cursor decode
with `chord_attn.FUSED_STEP` on and off on copies of one StaticKVLayerCache:

- outputs, the appended key / value rows and the device cursor equal bit for bit over
  consecutive steps (the arrival counters return to zero after every step), at the
  model's shape (B = 64, 12 / 3 heads, a 4096-position context) and at small shapes
  (one split, two new tokens per step);
- a captured step replayed several times, with eager work between the replays, equals
  the same number of eager steps.
'''
import pytest
import torch

from golden.weights import fill_params
from support import gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _layer(H, Hkv, hidden, seed=5):
    from motif.block.attention.chord_attn import ChordAttention
    layer = ChordAttention(hidden_size=hidden, num_heads=H, num_kv_heads=Hkv)
    fill_params(layer, seed)
    return layer.to(DEV, torch.bfloat16).eval()


def _cache(B, Hkv, ctx, capacity, seed):
    '''A static cache whose first `ctx` positions hold random keys / values.'''
    from motif.model.cache import StaticKVLayerCache
    c = StaticKVLayerCache().allocate(B, Hkv, capacity, 64, DEV, torch.bfloat16)
    g = gen(seed)
    k, v = c._slab
    k[:, :, :ctx] = (torch.randn(B, Hkv, ctx, 64, generator=g) * 0.5).to(DEV, torch.bfloat16)
    v[:, :, :ctx] = (torch.randn(B, Hkv, ctx, 64, generator=g) * 0.5).to(DEV, torch.bfloat16)
    c.length = ctx
    c.length_dev.fill_(ctx)
    return c


def _copy(c):
    from motif.model.cache import StaticKVLayerCache
    d = StaticKVLayerCache().allocate(c.k.shape[0], c._slab[0].shape[1], c.capacity, 64, DEV, torch.bfloat16)
    d._slab[0].copy_(c._slab[0])
    d._slab[1].copy_(c._slab[1])
    d.length = c.length
    d.length_dev.copy_(c.length_dev)
    return d


def _steps(layer, cache, xs, fused):
    import motif.block.attention.chord_attn as ca
    prev, ca.FUSED_STEP = ca.FUSED_STEP, fused
    try:
        return [layer(x, past_key_value=cache, embedding_start=cache.length).output for x in xs]
    finally:
        ca.FUSED_STEP = prev


@pytest.mark.parametrize('B,H,Hkv,hidden,ctx,cap,L,n', [
    (64, 12, 3, 768, 4096, 4200, 1, 4),   # the model's decode shape
    (2, 4, 2, 256, 37, 64, 1, 5),         # a short cache: one split
    (3, 8, 2, 512, 300, 400, 2, 3),       # two new tokens per step
])
@torch.no_grad()
def test_fused_step_equals_three_launches(B, H, Hkv, hidden, ctx, cap, L, n):
    layer = _layer(H, Hkv, hidden)
    g = gen(7)
    xs = [(torch.randn(B, L, hidden, generator=g) * 0.5).to(DEV, torch.bfloat16) for _ in range(n)]
    c_fused = _cache(B, Hkv, ctx, cap, 11)
    c_ref = _copy(c_fused)
    from motif.ops.chord_attention import chord_decode_step_serves
    proj = layer._fused_proj(xs[0])
    assert chord_decode_step_serves(proj, H, Hkv, 64)
    got = _steps(layer, c_fused, xs, True)
    ref = _steps(layer, c_ref, xs, False)
    assert c_fused.step_workspace is not None and c_ref.step_workspace is None
    for i, (a, b) in enumerate(zip(got, ref)):
        assert torch.equal(a, b), f'step {i}: {(a.float() - b.float()).abs().max().item()}'
    end = ctx + n * L
    assert int(c_fused.length_dev.item()) == int(c_ref.length_dev.item()) == end
    assert torch.equal(c_fused._slab[0][:, :, :end], c_ref._slab[0][:, :, :end]), 'keys'
    assert torch.equal(c_fused._slab[1][:, :, :end], c_ref._slab[1][:, :, :end]), 'values'
    # every arrival counter is back at zero
    cnt = c_fused.step_workspace[-(B * Hkv + 1) * 4:].view(torch.int32)
    assert int(cnt.abs().sum().item()) == 0


@torch.no_grad()
def test_fused_step_graph_replays_equal_eager_steps():
    B, H, Hkv, hidden, ctx, cap = 8, 12, 3, 768, 1000, 1100
    layer = _layer(H, Hkv, hidden, seed=6)
    x = (torch.randn(B, 1, hidden, generator=gen(8)) * 0.5).to(DEV, torch.bfloat16)
    c_graph = _cache(B, Hkv, ctx, cap, 12)
    c_eager = _copy(c_graph)
    # warm-up (lazy set-up: fused weights, log table, workspace), then the cursor back
    _steps(layer, c_graph, [x], True)
    c_graph.length = ctx
    c_graph.length_dev.fill_(ctx)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = layer(x, past_key_value=c_graph, embedding_start=c_graph.length).output
    c_graph.length = ctx  # the capture recorded the step without running it
    eager = _steps(layer, c_eager, [x] * 3, True)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[i]), f'replay {i}'
        layer(x, past_key_value=_copy(c_eager), embedding_start=c_eager.length)  # eager work between replays
        torch.cuda.synchronize()
    assert int(c_graph.length_dev.item()) == ctx + 3
