'''The graph-replayable decode step (DecodeGraph over ModelCache.for_decode): the
Chord layers append at, attend up to and advance a device cursor, the GatedDelta
layers update their state in place, so one captured step replays token after
token with no host rewinds.

- tiny model, fp32: prefill 75 tokens, then 5 graph replays -- logits within 1e-4
  of the reference's own decode fixture (tests/golden/tiny_model.safetensors).
- tiny model, bf16: N graph replays equal N eager steps over the same caches bit
  for bit, and match the growing-cache decode within the bf16 bar.
- the device cursors and host lengths agree after the replays; a step past the
  capacity raises before launching.
- the ordinary GatedDelta cache keeps the reference's replace-on-update semantics:
  a state tensor taken before a decode step is left unchanged by it.
'''
import pytest
import torch

from support import assert_bf16_close, assert_fp32_close
from test_gpu_layers import _tiny_model

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _prefilled(model, ids, n_pre, capacity, dtype):
    from motif.model.cache import ModelCache
    cache = ModelCache.for_decode(model, ids.shape[0], capacity, DEV, dtype)
    pre = model(ids[:, :n_pre], cache=cache).logits
    return cache, pre


@torch.no_grad()
def test_graph_decode_fp32_matches_reference_fixture():
    from motif.model.decode_graph import DecodeGraph
    cfg, t, model = _tiny_model(torch.float32)
    ids = t['ids'].to(DEV)
    cache, pre = _prefilled(model, ids, 75, 96, torch.float32)
    assert_fp32_close(pre, t['logits_pre'], 1e-4, 'prefill into fixed-capacity caches')
    graph = DecodeGraph(model, cache, ids.shape[0])
    steps = torch.cat([graph.step(ids[:, i:i + 1]).clone() for i in range(75, 80)], 1)
    assert_fp32_close(steps, t['logits_steps'], 1e-4, 'graph decode steps')
    for lc in cache.layer_caches():
        assert lc.length == 80
        if hasattr(lc, 'length_dev'):
            assert int(lc.length_dev.item()) == 80


@torch.no_grad()
def test_graph_replays_equal_eager_steps_bf16():
    from motif.model.decode_graph import DecodeGraph
    cfg, t, model = _tiny_model(torch.bfloat16)
    ids = t['ids'].to(DEV)
    cache, _ = _prefilled(model, ids, 60, 80, torch.bfloat16)
    kept = [(lc.state.clone(), tuple(c.clone() for c in lc.conv_state)) if hasattr(lc, 'state')
            else (lc._slab[0].clone(), lc._slab[1].clone(), lc.length_dev.clone()) for lc in cache.layer_caches()]
    graph = DecodeGraph(model, cache, ids.shape[0])
    g = torch.cat([graph.step(ids[:, i:i + 1]).clone() for i in range(60, 72)], 1)
    # the same 12 steps eagerly from the same caches
    for lc, saved in zip(cache.layer_caches(), kept):
        if hasattr(lc, 'state'):
            lc.state.copy_(saved[0])
            for dst, src in zip(lc.conv_state, saved[1]):
                dst.copy_(src)
        else:
            lc._slab[0].copy_(saved[0])
            lc._slab[1].copy_(saved[1])
            lc.length_dev.copy_(saved[2])
        lc.length = 60
    for b in cache.blocks:
        b.attn_res.seq_len = 60
    e = torch.cat([model(ids[:, i:i + 1], cache=cache).logits for i in range(60, 72)], 1)
    assert torch.equal(g, e), (g.float() - e.float()).abs().max().item()
    dyn = model.create_cache()
    model(ids[:, :60], cache=dyn)
    d = torch.cat([model(ids[:, i:i + 1], cache=dyn).logits for i in range(60, 72)], 1)
    assert_bf16_close(e, d, 2e-2, 5e-3, 'fixed-capacity vs growing caches')


@torch.no_grad()
def test_graph_step_past_capacity_raises():
    from motif.model.decode_graph import DecodeGraph
    cfg, t, model = _tiny_model(torch.bfloat16)
    ids = t['ids'].to(DEV)
    cache, _ = _prefilled(model, ids, 30, 32, torch.bfloat16)
    graph = DecodeGraph(model, cache, ids.shape[0])
    graph.step(ids[:, 30:31])
    graph.step(ids[:, 31:32])
    with pytest.raises(RuntimeError, match='capacity'):
        graph.step(ids[:, 32:33])
    assert all(lc.length == 32 for lc in cache.layer_caches())


@torch.no_grad()
def test_gdn_decode_replaces_the_state_of_an_ordinary_cache():
    cfg, t, model = _tiny_model(torch.bfloat16)
    ids = t['ids'].to(DEV)
    cache = model.create_cache()
    model(ids[:, :40], cache=cache)
    layer_cache = cache[0].attn[0]
    before = layer_cache.state
    before_copy = before.clone()
    tails = layer_cache.conv_state
    tails_copy = tuple(x.clone() for x in tails)
    model(ids[:, 40:41], cache=cache)
    assert layer_cache.state is not before
    assert torch.equal(before, before_copy)
    assert all(torch.equal(a, b) for a, b in zip(tails, tails_copy))
    assert not torch.equal(layer_cache.state, before)
