'''The static-graph step boundary (motif.onnx.step): the flat cache ordering of the
reference's motif/onnx/step.py (56 tensors for the 172M model), the flat / rebuild
round trip, zero_flats, and -- on the GPU -- that stepping through ModelStep from
zero state gives the logits of one full forward.'''
import pytest
import torch

from motif.model.cache import FunctionalKVLayerCache, GatedDeltaAttentionLayerCache
from motif.model.config import MotifChordConfig
from motif.model.motif import MotifChordModel
from motif.onnx.step import (ModelStep, flat_state, layer_plan, new_cache, rebuild_cache,
                             zero_flats)

TINY = MotifChordConfig(vocab_size=97, model_dim=64, num_heads=4, num_kv_heads=2, head_k_dim=16,
                        block=('gdn', 'chord'), block_n=2)


def test_plan_of_the_published_model():
    with torch.device('meta'):
        m = MotifChordModel(MotifChordConfig(vocab_size=32000))
    plan = layer_plan(m)
    assert len(plan) == 56
    assert plan == (['gdn'] * 12 + ['kv'] * 2) * 4


def _fake_flats(m, S=5):
    cfg = m.config
    out = []
    for kind in layer_plan(m):
        out.append(torch.randn(1, cfg.num_heads, S, cfg.model_dim // cfg.num_heads) if kind == 'kv'
                   else torch.randn(1, 3, 4))
    return out


def test_flat_rebuild_round_trip():
    m = MotifChordModel(TINY)
    flats = _fake_flats(m)
    cache = rebuild_cache(m, flats)
    kinds = [type(lc) for b in cache.blocks for lc in b.attn]
    assert kinds == [GatedDeltaAttentionLayerCache, FunctionalKVLayerCache] * 2
    assert all(lc.num_heads == TINY.num_heads for b in cache.blocks for lc in b.attn
               if isinstance(lc, FunctionalKVLayerCache))
    assert [lc.length for b in cache.blocks for lc in b.attn if isinstance(lc, FunctionalKVLayerCache)] == [5, 5]
    back = flat_state(m, cache)
    assert len(back) == len(flats) and all(a is b for a, b in zip(back, flats))


def test_zero_flats_and_errors():
    m = MotifChordModel(TINY)
    flats = _fake_flats(m, S=7)
    z = zero_flats(m, flats)
    for kind, t, src in zip(layer_plan(m), z, flats):
        if kind == 'kv':
            assert t.shape == (1, src.shape[1], 0, src.shape[3])
        else:
            assert t.shape == src.shape and not t.any()
    with pytest.raises(ValueError):
        zero_flats(m, flats[:-1])
    with pytest.raises(ValueError):
        rebuild_cache(m, flats + [torch.zeros(1)])
    assert isinstance(new_cache(m).blocks[0].attn[1], FunctionalKVLayerCache)


@pytest.mark.gpu
@pytest.mark.parametrize('dtype,tol', [(torch.float32, 1e-3), (torch.bfloat16, 6e-2)])
def test_model_step_from_zero_state_matches_full_forward(dtype, tol):
    '''Prefill 40 tokens through ModelStep from zero_flats, then 3 one-token steps:
    the logits equal one full forward over the 43 tokens (the step's caches carry
    everything the later tokens need).'''
    torch.manual_seed(0)
    cfg = MotifChordConfig(vocab_size=128, model_dim=256, num_heads=4, num_kv_heads=2, head_k_dim=64,
                           block=('gdn', 'chord'), block_n=2)
    m = MotifChordModel(cfg)
    with torch.no_grad():
        for p in m.parameters():
            p.add_(torch.randn_like(p) * 0.02)
    m = m.to('cuda', dtype).eval()
    ids = torch.randint(0, 128, (1, 43), generator=torch.Generator().manual_seed(1)).cuda()
    step = ModelStep(m)
    with torch.no_grad():
        full = m(ids).logits.float()
        warm = step(ids[:, :1], torch.tensor([0], device='cuda'), zero_flats(m, flat_state(m, _warm_cache(m, ids))))
        assert len(warm) == 1 + len(layer_plan(m))
        flats = zero_flats(m, list(warm[1:]))
        out = step(ids[:, :40], torch.tensor([0], device='cuda'), flats)
        logits = [out[0].float()]
        flats = list(out[1:])
        for t in range(40, 43):
            out = step(ids[:, t:t + 1], torch.tensor([t], device='cuda'), flats)
            logits.append(out[0].float())
            flats = list(out[1:])
    got = torch.cat(logits, 1)
    scale = full.abs().max().item()
    assert (got - full).abs().max().item() <= tol * scale, (got - full).abs().max().item()
    kv = [t for t, kind in zip(flats, layer_plan(m)) if kind == 'kv']
    assert all(t.shape == (1, cfg.num_heads, 43, cfg.model_dim // cfg.num_heads) for t in kv)


def _warm_cache(m, ids):
    cache = new_cache(m)
    m(ids[:, :1], cache=cache, position=torch.tensor([0], device=ids.device))
    return cache
