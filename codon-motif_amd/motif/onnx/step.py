'''The model step as a pure function of a flat list of cache tensors.

Mirrors the reference's step boundary (motif/onnx/step.py:7-92): per Chord layer its
key and value caches (wide: every query head), per GatedDelta layer its recurrent
state and the q / k / v conv tails, in layer order -- `('kv', 'kv')` and
`('gdn',) * 4` respectively (56 tensors for the 4 x (3 GDN + 1 Chord) model).
`ModelStep` maps `(input_ids [1, T], position [1], caches)` to
`(logits, *caches)`, running every layer on the HIP kernels the model uses.
'''
from typing import List, Sequence

import torch
import torch.nn as nn

from motif.model.cache import KVLayerCache, ModelCache, build_cache


def layers(model):
    '''The model's decoder layers in order (motif/onnx/step.py:7-10).'''
    for block in model.blocks:
        yield from block.features


def layer_plan(model) -> List[str]:
    '''`'kv'` twice per Chord layer, `'gdn'` four times per GatedDelta layer
    (motif/onnx/step.py:13-21).'''
    plan = []
    for layer in layers(model):
        plan += ['kv'] * 2 if issubclass(layer.cache_type, KVLayerCache) else ['gdn'] * 4
    return plan


def new_cache(model) -> ModelCache:
    '''A functional cache whose Chord keys / values are widened to every query head
    on write (motif/onnx/step.py:24-26).'''
    return build_cache(model, use_attn=True, functional=True, wide_kv=True)


def flat_state(model, cache: ModelCache) -> List[torch.Tensor]:
    '''The cache as one flat list in `layer_plan` order (motif/onnx/step.py:29-38).'''
    out = []
    for block_cache in cache.blocks:
        for lc in block_cache.attn:
            if isinstance(lc, KVLayerCache):
                out += [lc.k, lc.v]
            else:
                out += [lc.state, *lc.conv_state]
    return out


def rebuild_cache(model, flats: Sequence[torch.Tensor]) -> ModelCache:
    '''The inverse of `flat_state`: a fresh cache holding the given tensors
    (motif/onnx/step.py:41-56).  Key / value lengths come from their sequence axis.'''
    cache = new_cache(model)
    it = iter(flats)
    for block_cache in cache.blocks:
        for lc in block_cache.attn:
            if isinstance(lc, KVLayerCache):
                lc.k, lc.v = next(it), next(it)
                lc.length = lc.k.shape[2]
                lc._owned = True
            else:
                lc.state = next(it)
                lc.conv_state = (next(it), next(it), next(it))
    rest = list(it)
    if rest:
        raise ValueError(f'rebuild_cache: {len(rest)} tensors past the model\'s {len(layer_plan(model))}')
    return cache


def zero_flats(model, template: Sequence[torch.Tensor]) -> List[torch.Tensor]:
    '''The state of a model that has seen nothing, typed like `template` (any
    `flat_state` list): key / value entries become empty sequences, the rest zeros
    (motif/onnx/step.py:59-75).'''
    plan = layer_plan(model)
    if len(template) != len(plan):
        raise ValueError(f'zero_flats: {len(template)} tensors for a plan of {len(plan)}')
    return [t.new_zeros(1, t.shape[1], 0, t.shape[3]) if kind == 'kv' else torch.zeros_like(t)
            for kind, t in zip(plan, template)]


def dynamic_specs(model, kv_dim: int = 2):
    '''`torch.export` dynamic-shape specs: only the Chord layers' cached length varies
    (motif/onnx/step.py:78-81).'''
    return tuple({kv_dim: torch.export.Dim('S')} if kind == 'kv' else None for kind in layer_plan(model))


class ModelStep(nn.Module):
    '''`(input_ids [1, T], position [1], caches) -> (logits, *caches)`
    (motif/onnx/step.py:84-96).'''

    def __init__(self, model):
        super().__init__()
        self.model = model
        self.kinds = layer_plan(model)

    def forward(self, input_ids, position, caches):
        cache = rebuild_cache(self.model, caches)
        out = self.model(input_ids, cache=cache, position=position)
        return (out.logits, *flat_state(self.model, out.cache))
