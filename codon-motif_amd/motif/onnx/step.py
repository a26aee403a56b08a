'''The model step as a pure function of a flat list of cache tensors.

Public surface and flat order of motif/onnx/step.py:7-96: per Chord layer its
key and value caches (wide: every query head), per GatedDelta layer its
recurrent state and the q / k / v conv tails, layer after layer -- so the plan
reads `('kv', 'kv')` per Chord layer and `('gdn',) * 4` per GatedDelta layer
(56 tensors for the 4 x (3 GDN + 1 Chord) model).

Design: `slots(model)` lists, once per model, where each flat entry lives
(block, layer, field); flattening and rebuilding are two walks over that table,
so the order is defined in exactly one place.  `ModelStep` maps
`(input_ids [1, T], position [1], caches) -> (logits, *caches)` and runs every
layer on the same HIP kernels the model uses.
'''
from typing import List, NamedTuple, Sequence

import torch
import torch.nn as nn

from motif.model.cache import KVLayerCache, ModelCache, build_cache

# fields of one layer cache, in flat order, per kind
_FIELDS = {'kv': ('k', 'v'), 'gdn': ('state', 'conv_q', 'conv_k', 'conv_v')}


class Slot(NamedTuple):
    block: int
    layer: int
    kind: str    # 'kv' or 'gdn'
    field: str   # one of _FIELDS[kind]


def layers(model):
    '''The decoder layers of `model`, block by block.'''
    for block in model.blocks:
        yield from block.features


def _kind(layer) -> str:
    return 'kv' if issubclass(layer.cache_type, KVLayerCache) else 'gdn'


def slots(model) -> List[Slot]:
    '''Where every flat cache entry of `model` lives.'''
    return [Slot(b, j, _kind(layer), f)
            for b, block in enumerate(model.blocks)
            for j, layer in enumerate(block.features)
            for f in _FIELDS[_kind(layer)]]


def layer_plan(model) -> List[str]:
    '''The kind ('kv' / 'gdn') of every flat entry.'''
    return [s.kind for s in slots(model)]


def new_cache(model) -> ModelCache:
    '''A functional cache with keys / values expanded to every query head on write.'''
    return build_cache(model, use_attn=True, functional=True, wide_kv=True)


def _read(layer_cache, field: str) -> torch.Tensor:
    if field in ('k', 'v'):
        return getattr(layer_cache, field)
    if field == 'state':
        return layer_cache.state
    return layer_cache.conv_state[('conv_q', 'conv_k', 'conv_v').index(field)]


def flat_state(model, cache: ModelCache) -> List[torch.Tensor]:
    '''The cache as one flat list (the order of `slots(model)`).'''
    return [_read(cache.blocks[s.block].attn[s.layer], s.field) for s in slots(model)]


def rebuild_cache(model, flats: Sequence[torch.Tensor]) -> ModelCache:
    '''A fresh `new_cache(model)` holding the given tensors (inverse of flat_state);
    key / value lengths follow their sequence axis.'''
    table = slots(model)
    if len(flats) != len(table):
        raise ValueError(f'rebuild_cache: the model has {len(table)} cache entries, got {len(flats)}')
    cache = new_cache(model)
    grouped = {}
    for s, t in zip(table, flats):
        grouped.setdefault((s.block, s.layer), {})[s.field] = t
    for (b, j), fields in grouped.items():
        lc = cache.blocks[b].attn[j]
        if 'k' in fields:
            lc.adopt(fields['k'], fields['v'])
        else:
            lc.state = fields['state']
            lc.conv_state = (fields['conv_q'], fields['conv_k'], fields['conv_v'])
    return cache


def zero_flats(model, template: Sequence[torch.Tensor]) -> List[torch.Tensor]:
    '''The state of a model that has seen nothing, typed like `template` (a flat_state
    list): key / value entries hold no position, everything else is zero.'''
    table = slots(model)
    if len(template) != len(table):
        raise ValueError(f'zero_flats: the model has {len(table)} cache entries, got {len(template)}')
    out = []
    for s, t in zip(table, template):
        if s.kind == 'kv':
            out.append(torch.zeros((1, t.shape[1], 0, t.shape[3]), dtype=t.dtype, device=t.device))
        else:
            out.append(torch.zeros_like(t))
    return out


def dynamic_specs(model, kv_dim: int = 2):
    '''`torch.export` dynamic-shape specs: the Chord caches' length axis varies, nothing else.'''
    length = torch.export.Dim('S')
    return tuple({kv_dim: length} if s.kind == 'kv' else None for s in slots(model))


class ModelStep(nn.Module):
    '''`(input_ids [1, T], position [1], caches) -> (logits, *caches)`.'''

    def __init__(self, model):
        super().__init__()
        self.model = model
        self.kinds = layer_plan(model)

    def forward(self, input_ids, position, caches):
        result = self.model(input_ids, cache=rebuild_cache(self.model, caches), position=position)
        return (result.logits, *flat_state(self.model, result.cache))
