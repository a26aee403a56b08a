'''Unified per-layer caches with the reference's public API
(motif/model/cache.py:7-847): `BasicLayerCache`, `KVLayerCache`,
`FunctionalKVLayerCache`, `GatedDeltaAttentionLayerCache`, `AttnResCache`,
`DecoderBlockCache`, `ModelCache` and `build_cache`.

Added for the hipGraph decode step (no reference counterpart):
`StaticKVLayerCache` preallocates its full capacity and keeps the cached
length both on the host and in a device int32, so a captured step can append
in place and read its position without a host sync.
'''
from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

import torch


class BasicLayerCache:
    '''Interface of every per-layer attention cache.'''

    @property
    def seq_length(self) -> int:
        raise NotImplementedError

    def reset(self) -> None:
        raise NotImplementedError

    def to(self, device: Optional[torch.device] = None, dtype: Optional[torch.dtype] = None):
        raise NotImplementedError


def _widen_heads(x: torch.Tensor, num_heads: int) -> torch.Tensor:
    '''Repeat each kv head over its query group: [B, Hkv, T, D] -> [B, num_heads, T, D].'''
    b, hkv, t, d = x.shape
    if hkv == num_heads:
        return x
    if num_heads % hkv:
        raise ValueError(f'cannot store {num_heads} heads from {hkv} grouped heads: the '
                         f'query-head count must be a multiple of the key / value head count')
    return x[:, :, None].expand(b, hkv, num_heads // hkv, t, d).reshape(b, num_heads, t, d)


class KVLayerCache(BasicLayerCache):
    '''Growable key / value cache of a Chord layer.

    The first `update` keeps the given tensors (detached); later updates copy
    into owned buffers that grow by at least a quarter (and at least 1024
    positions) when full.  `update` returns views of the valid prefix.  With
    `num_heads` the cache is wide: incoming kv heads are expanded to every
    query head on write.
    '''

    def __init__(self, num_heads: Optional[int] = None):
        self.k: Optional[torch.Tensor] = None
        self.v: Optional[torch.Tensor] = None
        self.length: int = 0
        self._owned: bool = False
        self.num_heads: Optional[int] = None if num_heads is None else int(num_heads)

    @property
    def wide(self) -> bool:
        return self.num_heads is not None

    def _prepare(self, k_new, v_new):
        if self.num_heads is None:
            return k_new, v_new
        return _widen_heads(k_new, self.num_heads), _widen_heads(v_new, self.num_heads)

    @property
    def seq_length(self) -> int:
        return self.length

    def _grow(self, dim: int, need: int):
        cur = self.k.shape[dim]
        cap = max(need, cur + max(cur // 4, 1024))
        shape = list(self.k.shape)
        shape[dim] = cap
        k_buf, v_buf = self.k.new_empty(shape), self.v.new_empty(shape)
        k_buf.narrow(dim, 0, self.length).copy_(self.k.narrow(dim, 0, self.length))
        v_buf.narrow(dim, 0, self.length).copy_(self.v.narrow(dim, 0, self.length))
        self.k, self.v = k_buf, v_buf
        self._owned = True

    def update(self, k_new: torch.Tensor, v_new: torch.Tensor, dim: int = 2) -> Tuple[torch.Tensor, torch.Tensor]:
        k_new, v_new = self._prepare(k_new, v_new)
        n = k_new.shape[dim]
        if self.k is None:
            self.k, self.v = k_new.detach(), v_new.detach()
            self.length = n
            self._owned = False
            return self.k, self.v
        if self.k.device != k_new.device:
            self.to(k_new.device)
        if not self._owned or self.length + n > self.k.shape[dim]:
            self._grow(dim, self.length + n)
        self.k.narrow(dim, self.length, n).copy_(k_new)
        self.v.narrow(dim, self.length, n).copy_(v_new)
        self.length += n
        return self.k.narrow(dim, 0, self.length), self.v.narrow(dim, 0, self.length)

    def reset(self):
        self.k = None
        self.v = None
        self.length = 0
        self._owned = False

    def to(self, device=None, dtype=None):
        if self.k is not None:
            self.k = self.k.to(device=device, dtype=dtype)
            self.v = self.v.to(device=device, dtype=dtype)
            self._owned = True
        return self

    def __repr__(self):
        heads = '' if self.num_heads is None else f', heads={self.num_heads}'
        return f'KVLayerCache(seq_length={self.length}, owned={self._owned}{heads})'


class FunctionalKVLayerCache(KVLayerCache):
    '''Key / value cache that concatenates instead of writing in place.'''

    def update(self, k_new, v_new, dim: int = 2):
        k_new, v_new = self._prepare(k_new, v_new)
        if self.k is None:
            self.k, self.v = k_new.detach(), v_new.detach()
        else:
            if self.k.device != k_new.device:
                self.to(k_new.device)
            self.k = torch.cat([self.k, k_new.detach()], dim=dim)
            self.v = torch.cat([self.v, v_new.detach()], dim=dim)
        self.length = self.k.shape[dim]
        self._owned = True
        return self.k, self.v

    def __repr__(self):
        heads = '' if self.num_heads is None else f', heads={self.num_heads}'
        return f'FunctionalKVLayerCache(seq_length={self.length}{heads})'


class StaticKVLayerCache(KVLayerCache):
    '''Fixed-capacity key / value cache for graph-captured decoding.

    `allocate(batch, kv_heads, capacity, head_dim, ...)` reserves the whole
    capacity once; `update` writes the new positions in place and returns views
    of the valid prefix like `KVLayerCache`.  `length_dev` mirrors `length` in a
    device int32 for kernels that must not depend on host values.
    '''

    def __init__(self, num_heads: Optional[int] = None):
        super().__init__(num_heads)
        self.length_dev: Optional[torch.Tensor] = None

    def allocate(self, batch, kv_heads, capacity, head_dim, device, dtype):
        self.k = torch.zeros(batch, kv_heads, capacity, head_dim, device=device, dtype=dtype)
        self.v = torch.zeros_like(self.k)
        self.length = 0
        self._owned = True
        self.length_dev = torch.zeros(1, dtype=torch.int32, device=device)
        return self

    @property
    def capacity(self) -> int:
        return 0 if self.k is None else self.k.shape[2]

    def update(self, k_new, v_new, dim: int = 2):
        if dim != 2:
            raise ValueError('StaticKVLayerCache stores positions on dim 2')
        k_new, v_new = self._prepare(k_new, v_new)
        if self.k is None:
            raise RuntimeError('StaticKVLayerCache.update before allocate()')
        n = k_new.shape[2]
        if self.length + n > self.capacity:
            raise RuntimeError(f'StaticKVLayerCache capacity {self.capacity} exceeded '
                               f'({self.length} + {n})')
        self.k[:, :, self.length:self.length + n].copy_(k_new)
        self.v[:, :, self.length:self.length + n].copy_(v_new)
        self.length += n
        self.length_dev.fill_(self.length)
        return self.k[:, :, :self.length], self.v[:, :, :self.length]

    def reserve(self, n: int) -> int:
        '''Claim the next n positions for a caller that writes them itself (the fused
        Chord input kernel, which also sets length_dev); returns the first position.'''
        if self.k is None:
            raise RuntimeError('StaticKVLayerCache.reserve before allocate()')
        if self.length + n > self.capacity:
            raise RuntimeError(f'StaticKVLayerCache capacity {self.capacity} exceeded ({self.length} + {n})')
        pos = self.length
        self.length += n
        return pos

    def reset(self):
        self.length = 0
        if self.length_dev is not None:
            self.length_dev.zero_()

    def __repr__(self):
        return f'StaticKVLayerCache(seq_length={self.length}, capacity={self.capacity})'


class GatedDeltaAttentionLayerCache(BasicLayerCache):
    '''Recurrent state (fp32 [B, H, dk, dv]) and q/k/v conv tails of a GDN layer.'''

    def __init__(self):
        self.state: Optional[torch.Tensor] = None
        self.conv_state: Optional[Tuple[torch.Tensor, ...]] = None
        self.length: int = 0

    @property
    def seq_length(self) -> int:
        return self.length

    def update(self, state: torch.Tensor, conv_state: Tuple[torch.Tensor, ...], steps: int = 1) -> torch.Tensor:
        self.state = state.detach()
        self.conv_state = tuple(c.detach() for c in conv_state)
        self.length += steps
        return self.state

    def reset(self):
        self.state = None
        self.conv_state = None
        self.length = 0

    def to(self, device=None, dtype=None):
        if self.state is not None:
            self.state = self.state.to(device=device, dtype=dtype)
        if self.conv_state is not None:
            self.conv_state = tuple(c.to(device=device, dtype=dtype) for c in self.conv_state)
        return self

    def __repr__(self):
        return (f'GatedDeltaAttentionLayerCache(seq_length={self.length}, '
                f'has_state={self.state is not None})')


@dataclass
class AttnResCache:
    '''Attention-residual history of one DecoderBlock for the current chunk.

    blocks[0] is the block input, blocks[j] (j >= 1) the increment of decoder
    j-1; partial_block is their running sum (the block output).
    '''

    blocks: List[torch.Tensor] = field(default_factory=list)
    partial_block: Optional[torch.Tensor] = None
    seq_len: int = 0
    chunk_len: int = 0

    def _cat_or_add(self, cached, new):
        if cached.shape[1] == new.shape[1]:
            return cached + new
        return torch.cat([cached, new], dim=1)

    def _align(self, entries):
        q_len = self.chunk_len if self.chunk_len > 0 else min(e.shape[1] for e in entries)
        return [e if e.shape[1] == q_len else e[:, max(e.shape[1] - q_len, 0):, :] for e in entries]

    def aligned_values(self) -> List[torch.Tensor]:
        if not self.blocks:
            raise RuntimeError('AttnResCache is empty, there is no value to read')
        return self._align(list(self.blocks))

    def values(self) -> torch.Tensor:
        return torch.stack(self.aligned_values(), dim=0)

    def init_embedding(self, hidden_states: torch.Tensor):
        q_len = hidden_states.shape[1]
        if not self.blocks:
            self.seq_len = q_len
        else:
            self.seq_len += q_len
            self.partial_block = None
        self.blocks = [hidden_states]
        self.chunk_len = q_len

    def update_increment(self, f_h: torch.Tensor, partial: Optional[torch.Tensor] = None):
        '''Append one decoder's increment and fold it into the running block sum.
        `partial` (optional, new): that sum already computed by the caller (the decode
        projection kernel folds it in its epilogue); it must equal partial_block + f_h.'''
        self.blocks.append(f_h)
        if partial is not None:
            self.partial_block = partial
        else:
            self.partial_block = f_h if self.partial_block is None else self._cat_or_add(self.partial_block, f_h)
        self.seq_len = max(self.seq_len, f_h.shape[1])

    def reset(self):
        self.blocks.clear()
        self.partial_block = None
        self.seq_len = 0
        self.chunk_len = 0

    def to(self, device=None, dtype=None):
        self.blocks = [b.to(device=device, dtype=dtype) for b in self.blocks]
        if self.partial_block is not None:
            self.partial_block = self.partial_block.to(device=device, dtype=dtype)
        return self

    def num_sources(self) -> int:
        return len(self.blocks)

    @property
    def is_empty(self) -> bool:
        return len(self.blocks) == 0

    @property
    def current_seq_len(self) -> int:
        if self.partial_block is not None:
            return self.partial_block.shape[1]
        return self.blocks[-1].shape[1] if self.blocks else 0


@dataclass
class DecoderBlockCache:
    attn_res: AttnResCache = field(default_factory=AttnResCache)
    attn: List[Optional[BasicLayerCache]] = field(default_factory=list)

    def ensure_attn(self, cache_types: Sequence[type]) -> None:
        if not self.attn:
            self.attn = [t() for t in cache_types]

    def reset(self):
        self.attn_res.reset()
        self.attn.clear()

    def is_empty(self) -> bool:
        return self.attn_res.is_empty and not self.attn

    def to(self, device=None, dtype=None):
        self.attn_res.to(device, dtype)
        for c in self.attn:
            if c is not None:
                c.to(device, dtype)
        return self

    @property
    def blocks(self):
        return self.attn_res.blocks

    @property
    def seq_len(self) -> int:
        return self.attn_res.seq_len


@dataclass
class ModelCache:
    blocks: List[DecoderBlockCache] = field(default_factory=list)

    @classmethod
    def create(cls, num_blocks: int) -> 'ModelCache':
        return cls(blocks=[DecoderBlockCache() for _ in range(num_blocks)])

    def reset(self):
        for b in self.blocks:
            b.reset()

    @property
    def seq_len(self) -> int:
        return self.blocks[0].seq_len if self.blocks else 0

    def to(self, device=None, dtype=None):
        for b in self.blocks:
            b.to(device, dtype)
        return self

    def __len__(self):
        return len(self.blocks)

    def __getitem__(self, idx):
        return self.blocks[idx]

    def __iter__(self):
        return iter(self.blocks)


def build_cache(model, use_attn: Optional[bool] = None, functional: bool = False,
                wide_kv: bool = False) -> ModelCache:
    '''One DecoderBlockCache per block; layer caches instantiated when use_attn
    (default: outside training mode).'''
    if use_attn is None:
        use_attn = not getattr(model, 'training', False)
    if not use_attn:
        return ModelCache.create(len(model.blocks))
    blocks = []
    for block in model.blocks:
        attn = []
        for decoder in block.features:
            ctype = decoder.cache_type
            if functional and issubclass(ctype, KVLayerCache):
                ctype = FunctionalKVLayerCache
            if wide_kv and issubclass(ctype, KVLayerCache):
                attn.append(ctype(num_heads=decoder.attn.num_heads))
            else:
                attn.append(ctype())
        blocks.append(DecoderBlockCache(attn=attn))
    return ModelCache(blocks=blocks)
