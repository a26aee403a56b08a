'''Per-layer caches of the Motif Chord model.

Public surface of motif/model/cache.py:7-847 (class names, constructor
arguments, attributes and methods the layers and callers use): BasicLayerCache,
KVLayerCache, FunctionalKVLayerCache, GatedDeltaAttentionLayerCache,
AttnResCache, DecoderBlockCache, ModelCache and build_cache.

Design.  A key / value cache is a slab `[B, heads, capacity, D]` plus a cursor
(the number of valid positions).  The three key / value classes differ only in
how the slab gets room for new positions:

  * KVLayerCache            grows: the capacity doubles, in whole 256-position
                            pages, and the valid prefix moves once per doubling;
  * FunctionalKVLayerCache  never writes in place: every append builds a new
                            tensor of exactly the valid length (traceable);
  * StaticKVLayerCache      one allocation for the whole run; the cursor is also
                            kept in a device int32 (`length_dev`), the value the
                            Chord decode kernels read and advance, so a decode
                            step captured once as a hipGraph can be replayed token
                            after token without host involvement.

`append_slots(n)` hands the slab and the first free position to a writer (the
fused Chord input kernel writes new keys / values straight into the cache);
`update()` is append_slots plus a copy.

GatedDeltaAttentionLayerCache replaces its tensors on `update` (the state a
caller received before stays untouched) unless it was made `in_place`, the form
graph-captured decoding needs: then the state and conv tails keep their
storage and the decode kernel updates them there.

`ModelCache.for_decode(model, batch, capacity, ...)` builds the fixed-capacity
form of the whole cache (static key / value slabs, in-place recurrent state).
'''
from typing import Iterator, List, Optional, Sequence, Tuple

import torch

from motif.ops.epilogue import MAX_CHAIN, residual_fold

PAGE = 256  # positions per allocation unit of a growing key / value slab


def _pages(n: int) -> int:
    return max(PAGE, -(-n // PAGE) * PAGE)


class BasicLayerCache:
    '''What every per-layer cache provides: its length, `reset` and `to`.'''

    @property
    def seq_length(self) -> int:
        raise NotImplementedError

    def reset(self) -> None:
        raise NotImplementedError

    def to(self, device: Optional[torch.device] = None, dtype: Optional[torch.dtype] = None):
        raise NotImplementedError


def expand_kv_heads(x: torch.Tensor, num_heads: int) -> torch.Tensor:
    '''Grouped keys / values `[B, Hkv, T, D]` to one copy per query head: query head
    h reads kv head h // (num_heads / Hkv), so each kv head is repeated over a
    consecutive run of query heads (the grouping motif/ops/chord_attention.py:154 uses).'''
    hkv = x.shape[1]
    if hkv == num_heads:
        return x
    if num_heads % hkv != 0:
        raise ValueError(f'a wide cache of {num_heads} heads needs a whole number of query heads '
                         f'per kv head; the projection has {hkv} kv heads')
    return torch.repeat_interleave(x, num_heads // hkv, dim=1)


class KVLayerCache(BasicLayerCache):
    '''Key / value cache of a Chord layer (growing slab).

    `k` / `v` are the valid prefix `[B, heads, length, D]`.  With `num_heads` the
    cache is wide: incoming kv heads are expanded to every query head on write.
    '''

    def __init__(self, num_heads: Optional[int] = None):
        self.num_heads: Optional[int] = None if num_heads is None else int(num_heads)
        self.length: int = 0
        self._slab: Optional[Tuple[torch.Tensor, torch.Tensor]] = None

    # ---- storage policy (overridden by the other forms)
    def _room(self, like: torch.Tensor, n: int) -> None:
        '''Make room for n more positions in a slab shaped like `like` [B, h, *, D].'''
        need = self.length + n
        if self._slab is not None and self._slab[0].shape[2] >= need:
            return
        cap = _pages(max(need, 2 * (0 if self._slab is None else self._slab[0].shape[2])))
        shape = (like.shape[0], like.shape[1], cap, like.shape[3])
        k = torch.empty(shape, dtype=like.dtype, device=like.device)
        v = torch.empty(shape, dtype=like.dtype, device=like.device)
        if self._slab is not None and self.length:
            k[:, :, :self.length].copy_(self._slab[0][:, :, :self.length])
            v[:, :, :self.length].copy_(self._slab[1][:, :, :self.length])
        self._slab = (k, v)

    # ---- public surface
    @property
    def wide(self) -> bool:
        return self.num_heads is not None

    @property
    def seq_length(self) -> int:
        return self.length

    @property
    def capacity(self) -> int:
        return 0 if self._slab is None else self._slab[0].shape[2]

    @property
    def k(self) -> Optional[torch.Tensor]:
        return None if self._slab is None else self._slab[0][:, :, :self.length]

    @property
    def v(self) -> Optional[torch.Tensor]:
        return None if self._slab is None else self._slab[1][:, :, :self.length]

    def adopt(self, k: torch.Tensor, v: torch.Tensor) -> None:
        '''Make the given tensors the whole cache content (length = k.shape[2]).'''
        self._slab = (k, v)
        self.length = k.shape[2]

    @k.setter
    def k(self, value):
        self._slab = None if value is None else (value, self._slab[1] if self._slab else value)
        self.length = 0 if value is None else value.shape[2]

    @v.setter
    def v(self, value):
        if value is None:
            self._slab = None
            self.length = 0
        else:
            self._slab = (self._slab[0] if self._slab else value, value)

    def append_slots(self, n: int, like: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, int]:
        '''Reserve n positions: returns (k slab, v slab, first position).  The caller
        writes positions [first, first + n) of both slabs; the cursor already counts them.'''
        if self._slab is not None and self._slab[0].device != like.device:
            self.to(like.device)
        self._room(like, n)
        first = self.length
        self.length += n
        return self._slab[0], self._slab[1], first

    def update(self, k_new: torch.Tensor, v_new: torch.Tensor, dim: int = 2) -> Tuple[torch.Tensor, torch.Tensor]:
        '''Append new keys / values (detached) along `dim`; returns every cached position.'''
        if dim != 2:
            k, v = self.update(k_new.movedim(dim, 2), v_new.movedim(dim, 2), 2)
            return k.movedim(2, dim), v.movedim(2, dim)
        if self.wide:
            k_new, v_new = expand_kv_heads(k_new, self.num_heads), expand_kv_heads(v_new, self.num_heads)
        n = k_new.shape[2]
        ks, vs, first = self.append_slots(n, k_new)
        ks[:, :, first:first + n].copy_(k_new.detach())
        vs[:, :, first:first + n].copy_(v_new.detach())
        return self.k, self.v

    def reset(self):
        self._slab = None
        self.length = 0

    def to(self, device=None, dtype=None):
        if self._slab is not None:
            self._slab = tuple(t[:, :, :self.length].to(device=device, dtype=dtype).contiguous()
                               for t in self._slab)
        return self

    def __repr__(self):
        kind = f'wide x{self.num_heads}' if self.wide else 'grouped'
        return f'{type(self).__name__}<{kind}>(positions={self.length}/{self.capacity})'


class FunctionalKVLayerCache(KVLayerCache):
    '''Key / value cache that never writes in place: every update returns new tensors
    holding exactly the valid positions (a traced step can take them as inputs).'''

    def update(self, k_new, v_new, dim: int = 2):
        if self.wide:
            k_new = expand_kv_heads(k_new.movedim(dim, 2), self.num_heads).movedim(2, dim)
            v_new = expand_kv_heads(v_new.movedim(dim, 2), self.num_heads).movedim(2, dim)
        k_new, v_new = k_new.detach(), v_new.detach()
        if self._slab is None:
            k, v = k_new, v_new
        else:
            old_k, old_v = self._slab
            if old_k.device != k_new.device:
                old_k, old_v = old_k.to(k_new.device), old_v.to(k_new.device)
            k, v = torch.cat((old_k, k_new), dim), torch.cat((old_v, v_new), dim)
        self._slab = (k, v)
        self.length = k.shape[dim]
        return k, v

    def append_slots(self, n, like):
        raise TypeError('FunctionalKVLayerCache has no writable slots; use update()')

    @property
    def k(self):
        return None if self._slab is None else self._slab[0]

    @property
    def v(self):
        return None if self._slab is None else self._slab[1]

    @k.setter
    def k(self, value):
        KVLayerCache.k.fset(self, value)

    @v.setter
    def v(self, value):
        KVLayerCache.v.fset(self, value)

    def to(self, device=None, dtype=None):
        if self._slab is not None:
            self._slab = tuple(t.to(device=device, dtype=dtype) for t in self._slab)
        return self


class StaticKVLayerCache(KVLayerCache):
    '''Fixed-capacity key / value cache for graph-captured decoding (new; the
    reference's caches grow on the host).

    `allocate(batch, kv_heads, capacity, head_dim, device, dtype)` reserves the slab
    once.  The cursor lives twice: `length` on the host and `length_dev` (int32) on
    the device.  On the kernel path the device value is the authority: the Chord
    input kernel writes new keys at `length_dev`, the decode kernel attends over
    `length_dev + L` keys and advances `length_dev`.  A captured step replayed n
    times advances the device cursor n times; `advance(n)` brings the host mirror
    along (ModelCache.advance does it for every layer).
    '''

    def __init__(self, num_heads: Optional[int] = None):
        super().__init__(num_heads)
        self.length_dev: Optional[torch.Tensor] = None
        self.decode_workspace: Optional[torch.Tensor] = None
        self.step_workspace: Optional[torch.Tensor] = None  # the fused decode step's (zeroed once)

    def allocate(self, batch, kv_heads, capacity, head_dim, device, dtype):
        shape = (batch, kv_heads, capacity, head_dim)
        self._slab = (torch.zeros(shape, device=device, dtype=dtype), torch.zeros(shape, device=device, dtype=dtype))
        self.length = 0
        self.length_dev = torch.zeros(1, dtype=torch.int32, device=device)
        self.decode_workspace = None
        self.step_workspace = None
        return self

    def _room(self, like, n):
        if self._slab is None:
            raise RuntimeError('StaticKVLayerCache: allocate() before writing')
        if self.length + n > self.capacity:
            raise RuntimeError(f'StaticKVLayerCache: {self.length} + {n} positions exceed the '
                               f'capacity of {self.capacity}')

    def update(self, k_new, v_new, dim: int = 2):
        out = super().update(k_new, v_new, dim)
        self.length_dev.fill_(self.length)
        return out

    def fill(self, k: torch.Tensor, v: torch.Tensor) -> None:
        '''Set the first k.shape[2] positions (and both cursors) from given tensors.'''
        n = k.shape[2]
        self._room(k, n - self.length)
        self._slab[0][:, :, :n].copy_(k)
        self._slab[1][:, :, :n].copy_(v)
        self.length = n
        self.length_dev.fill_(n)

    def advance(self, n: int) -> None:
        '''Host mirror of n positions appended by replayed kernels.'''
        if self.length + n > self.capacity:
            raise RuntimeError(f'StaticKVLayerCache: {self.length} + {n} positions exceed the '
                               f'capacity of {self.capacity}')
        self.length += n

    def reset(self):
        self.length = 0
        if self.length_dev is not None:
            self.length_dev.zero_()

    def to(self, device=None, dtype=None):
        if self._slab is not None:
            self._slab = tuple(t.to(device=device, dtype=dtype) for t in self._slab)
            self.length_dev = self.length_dev.to(device=device)
        return self


class GatedDeltaAttentionLayerCache(BasicLayerCache):
    '''Recurrent state (fp32 `[B, H, dk, dv]`) and the q / k / v conv tails
    (`[B, channels, K-1]`) of a GatedDelta layer, plus the processed length.

    `update` stores detached tensors in place of the previous ones.  An `in_place`
    cache keeps its storage instead: updates copy into it, and the fused decode
    kernel writes the new state and tails there directly.
    '''

    def __init__(self, in_place: bool = False):
        self.state: Optional[torch.Tensor] = None
        self.conv_state: Optional[Tuple[torch.Tensor, ...]] = None
        self.length: int = 0
        self.in_place = bool(in_place)

    @property
    def seq_length(self) -> int:
        return self.length

    def allocate(self, batch, heads, dk, dv, conv_channels: Sequence[int], conv_size, device, dtype):
        '''Zero state and tails (an in-place cache that has seen nothing).'''
        self.state = torch.zeros(batch, heads, dk, dv, dtype=torch.float32, device=device)
        self.conv_state = tuple(torch.zeros(batch, c, conv_size - 1, dtype=dtype, device=device)
                                for c in conv_channels)
        self.length = 0
        self.in_place = True
        return self

    def update(self, state: torch.Tensor, conv_state: Tuple[torch.Tensor, ...], steps: int = 1) -> torch.Tensor:
        keep = (self.in_place and self.state is not None and self.conv_state is not None
                and self.state.shape == state.shape and len(self.conv_state) == len(conv_state)
                and all(a.shape == b.shape for a, b in zip(self.conv_state, conv_state)))
        if keep:
            if state is not self.state:
                self.state.copy_(state.detach())
            for dst, src in zip(self.conv_state, conv_state):
                if src is not dst:
                    dst.copy_(src.detach())
        else:
            self.state = state.detach()
            self.conv_state = tuple(c.detach() for c in conv_state)
        self.length += steps
        return self.state

    def advance(self, n: int) -> None:
        self.length += n

    def reset(self):
        if self.in_place and self.state is not None:
            self.state.zero_()
            for t in self.conv_state:
                t.zero_()
        else:
            self.state, self.conv_state = None, None
        self.length = 0

    def to(self, device=None, dtype=None):
        if self.state is not None:
            self.state = self.state.to(device=device, dtype=dtype)
        if self.conv_state is not None:
            self.conv_state = tuple(t.to(device=device, dtype=dtype) for t in self.conv_state)
        return self

    def __repr__(self):
        shape = 'empty' if self.state is None else 'x'.join(map(str, self.state.shape))
        return f'GatedDeltaAttentionLayerCache(positions={self.length}, state={shape}, in_place={self.in_place})'


def _last(t: torch.Tensor, n: int) -> torch.Tensor:
    return t if t.shape[1] == n else t[:, t.shape[1] - min(n, t.shape[1]):]


class AttnResCache:
    '''Attention-residual history of one DecoderBlock for the current chunk.

    `blocks[0]` is the block input and `blocks[j]` (j >= 1) the increment f_h of
    decoder j-1, each `[B, q_len, D]`; decoder i reads the first i+1 entries.
    `partial_block` is the running sum of the increments (the block output).
    `seq_len` counts every position the block has processed, `chunk_len` the
    positions of the current forward.
    '''

    def __init__(self, blocks: Optional[List[torch.Tensor]] = None, partial_block: Optional[torch.Tensor] = None,
                 seq_len: int = 0, chunk_len: int = 0):
        self.blocks: List[torch.Tensor] = [] if blocks is None else list(blocks)
        self._chain: List[torch.Tensor] = []  # addends of the running sum not yet summed
        self.partial_block = partial_block
        self.seq_len = seq_len
        self.chunk_len = chunk_len

    @property
    def partial_block(self) -> Optional[torch.Tensor]:
        '''The running sum of the increments.  Increments registered with `defer=True`
        are added here, on first access, in one pass: one add and one rounding each, in
        registration order (motif.ops.epilogue.residual_fold), so the value equals the
        add-per-increment one.'''
        if self._chain:
            chain, self._chain = self._chain, []
            self._partial = chain[0] if len(chain) == 1 else residual_fold(None, None, chain=chain)[1]
        return self._partial

    @partial_block.setter
    def partial_block(self, value: Optional[torch.Tensor]) -> None:
        self._partial = value
        self._chain = []

    def pending_sum(self) -> List[torch.Tensor]:
        '''The running sum's addends that are not summed yet, in order (the stored sum
        first, when there is one); empty when no add is put off.  A caller that folds
        them into its own pass registers its result with update_increment(f_h, partial).'''
        return list(self._chain)

    def aligned_values(self) -> List[torch.Tensor]:
        '''Every source, each cut to the last `chunk_len` positions (the shortest entry's
        length when no chunk is registered).'''
        if not self.blocks:
            raise RuntimeError('AttnResCache.aligned_values: no block input registered yet')
        n = self.chunk_len if self.chunk_len > 0 else min(b.shape[1] for b in self.blocks)
        return [_last(b, n) for b in self.blocks]

    def values(self) -> torch.Tensor:
        return torch.stack(self.aligned_values())

    def init_embedding(self, hidden_states: torch.Tensor) -> None:
        '''Start a forward: the input becomes the only source and the previous forward's
        increments are dropped; `seq_len` keeps counting.'''
        n = hidden_states.shape[1]
        self.seq_len = n if not self.blocks else self.seq_len + n
        if self.blocks:
            self.partial_block = None
        self.blocks = [hidden_states]
        self.chunk_len = n

    def update_increment(self, f_h: torch.Tensor, partial: Optional[torch.Tensor] = None,
                         defer: bool = False) -> None:
        '''Register decoder output f_h.  `partial` (new, optional) is partial_block + f_h
        already computed by the caller (the decode projection kernel folds it in).
        `defer` (new): put the add partial_block + f_h off until partial_block is read
        or a caller folds pending_sum() into its own pass (same value; up to
        MAX_CHAIN adds are summed in one pass).'''
        self.blocks.append(f_h)
        if partial is None and defer and not self._chain and (
                self._partial is None or self._partial.shape == f_h.shape):
            self._chain = ([self._partial] if self._partial is not None else []) + [f_h]
            return
        if partial is None and defer and self._chain and len(self._chain) < MAX_CHAIN and \
                self._chain[0].shape == f_h.shape:
            self._chain.append(f_h)
            return
        if partial is None:
            prev = self.partial_block
            if prev is None:
                partial = f_h
            elif prev.shape[1] == f_h.shape[1]:
                partial = prev + f_h
            else:
                partial = torch.cat((prev, f_h), dim=1)
        self.partial_block = partial
        if f_h.shape[1] > self.seq_len:
            self.seq_len = f_h.shape[1]

    def reset(self) -> None:
        self.blocks = []
        self.partial_block = None
        self.seq_len = self.chunk_len = 0

    def to(self, device=None, dtype=None):
        self.blocks = [b.to(device=device, dtype=dtype) for b in self.blocks]
        if self.partial_block is not None:
            self.partial_block = self.partial_block.to(device=device, dtype=dtype)
        return self

    def num_sources(self) -> int:
        return len(self.blocks)

    @property
    def is_empty(self) -> bool:
        return not self.blocks

    @property
    def current_seq_len(self) -> int:
        newest = self.partial_block if self.partial_block is not None else (self.blocks[-1] if self.blocks else None)
        return 0 if newest is None else newest.shape[1]

    def __repr__(self):
        return f'AttnResCache(sources={len(self.blocks)}, positions={self.seq_len}, chunk={self.chunk_len})'


class DecoderBlockCache:
    '''The attention-residual history and the per-layer caches of one DecoderBlock.'''

    def __init__(self, attn_res: Optional[AttnResCache] = None, attn: Optional[List[Optional[BasicLayerCache]]] = None):
        self.attn_res = AttnResCache() if attn_res is None else attn_res
        self.attn: List[Optional[BasicLayerCache]] = [] if attn is None else list(attn)

    def ensure_attn(self, cache_types: Sequence[type]) -> None:
        '''Create one cache per layer if none exist yet (existing ones are kept).'''
        if not self.attn:
            self.attn = [make() for make in cache_types]

    def reset(self) -> None:
        self.attn_res.reset()
        self.attn = []

    def is_empty(self) -> bool:
        return self.attn_res.is_empty and not self.attn

    def to(self, device=None, dtype=None):
        self.attn_res.to(device, dtype)
        for layer_cache in filter(None, self.attn):
            layer_cache.to(device, dtype)
        return self

    @property
    def blocks(self) -> List[torch.Tensor]:
        return self.attn_res.blocks

    @property
    def seq_len(self) -> int:
        return self.attn_res.seq_len

    def __repr__(self):
        return f'DecoderBlockCache({self.attn_res!r}, layers={[type(c).__name__ for c in self.attn]})'


class ModelCache:
    '''The cache of a whole model: one DecoderBlockCache per block.'''

    def __init__(self, blocks: Optional[List[DecoderBlockCache]] = None):
        self.blocks: List[DecoderBlockCache] = [] if blocks is None else list(blocks)

    @classmethod
    def create(cls, num_blocks: int) -> 'ModelCache':
        return cls([DecoderBlockCache() for _ in range(num_blocks)])

    @classmethod
    def for_decode(cls, model, batch: int, capacity: int, device, dtype) -> 'ModelCache':
        '''Fixed-capacity cache of `model` for graph-captured decoding (new): a
        StaticKVLayerCache of `capacity` positions per Chord layer, an in-place
        GatedDelta cache with zero state and tails per GatedDelta layer.'''
        blocks = []
        for block in model.blocks:
            layers = []
            for decoder in block.features:
                attn = decoder.attn
                if issubclass(decoder.cache_type, KVLayerCache):
                    layers.append(StaticKVLayerCache().allocate(batch, attn.num_kv_heads, capacity, attn.head_dim,
                                                                device, dtype))
                else:
                    chans = (attn.num_heads * attn.dk, attn.num_heads * attn.dk, attn.num_heads * attn.dv)
                    layers.append(GatedDeltaAttentionLayerCache().allocate(
                        batch, attn.num_heads, attn.dk, attn.dv, chans, attn.conv_size, device, dtype))
            blocks.append(DecoderBlockCache(attn=layers))
        return cls(blocks)

    def layer_caches(self) -> Iterator[BasicLayerCache]:
        for block in self.blocks:
            yield from filter(None, block.attn)

    def advance(self, n: int) -> None:
        '''Host bookkeeping of n positions processed by replayed kernels (a captured
        decode step): layer cursors and every block's position count.'''
        for layer_cache in self.layer_caches():
            layer_cache.advance(n)
        for block in self.blocks:
            block.attn_res.seq_len += n

    def reset(self) -> None:
        for block in self.blocks:
            block.reset()

    @property
    def seq_len(self) -> int:
        return self.blocks[0].seq_len if self.blocks else 0

    def to(self, device=None, dtype=None):
        for block in self.blocks:
            block.to(device, dtype)
        return self

    def __len__(self):
        return len(self.blocks)

    def __getitem__(self, idx):
        return self.blocks[idx]

    def __iter__(self):
        return iter(self.blocks)

    def __repr__(self):
        return f'ModelCache(blocks={len(self.blocks)}, positions={self.seq_len})'


def build_cache(model, use_attn: Optional[bool] = None, functional: bool = False,
                wide_kv: bool = False) -> ModelCache:
    '''The cache of `model` (anything with `training` and `blocks[i].features[j].cache_type`).

    use_attn: create the per-layer caches (default: outside training mode).
    functional: Chord layers keep keys / values by concatenation (traceable).
    wide_kv: Chord layers store keys / values expanded to every query head.
    '''
    if use_attn is None:
        use_attn = not getattr(model, 'training', False)
    cache = ModelCache.create(len(model.blocks))
    if not use_attn:
        return cache
    kv_type = FunctionalKVLayerCache if functional else None

    def make(decoder):
        ctype = decoder.cache_type
        if not issubclass(ctype, KVLayerCache):
            return ctype()
        ctype = kv_type or ctype
        return ctype(num_heads=decoder.attn.num_heads) if wide_kv else ctype()

    for block_cache, block in zip(cache.blocks, model.blocks):
        block_cache.attn = [make(d) for d in block.features]
    return cache
