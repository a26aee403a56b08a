'''One decode step of a MotifChordModel captured once as a HIP graph and replayed
token after token (new; the reference's decode step is not graph-capturable,
motif/model/generate.py:138-171 with the host-side cache lengths of
motif/model/cache.py:144-215).

The step runs over a fixed-capacity cache (`ModelCache.for_decode`): every Chord
layer appends at, attends up to and advances its device cursor, every GatedDelta
layer updates its state and conv tails in place.  The launch sequence is
therefore the same for every token, so one capture serves the whole decode; only
host bookkeeping (`ModelCache.advance`) runs between replays.
'''
from typing import Optional

import torch

from motif.model.cache import GatedDeltaAttentionLayerCache, ModelCache, StaticKVLayerCache


def _check_static(cache: ModelCache) -> None:
    for lc in cache.layer_caches():
        if isinstance(lc, StaticKVLayerCache):
            if lc.capacity == 0:
                raise ValueError('DecodeGraph: a StaticKVLayerCache is not allocated')
        elif isinstance(lc, GatedDeltaAttentionLayerCache):
            if not lc.in_place or lc.state is None:
                raise ValueError('DecodeGraph: GatedDelta caches must be in-place with allocated state '
                                 '(use ModelCache.for_decode)')
        else:
            raise ValueError(f'DecodeGraph: {type(lc).__name__} cannot be replayed (use ModelCache.for_decode)')


class _Snapshot:
    '''Device state a warm-up step changes: cursors, recurrent states, conv tails
    (key / value rows written past the cursor are overwritten by the next real step).'''

    def __init__(self, cache: ModelCache):
        self.cache = cache
        self.lengths = [lc.length for lc in cache.layer_caches()]
        self.seq = [b.attn_res.seq_len for b in cache.blocks]
        self.saved = []
        for lc in cache.layer_caches():
            if isinstance(lc, StaticKVLayerCache):
                self.saved.append((lc.length_dev, lc.length_dev.clone()))
            else:
                self.saved.append((lc.state, lc.state.clone()))
                self.saved.extend((t, t.clone()) for t in lc.conv_state)

    def restore_device(self):
        for dst, src in self.saved:
            dst.copy_(src)

    def restore_host(self):
        for lc, n in zip(self.cache.layer_caches(), self.lengths):
            lc.length = n
        for b, n in zip(self.cache.blocks, self.seq):
            b.attn_res.seq_len = n


class DecodeGraph:
    '''`step(tokens [B, 1]) -> logits [B, 1, vocab]` for `model` over `cache`.

    The returned logits tensor is the graph's output buffer: the next step
    overwrites it (clone it to keep it).  Steps past the cache capacity raise.
    '''

    def __init__(self, model, cache: ModelCache, batch: int, device=None):
        _check_static(cache)
        self.model, self.cache, self.batch = model, cache, batch
        device = torch.device(device) if device is not None else next(model.parameters()).device
        self.tokens = torch.zeros(batch, 1, dtype=torch.long, device=device)
        self.capacity = min((lc.capacity for lc in cache.layer_caches() if isinstance(lc, StaticKVLayerCache)),
                            default=None)
        snap = _Snapshot(cache)
        kv = [lc for lc in cache.layer_caches() if isinstance(lc, StaticKVLayerCache)]
        for lc in kv:
            lc.cursor_steps = 0
        # warm-up step (lazy set-up: fused weights, workspaces, tables), undone after.  It
        # runs on the current stream, so the tensors it creates and keeps (cached fused
        # weights, the decode workspaces) belong to the pool of the stream that later uses
        # them: the caching allocator then cannot hand their memory to another stream while
        # this one's kernels may still read it.  (With the warm-up on a side stream, runs
        # after a capture now and then differed from the same runs before it.)
        with torch.no_grad():
            model(self.tokens, cache=cache)
        snap.restore_device()
        snap.restore_host()
        if any(lc.cursor_steps != 1 for lc in kv):
            raise ValueError('DecodeGraph: a Chord layer did not decode on its device cursor (the HIP kernels '
                             'serve bf16 / fp32 with head_dim 64); its replays would not advance')
        torch.cuda.synchronize(device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph):
            self.logits = model(self.tokens, cache=cache).logits
        snap.restore_host()  # capture recorded the step without running it

    @property
    def position(self) -> int:
        return self.cache.seq_len

    def step(self, tokens: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self.capacity is not None:
            used = max(lc.length for lc in self.cache.layer_caches() if isinstance(lc, StaticKVLayerCache))
            if used + 1 > self.capacity:
                raise RuntimeError(f'DecodeGraph: the cache capacity of {self.capacity} positions is used up')
        if tokens is not None:
            self.tokens.copy_(tokens.view(self.batch, 1))
        self.graph.replay()
        self.cache.advance(1)
        return self.logits
