'''CPU tests of the cache classes (motif/model/cache.py): the reference's update
semantics (motif/model/cache.py:170-215, :255-302, :332-356, :487-532) and the
fixed-capacity / in-place forms the graph decode step uses.'''
import pytest
import torch

from motif.model.cache import (AttnResCache, DecoderBlockCache, FunctionalKVLayerCache,
                               GatedDeltaAttentionLayerCache, KVLayerCache, ModelCache, StaticKVLayerCache,
                               build_cache, expand_kv_heads)


def _kv(B=2, H=3, T=5, D=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, H, T, D, generator=g), torch.randn(B, H, T, D, generator=g)


def test_growing_cache_appends_and_keeps_contents_across_growth():
    c = KVLayerCache()
    ks, vs = [], []
    for i, n in enumerate([3, 1, 300, 1, 500]):
        k, v = _kv(T=n, seed=i)
        out_k, out_v = c.update(k, v)
        ks.append(k)
        vs.append(v)
        assert torch.equal(out_k, torch.cat(ks, 2)) and torch.equal(out_v, torch.cat(vs, 2))
    assert c.seq_length == 805 and c.capacity >= 805 and c.capacity % 256 == 0


def test_growing_cache_update_on_another_dim_and_detaches():
    c = KVLayerCache()
    k, v = _kv(T=4)
    k.requires_grad_(True)
    out_k, _ = c.update(k.transpose(1, 2), v.transpose(1, 2), dim=1)
    assert out_k.shape == (2, 4, 3, 4) and not out_k.requires_grad
    assert torch.equal(out_k, k.detach().transpose(1, 2))


def test_wide_cache_expands_each_kv_head_over_its_query_group():
    c = KVLayerCache(num_heads=6)
    k, v = _kv(H=2, T=3)
    out_k, out_v = c.update(k, v)
    assert c.wide and out_k.shape == (2, 6, 3, 4)
    for h in range(6):
        assert torch.equal(out_k[:, h], k[:, h // 3])
    with pytest.raises(ValueError):
        expand_kv_heads(k, 5)


def test_functional_cache_concatenates_without_padding_or_mutation():
    c = FunctionalKVLayerCache()
    k1, v1 = _kv(T=3, seed=1)
    a, _ = c.update(k1, v1)
    k2, v2 = _kv(T=4, seed=2)
    b, _ = c.update(k2, v2)
    assert b.shape[2] == 7 and c.k.shape[2] == 7 and c.seq_length == 7
    assert torch.equal(a, k1)  # the earlier result is not written into
    assert torch.equal(b, torch.cat([k1, k2], 2))


def test_assigning_k_v_adopts_them():
    c = FunctionalKVLayerCache(num_heads=3)
    k, v = _kv(T=6)
    c.k, c.v = k, v
    assert c.seq_length == 6 and torch.equal(c.k, k) and torch.equal(c.v, v)
    k2, v2 = _kv(T=1, seed=3)
    out_k, _ = c.update(k2, v2)
    assert out_k.shape[2] == 7


def test_static_cache_fixed_capacity_and_device_length():
    c = StaticKVLayerCache().allocate(2, 3, 8, 4, 'cpu', torch.float32)
    k, v = _kv(T=5)
    out_k, _ = c.update(k, v)
    assert torch.equal(out_k, k) and int(c.length_dev.item()) == 5 and c.capacity == 8
    with pytest.raises(RuntimeError, match='capacity'):
        c.update(*_kv(T=4))
    c.advance(2)
    assert c.length == 7
    with pytest.raises(RuntimeError, match='capacity'):
        c.advance(2)
    c.reset()
    assert c.length == 0 and int(c.length_dev.item()) == 0
    c.fill(*_kv(T=6))
    assert c.length == 6 and int(c.length_dev.item()) == 6


def test_gdn_cache_replaces_unless_in_place():
    c = GatedDeltaAttentionLayerCache()
    s0 = torch.zeros(1, 2, 4, 4)
    tails0 = (torch.zeros(1, 8, 3),)
    c.update(s0, tails0, steps=3)
    s1 = torch.ones(1, 2, 4, 4)
    c.update(s1, (torch.ones(1, 8, 3),), steps=1)
    assert c.state is not s0 and torch.equal(s0, torch.zeros(1, 2, 4, 4)) and c.length == 4
    p = GatedDeltaAttentionLayerCache().allocate(1, 2, 4, 4, (8, 8, 16), 4, 'cpu', torch.float32)
    keep = p.state
    p.update(torch.full((1, 2, 4, 4), 2.0), tuple(torch.ones(1, n, 3) for n in (8, 8, 16)), steps=5)
    assert p.state is keep and float(keep[0, 0, 0, 0]) == 2.0 and p.length == 5
    p.reset()
    assert p.state is keep and float(keep.abs().sum()) == 0.0 and p.length == 0


def test_attn_res_history_alignment_and_partial_sum():
    c = AttnResCache()
    with pytest.raises(RuntimeError):
        c.aligned_values()
    x = torch.randn(1, 6, 4)
    c.init_embedding(x)
    f1, f2 = torch.randn(1, 6, 4), torch.randn(1, 6, 4)
    c.update_increment(f1)
    c.update_increment(f2)
    assert c.num_sources() == 3 and torch.allclose(c.partial_block, f1 + f2) and c.seq_len == 6
    assert c.values().shape == (3, 1, 6, 4)
    # continuation: the new chunk replaces the history; seq_len keeps counting
    y = torch.randn(1, 1, 4)
    c.init_embedding(y)
    assert c.num_sources() == 1 and c.partial_block is None and c.seq_len == 7 and c.chunk_len == 1
    c.blocks.append(torch.randn(1, 6, 4))  # a longer entry is cut to the chunk's tail
    assert all(t.shape[1] == 1 for t in c.aligned_values())
    c.reset()
    assert c.is_empty and c.current_seq_len == 0


def test_attn_res_deferred_adds_equal_eager_adds():
    """update_increment(defer=True) puts the running-sum adds off; partial_block then
    sums them in registration order with one rounding per add (bf16 here), equal bit
    for bit to the add-per-increment sums, and pending_sum lists what is put off."""
    g = torch.Generator().manual_seed(3)
    fs = [(torch.randn(2, 5, 8, generator=g) * 10 ** (i % 3)).to(torch.bfloat16) for i in range(11)]
    eager, lazy = AttnResCache(), AttnResCache()
    for c in (eager, lazy):
        c.init_embedding(torch.zeros(2, 5, 8, dtype=torch.bfloat16))
    for i, f in enumerate(fs):
        eager.update_increment(f)
        lazy.update_increment(f, defer=True)
        if i == 0:
            assert lazy.pending_sum() == [f]  # the first increment is the sum itself
        if i == 2:
            assert len(lazy.pending_sum()) == 3 and torch.equal(lazy.partial_block, eager.partial_block)
            assert lazy.pending_sum() == []   # read: summed and stored
    assert len(lazy.pending_sum()) <= 8       # at most eight addends wait
    assert torch.equal(lazy.partial_block, eager.partial_block)
    assert lazy.num_sources() == eager.num_sources() == 12
    # a stored sum heads the pending list; a caller's own result replaces the list
    c = AttnResCache(partial_block=fs[0])
    c.update_increment(fs[1], defer=True)
    assert c.pending_sum() == [fs[0], fs[1]]
    c.update_increment(fs[2], partial=fs[3])
    assert c.pending_sum() == [] and c.partial_block is fs[3]
    # an increment of another shape is added at once (the stored sum first)
    c = AttnResCache(partial_block=fs[0])
    c.update_increment(fs[1], defer=True)
    c.update_increment(torch.ones(2, 1, 8, dtype=torch.bfloat16), defer=True)
    assert c.pending_sum() == [] and c.partial_block.shape == (2, 6, 8)


class _Dec:
    def __init__(self, ctype, heads=4):
        self.cache_type = ctype
        self.attn = type('A', (), {'num_heads': heads})()


class _Blk:
    def __init__(self):
        self.features = [_Dec(GatedDeltaAttentionLayerCache), _Dec(KVLayerCache)]


class _Model:
    training = False
    blocks = [_Blk(), _Blk()]


def test_build_cache_structure_and_flags():
    c = build_cache(_Model())
    assert isinstance(c, ModelCache) and len(c) == 2 and all(isinstance(b, DecoderBlockCache) for b in c)
    assert [type(x) for x in c[0].attn] == [GatedDeltaAttentionLayerCache, KVLayerCache]
    f = build_cache(_Model(), functional=True, wide_kv=True)
    assert type(f[1].attn[1]) is FunctionalKVLayerCache and f[1].attn[1].num_heads == 4
    t = build_cache(_Model(), use_attn=False)
    assert all(b.attn == [] for b in t)
    c.reset()
    assert all(b.is_empty() for b in c) and c.seq_len == 0


def test_chord_only_model_prefills_on_the_cpu():
    '''A decoder block of Chord layers runs on CPU tensors (the materialised attention
    path): the ROCm-only prefill steps and the second-stream fork stand aside.'''
    from motif.model.config import MotifChordConfig
    from motif.model.motif import MotifChordModel
    import motif.block.decoder as decmod
    cfg = MotifChordConfig(vocab_size=50, model_dim=64, num_heads=2, num_kv_heads=1, head_k_dim=32,
                           block=('chord', 'chord'), block_n=1)
    model = MotifChordModel(cfg).eval().to(torch.bfloat16)
    with torch.no_grad():
        out = model(torch.randint(0, 50, (1, 9), generator=torch.Generator().manual_seed(0)))
    assert out.logits.shape == (1, 9, 50) and bool(torch.isfinite(out.logits.float()).all())
    assert decmod._Fork(torch.device('cpu')).on is False
