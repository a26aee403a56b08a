'''ChordAttention's fused input stage (motif_chord_qkv_prep: q / k RMSNorm and the
k / v placement, straight into a preallocated StaticKVLayerCache or into new tensors
a growing cache appends) and the gated decode projection must give the results of the
unfused path (separate projections, torch RMSNorms, cache.update) -- taken here by
passing kv_states as a separate tensor of the same values.

- fp32: static-cache prefill + decode steps within 1e-5 of the KVLayerCache path,
  and the cache contents equal (same k / v rows).
- bf16: static vs general path within the bf16 bar; both against the fp64 oracle
  layer (oracle/chord.py chord_layer) for a full prefill.
- The tiny model: decoding through static caches equals decoding through the
  growing caches.
'''
import pytest
import torch

from golden.weights import fill_params
from support import assert_bf16_close, assert_fp32_close, gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _layer(dtype, H=4, Hkv=2, hidden=256, seed=3):
    from motif.block.attention.chord_attn import ChordAttention
    layer = ChordAttention(hidden_size=hidden, num_heads=H, num_kv_heads=Hkv)
    fill_params(layer, seed)
    return layer.to(DEV, dtype).eval()


def _run(layer, cache, x, splits, unfused=False):
    outs, s = [], 0
    for n in splits:
        xs = x[:, s:s + n]
        kv = xs.clone() if unfused else None
        outs.append(layer(xs, kv_states=kv, past_key_value=cache).output)
        s += n
    return torch.cat(outs, 1)


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
@torch.no_grad()
def test_static_cache_matches_general_path(dtype):
    from motif.model.cache import KVLayerCache, StaticKVLayerCache
    layer = _layer(dtype)
    B, T = 3, 40
    x = (torch.randn(B, T, 256, generator=gen(1)) * 0.5).to(DEV, dtype)
    splits = [33, 1, 1, 5]
    ref_cache = KVLayerCache()
    ref = _run(layer, ref_cache, x, splits, unfused=True)
    st = StaticKVLayerCache().allocate(B, 2, 64, 64, DEV, dtype)
    assert layer._prep_fusable(x[:, :1], None)
    out = _run(layer, st, x, splits)
    grow = _run(layer, KVLayerCache(), x, splits)
    if dtype == torch.float32:
        assert_fp32_close(grow, ref, 1e-5, 'fused growing vs unfused')
    else:
        assert_bf16_close(grow, ref, 2e-2, 5e-3, 'fused growing vs unfused')
    assert st.length == T and st.seq_length == T and int(st.length_dev.item()) == T
    k_ref, v_ref = ref_cache.k[:, :, :T], ref_cache.v[:, :, :T]
    if dtype == torch.float32:
        assert_fp32_close(out, ref, 1e-5, 'static vs general')
        assert_fp32_close(st.k[:, :, :T], k_ref, 1e-5, 'k cache')
        assert_fp32_close(st.v[:, :, :T], v_ref, 1e-5, 'v cache')
    else:
        assert_bf16_close(out, ref, 2e-2, 5e-3, 'static vs general')
        assert_bf16_close(st.k[:, :, :T], k_ref, 2e-2, 5e-3, 'k cache')
        assert_bf16_close(st.v[:, :, :T], v_ref, 2e-2, 5e-3, 'v cache')


@torch.no_grad()
def test_static_cache_prefill_matches_oracle():
    """Model-shape layer (768 wide, 12 / 3 heads): both paths against the fp64 oracle.
    The bf16 bar is scaled by the output magnitude (max-abs 2e-2 per unit of
    max|ref|, mean-rel 1e-2); the static path must also be no worse than the
    general one (same roundings, other kernels)."""
    from motif.model.cache import KVLayerCache, StaticKVLayerCache
    from oracle.chord import chord_layer
    layer = _layer(torch.bfloat16, H=12, Hkv=3, hidden=768, seed=4)
    p = {k: v.detach().double().cpu() for k, v in layer.state_dict().items()}
    x = (torch.randn(2, 70, 768, generator=gen(2)) * 0.5).to(torch.bfloat16)
    st = StaticKVLayerCache().allocate(2, 3, 80, 64, DEV, torch.bfloat16)
    out = layer(x.to(DEV), past_key_value=st).output.double().cpu()
    xd = x.to(DEV)
    gen_out = layer(xd, kv_states=xd.clone(), past_key_value=KVLayerCache()).output.double().cpu()
    ref, _, _ = chord_layer(x.double(), p, 12, 3)
    scale = max(1.0, ref.abs().max().item())
    e_st = (out - ref).abs()
    e_gen = (gen_out - ref).abs()
    assert_bf16_close(out, ref, 2e-2 * scale, 1e-2, 'static prefill vs oracle')
    assert e_st.max().item() <= 1.5 * e_gen.max().item() + 4e-3, (e_st.max().item(), e_gen.max().item())
    assert e_st.mean().item() <= 1.2 * e_gen.mean().item() + 1e-4, (e_st.mean().item(), e_gen.mean().item())


@torch.no_grad()
def test_tiny_model_static_decode_matches_growing_caches():
    from motif.model.cache import StaticKVLayerCache
    from test_gpu_layers import _tiny_model
    cfg, t, model = _tiny_model(torch.float32)
    ids = t['ids'][:, :40].to(DEV)
    dyn = model.create_cache()
    pre = model(ids[:, :32], cache=dyn).logits
    steps = [model(ids[:, i:i + 1], cache=dyn).logits for i in range(32, 40)]
    stc = model.create_cache()
    # every Chord layer gets a preallocated cache before the first call
    for b_i, block in enumerate(model.blocks):
        bc = stc[b_i]
        bc.ensure_attn([d.cache_type for d in block.features])
        for j, dec in enumerate(block.features):
            if dec.attn_type == 'chord':
                a = dec.attn
                bc.attn[j] = StaticKVLayerCache().allocate(ids.shape[0], a.num_kv_heads, 48, a.head_dim, DEV,
                                                           torch.float32)
    out_pre = model(ids[:, :32], cache=stc).logits
    out_steps = [model(ids[:, i:i + 1], cache=stc).logits for i in range(32, 40)]
    assert_fp32_close(out_pre, pre, 1e-5, 'prefill')
    assert_fp32_close(torch.cat(out_steps, 1), torch.cat(steps, 1), 1e-5, 'steps')
