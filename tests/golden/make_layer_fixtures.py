'''Write the layer / model composition fixtures from the reference implementation.

Runs ONLY in the build container, where the reference is mounted read-only at
/root/reference; the reference never travels to the GPU box.  The fixtures pin
what no closed form fixes: the composition inside GatedDeltaAttention.forward,
ChordAttention.forward, DecoderBlock.forward and MotifChordModel.forward
(order of conv / SiLU / normalise / gates, GatedRMSNorm layout, the q/k RMSNorm
and sigmoid gate of Chord, log_n indexing, the attention-residual read, cache
continuation).  Weights come from tests/golden/weights.py (deterministic by
parameter name), so only inputs and outputs are stored.

Usage: python tests/golden/make_layer_fixtures.py  (writes tests/golden/*.safetensors)
'''
import json
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get('MOTIF_REFERENCE', '/root/reference')
sys.path.insert(0, REF)
sys.path.insert(0, HERE)

from safetensors.torch import save_file  # noqa: E402

from weights import fill_params  # noqa: E402

torch.set_grad_enabled(False)
torch.manual_seed(0)


def gdn_fixture():
    from motif.block.attention.gdn_attn import GatedDeltaAttention
    from motif.model.cache import GatedDeltaAttentionLayerCache
    cfg = dict(hidden_size=128, num_heads=2, head_k_dim=64, expand_v=2.0, conv_size=4, chunk_size=64)
    layer = GatedDeltaAttention(**cfg).float()
    fill_params(layer, seed=1)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 130, 128, generator=g)
    steps = torch.randn(2, 3, 128, generator=g)
    full = layer(x)
    cache = GatedDeltaAttentionLayerCache()
    pre = layer(x[:, :100], past_key_value=cache)
    mid = layer(x[:, 100:], past_key_value=cache)
    outs = [layer(steps[:, i:i + 1], past_key_value=cache).output for i in range(3)]
    t = {
        'x': x, 'steps': steps,
        'out_full': full.output, 'state_full': full.payload['state'],
        'conv_q_full': full.payload['conv_state'][0], 'conv_k_full': full.payload['conv_state'][1],
        'conv_v_full': full.payload['conv_state'][2],
        'out_pre': pre.output, 'out_mid': mid.output, 'out_steps': torch.cat(outs, 1),
        'state_end': cache.state, 'conv_v_end': cache.conv_state[2],
    }
    return cfg, t


def chord_fixture():
    from motif.block.attention.chord_attn import ChordAttention
    from motif.model.cache import KVLayerCache
    cfg = dict(hidden_size=256, num_heads=4, num_kv_heads=2)
    layer = ChordAttention(**cfg).float()
    fill_params(layer, seed=3)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 70, 256, generator=g)
    steps = torch.randn(2, 2, 256, generator=g)
    full = layer(x)
    cache = KVLayerCache()
    pre = layer(x[:, :50], past_key_value=cache)
    mid = layer(x[:, 50:], past_key_value=cache)
    outs = [layer(steps[:, i:i + 1], past_key_value=cache).output for i in range(2)]
    t = {'x': x, 'steps': steps, 'out_full': full.output, 'out_pre': pre.output, 'out_mid': mid.output,
         'out_steps': torch.cat(outs, 1), 'k_end': cache.k[:, :, :cache.length], 'v_end': cache.v[:, :, :cache.length]}
    return cfg, t


def model_fixture():
    from motif.model.config import MotifChordConfig
    from motif.model.motif import MotifChordModel
    cfg = dict(vocab_size=256, model_dim=128, num_heads=2, num_kv_heads=1, head_k_dim=64,
               block=('gdn', 'chord', 'gdn'), block_n=2)
    model = MotifChordModel(MotifChordConfig(**{**cfg, 'block': tuple(cfg['block'])})).float().eval()
    fill_params(model, seed=5)
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, 256, (2, 80), generator=g)
    full = model(ids)
    cache = model.create_cache()
    pre = model(ids[:, :75], cache=cache)
    steps = []
    for i in range(75, 80):
        steps.append(model(ids[:, i:i + 1], cache=cache).logits)
    t = {'ids': ids, 'logits_full': full.logits, 'logits_pre': pre.logits, 'logits_steps': torch.cat(steps, 1)}
    return cfg, t


def main():
    for name, fn in (('gdn_layer', gdn_fixture), ('chord_layer', chord_fixture), ('tiny_model', model_fixture)):
        cfg, tensors = fn()
        meta = {'config': json.dumps(cfg), 'source': 'reference CPU path, float32'}
        path = os.path.join(HERE, f'{name}.safetensors')
        save_file({k: v.contiguous() for k, v in tensors.items()}, path, metadata=meta)
        print(path, os.path.getsize(path))


if __name__ == '__main__':
    main()
