'''Pin the oracle's layer / model composition against fixtures written by the
reference implementation (tests/golden/make_layer_fixtures.py, float32 CPU).

The parameters come from tests/golden/weights.py by name on this build's own
module trees (same names as the reference), so this also checks that the
module trees and parameter names line up.
'''
import json
import os

import pytest
import torch
from safetensors.torch import load_file, safe_open

from golden.weights import fill_params
from oracle.chord import chord_layer
from oracle.gdn import gdn_layer
from oracle.model import OracleModel

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')
D64 = torch.float64


def _fixture(name):
    path = os.path.join(GOLD, f'{name}.safetensors')
    with safe_open(path, 'pt') as f:
        cfg = json.loads(f.metadata()['config'])
    return cfg, load_file(path)


def _close(a, b, tol=2e-5):
    a, b = a.double(), b.double()
    err = (a - b).abs().max().item()
    scale = b.abs().max().item()
    assert err <= tol * max(1.0, scale), f'max abs err {err:.3e} (scale {scale:.3e})'


def gdn_params(cfg, seed=1):
    from motif.block.attention.gdn_attn import GatedDeltaAttention
    layer = GatedDeltaAttention(**cfg)
    fill_params(layer, seed)
    return layer, {k: v.detach().double() for k, v in layer.state_dict().items()}


def chord_params(cfg, seed=3):
    from motif.block.attention.chord_attn import ChordAttention
    layer = ChordAttention(**cfg)
    fill_params(layer, seed)
    return layer, {k: v.detach().double() for k, v in layer.state_dict().items()}


def model_params(cfg, seed=5):
    from motif.model.config import MotifChordConfig
    from motif.model.motif import MotifChordModel
    model = MotifChordModel(MotifChordConfig(**{**cfg, 'block': tuple(cfg['block'])})).eval()
    fill_params(model, seed)
    return model, {k: v.detach().double() for k, v in model.state_dict().items()}


def test_gdn_layer_oracle_matches_reference():
    cfg, t = _fixture('gdn_layer')
    _, p = gdn_params(cfg)
    H, dk = cfg['num_heads'], cfg['head_k_dim']
    x = t['x'].double()
    out, S, conv = gdn_layer(x, p, H, dk, 2 * dk)
    _close(out, t['out_full'])
    _close(S, t['state_full'])
    _close(conv[0], t['conv_q_full'])
    _close(conv[2], t['conv_v_full'])
    # continuation: prefill 100, then 30, then three single tokens
    o1, S1, c1 = gdn_layer(x[:, :100], p, H, dk, 2 * dk)
    o2, S2, c2 = gdn_layer(x[:, 100:], p, H, dk, 2 * dk, S1, c1)
    _close(o1, t['out_pre'])
    _close(o2, t['out_mid'])
    steps, S, c = [], S2, c2
    for i in range(3):
        o, S, c = gdn_layer(t['steps'][:, i:i + 1].double(), p, H, dk, 2 * dk, S, c)
        steps.append(o)
    _close(torch.cat(steps, 1), t['out_steps'])
    _close(S, t['state_end'])
    _close(c[2], t['conv_v_end'])


def test_chord_layer_oracle_matches_reference():
    cfg, t = _fixture('chord_layer')
    _, p = chord_params(cfg)
    H, Hkv = cfg['num_heads'], cfg['num_kv_heads']
    x = t['x'].double()
    out, _, _ = chord_layer(x, p, H, Hkv)
    _close(out, t['out_full'])
    o1, kc, vc = chord_layer(x[:, :50], p, H, Hkv)
    o2, kc, vc = chord_layer(x[:, 50:], p, H, Hkv, kc, vc)
    _close(o1, t['out_pre'])
    _close(o2, t['out_mid'])
    steps = []
    for i in range(2):
        o, kc, vc = chord_layer(t['steps'][:, i:i + 1].double(), p, H, Hkv, kc, vc)
        steps.append(o)
    _close(torch.cat(steps, 1), t['out_steps'])
    _close(kc, t['k_end'])


def test_model_oracle_matches_reference():
    cfg, t = _fixture('tiny_model')
    _, p = model_params(cfg)
    om = OracleModel(p, cfg)
    # six layers + the head in float32 on the reference side: ~3e-5 of rounding noise
    _close(om.forward(t['ids']), t['logits_full'], 1e-4)
    om.reset()
    _close(om.forward(t['ids'][:, :75]), t['logits_pre'], 1e-4)
    steps = [om.forward(t['ids'][:, i:i + 1]) for i in range(75, 80)]
    _close(torch.cat(steps, 1), t['logits_steps'], 1e-4)


def test_parameter_count_of_published_shape():
    '''172,256,480 parameters at the reference shape (tests/test_checkpoint_compat.py:41),
    165,375,200 with the 32000 vocabulary of the benchmark configs.'''
    from motif.model.config import MotifChordConfig
    from motif.model.motif import MotifChordModel
    assert MotifChordModel(MotifChordConfig()).count_param() == 172_256_480
    assert MotifChordModel(MotifChordConfig(vocab_size=32000)).count_param() == 165_375_200


@pytest.mark.parametrize('name', ['gdn_layer', 'chord_layer', 'tiny_model'])
def test_fixtures_are_small_and_safe(name):
    path = os.path.join(GOLD, f'{name}.safetensors')
    assert os.path.getsize(path) < 1_000_000


def test_attn_res_read_bruteforce():
    '''oracle.model.attn_res_read against scalar loops of its definition
    (softmax over sources of q . (w * x / rms(x)), then the weighted sum).'''
    import math
    from oracle.model import attn_res_read
    g = torch.Generator().manual_seed(3)
    N, B, T, D, eps = 3, 2, 4, 8, 1e-6
    srcs = [torch.randn(B, T, D, generator=g, dtype=torch.float64) for _ in range(N)]
    q = torch.randn(D, generator=g, dtype=torch.float64)
    w = torch.randn(D, generator=g, dtype=torch.float64)
    out = attn_res_read(srcs, q, w, eps)
    for b in range(B):
        for t in range(T):
            s = []
            for n in range(N):
                x = [float(srcs[n][b, t, d]) for d in range(D)]
                r = 1.0 / math.sqrt(sum(v * v for v in x) / D + eps)
                s.append(sum(float(q[d]) * float(w[d]) * x[d] * r for d in range(D)))
            m = max(s)
            e = [math.exp(v - m) for v in s]
            a = [v / sum(e) for v in e]
            for d in range(D):
                h = sum(a[n] * float(srcs[n][b, t, d]) for n in range(N))
                assert abs(h - float(out[b, t, d])) < 1e-12
    assert attn_res_read(srcs[:1], q, w, eps) is srcs[0]
