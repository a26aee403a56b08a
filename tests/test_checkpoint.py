'''Checkpoint IO (weights on disk): config inference from tensor shapes, the three file
layouts, wrapper prefixes and the published parameter counts.

The counts are those the reference's tests/test_checkpoint_compat.py:39-54 asserts for
the published 172M trunk (vocab 40,960): 172,256,480 parameters in 299 state_dict
tensors, embed / lm_head tied.  All CPU but the last test, which runs a reloaded model
on the kernels.
'''
import json

import pytest
import torch

from motif.model.checkpoint import (
    config_from_mapping, config_from_state_dict, load_checkpoint, looks_like_safetensors,
    strip_wrapper_prefixes)
from motif.model.config import MotifChordConfig
from motif.model.motif import MotifChordModel

TINY = MotifChordConfig(vocab_size=97, model_dim=64, num_heads=4, num_kv_heads=2, head_k_dim=16,
                        block=('gdn', 'chord'), block_n=2)


def _tiny(cfg=TINY, seed=0):
    torch.manual_seed(seed)
    m = MotifChordModel(cfg)
    with torch.no_grad():
        for p in m.parameters():
            p.add_(torch.randn_like(p) * 0.01)
    return m


def _same_weights(a, b):
    sa, sb = a.state_dict(), b.state_dict()
    assert sa.keys() == sb.keys()
    for k in sa:
        assert torch.equal(sa[k], sb[k]), k


@pytest.mark.parametrize('vocab,params', [(40960, 172_256_480), (32000, 165_375_200)])
def test_published_shape_counts(vocab, params):
    with torch.device('meta'):
        m = MotifChordModel(MotifChordConfig(vocab_size=vocab))
    assert m.count_param() == params
    sd = m.state_dict()
    assert len(sd) == 299
    assert config_from_state_dict(sd) == MotifChordConfig(vocab_size=vocab)


@pytest.mark.parametrize('cfg', [
    TINY,
    MotifChordConfig(vocab_size=50, model_dim=32, num_heads=2, num_kv_heads=1, head_k_dim=16,
                     block=('chord',), block_n=3),
    MotifChordConfig(vocab_size=50, model_dim=32, num_heads=2, num_kv_heads=2, head_k_dim=8,
                     block=('gdn', 'gdn'), block_n=1, tied_weight=False),
])
def test_config_from_state_dict_round_trip(cfg):
    m = _tiny(cfg)
    got = config_from_state_dict(m.state_dict())
    if cfg.block == ('chord',):   # a chord-only model leaves no trace of head_k_dim
        assert got.head_k_dim == 64
        got = MotifChordConfig(**{**got.__dict__, 'head_k_dim': cfg.head_k_dim})
    if 'chord' not in cfg.block:  # no chord layer: kv heads default to the head count
        assert got.num_kv_heads == got.num_heads
        got = MotifChordConfig(**{**got.__dict__, 'num_kv_heads': cfg.num_kv_heads})
    assert got == cfg


def test_config_errors():
    with pytest.raises(ValueError):
        config_from_state_dict({'x': torch.zeros(2)})
    with pytest.raises(ValueError):
        config_from_state_dict({'embed.weight': torch.zeros(5, 4)})


def test_strip_wrapper_prefixes():
    sd = {'module._orig_mod.embed.weight': torch.zeros(1), 'module._orig_mod.norm.weight': torch.ones(1)}
    assert set(strip_wrapper_prefixes(sd)) == {'embed.weight', 'norm.weight'}
    mixed = {'model.a': torch.zeros(1), 'b': torch.zeros(1)}   # not every key: kept
    assert set(strip_wrapper_prefixes(mixed)) == {'model.a', 'b'}


def test_config_from_mapping_aliases():
    cfg = config_from_mapping({'hidden_size': 128, 'num_hidden_layers': 2, 'num_attention_heads': 4,
                               'num_key_value_heads': 2, 'block': ['gdn', 'chord'], 'rope_theta': 1e4})
    assert (cfg.model_dim, cfg.block_n, cfg.num_heads, cfg.num_kv_heads, cfg.block) == \
        (128, 2, 4, 2, ('gdn', 'chord'))


def test_safetensors_round_trip(tmp_path):
    m = _tiny()
    path = str(tmp_path / 'm.safetensors')
    info = m.save_pretrained(path, metadata={'license': 'test'})
    assert info['dropped'] == ['lm_head.weight'] and info['params'] == m.count_param()
    assert looks_like_safetensors(path)
    loaded = load_checkpoint(path)
    assert loaded.source == 'safetensors' and loaded.config == TINY
    assert loaded.metadata['license'] == 'test'
    m2 = MotifChordModel.from_pretrained(path, verbose=False)
    assert m2.config == TINY and m2.lm_head.weight.data_ptr() == m2.embed.weight.data_ptr()
    _same_weights(m, m2)


def test_safetensors_directory_with_sidecar_config(tmp_path):
    m = _tiny()
    from safetensors.torch import save_file
    sd = {k: v.contiguous() for k, v in m.state_dict().items() if k != 'lm_head.weight'}
    save_file(sd, str(tmp_path / 'model.safetensors'))
    cfg = {**m.config.__dict__, 'block': list(m.config.block)}
    (tmp_path / 'config.json').write_text(json.dumps(cfg))
    m2 = MotifChordModel.from_pretrained(str(tmp_path), verbose=False)
    assert m2.config == TINY
    _same_weights(m, m2)


@pytest.mark.parametrize('layout', ['bare', 'prefixed', 'pipeline', 'state_dict_key'])
def test_torch_layouts(tmp_path, layout):
    m = _tiny()
    sd = m.state_dict()
    if layout == 'bare':
        obj = sd
    elif layout == 'prefixed':
        obj = {f'module.{k}': v for k, v in sd.items()}
    elif layout == 'pipeline':
        obj = {'payload': {'model': sd, 'config': {**m.config.__dict__, 'block': list(m.config.block)}},
               '__pipeline__': 'PretrainPipeline'}
    else:
        obj = {'state_dict': sd, 'step': torch.tensor(3)}
    path = str(tmp_path / 'ckpt.pt')
    torch.save(obj, path)
    loaded = load_checkpoint(path)
    assert 'embed.weight' in loaded.state_dict
    if layout == 'pipeline':
        assert loaded.config == TINY and 'pipeline' in loaded.source
    m2 = MotifChordModel.from_pretrained(path, verbose=False)
    assert m2.config == TINY
    _same_weights(m, m2)


def test_overrides_and_strict(tmp_path):
    m = _tiny()
    path = str(tmp_path / 'm.safetensors')
    m.save_pretrained(path)
    with pytest.raises(TypeError):
        MotifChordModel.from_pretrained(path, verbose=False, not_a_field=1)
    with pytest.raises(RuntimeError):   # a wider model does not match the tensors
        MotifChordModel.from_pretrained(path, verbose=False, model_dim=128)
    sd = {k: v for k, v in m.state_dict().items() if not k.startswith('norm.')}
    torch.save(sd, str(tmp_path / 'partial.pt'))
    with pytest.raises(RuntimeError):
        MotifChordModel.from_pretrained(str(tmp_path / 'partial.pt'), verbose=False, strict=True)
    MotifChordModel.from_pretrained(str(tmp_path / 'partial.pt'), verbose=False, strict=False)


class _Opaque:
    pass


def test_refuses_files_that_need_the_unpickler(tmp_path):
    path = str(tmp_path / 'evil.pt')
    torch.save({'weights': _Opaque()}, path)
    with pytest.raises(ValueError, match='weights_only'):
        load_checkpoint(path)


def test_missing_path():
    with pytest.raises(FileNotFoundError):
        load_checkpoint('/nonexistent/ckpt.pt')


@pytest.mark.gpu
def test_from_pretrained_runs_on_the_kernels(tmp_path):
    '''A saved model reloaded with from_pretrained gives the same logits on the GPU.'''
    cfg = MotifChordConfig(vocab_size=128, model_dim=256, num_heads=4, num_kv_heads=2, head_k_dim=64,
                           block=('gdn', 'chord'), block_n=1)
    m = _tiny(cfg)
    path = str(tmp_path / 'm.safetensors')
    m.save_pretrained(path)
    m2 = MotifChordModel.from_pretrained(path, device='cuda', verbose=False).to(torch.bfloat16)
    m = m.to('cuda', torch.bfloat16).eval()
    ids = torch.randint(0, 128, (2, 70), generator=torch.Generator().manual_seed(0)).cuda()
    with torch.no_grad():
        a, b = m(ids).logits, m2(ids).logits
    assert torch.equal(a, b)
