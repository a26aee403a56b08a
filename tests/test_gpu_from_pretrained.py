'''Weights on disk through MotifChordModel.from_pretrained on the GPU, checked against the
logits the reference itself wrote for the tiny model (tests/golden/tiny_model.safetensors,
fp32, 1e-4 as the layer fixtures):

- a plain reference-layout state_dict file (the reference's parameter names, the tied
  head stored once, no config: the config is inferred from the tensor shapes);
- the same weights written by save_pretrained (config in the file's metadata) and
  loaded back in bf16, within the bf16 layer criterion against the fp64 oracle.
The weights are the fixture's deterministic-by-name fill (tests/golden/weights.py).'''
import os

import pytest
import torch
from safetensors.torch import save_file

from golden.weights import fill_params
from support import assert_fp32_close
from test_gpu_layers import _fixture, _oracle_runs

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _reference_layout_file(tmp_path):
    '''The tiny model's weights as a plain state_dict file with the reference's names.'''
    from motif.model.config import MotifChordConfig
    from motif.model.motif import MotifChordModel
    cfg, t = _fixture('tiny_model')
    cpu = MotifChordModel(MotifChordConfig(**{**cfg, 'block': tuple(cfg['block'])}))
    fill_params(cpu, 5)
    sd = cpu.state_dict()
    tensors = {k: v.detach().clone().contiguous() for k, v in sd.items()
               if not (k == 'lm_head.weight' and cfg.get('tied_weight', True))}
    path = os.path.join(tmp_path, 'tiny_reference_layout.safetensors')
    save_file(tensors, path)
    return cfg, t, cpu, path


@torch.no_grad()
def test_from_pretrained_reference_layout_matches_reference_logits(tmp_path):
    from motif.model.motif import MotifChordModel
    cfg, t, cpu, path = _reference_layout_file(tmp_path)
    model = MotifChordModel.from_pretrained(path).to(DEV, torch.float32).eval()
    assert model.config.model_dim == cfg['model_dim'] and model.config.block_n == cfg['block_n']
    assert tuple(model.config.block) == tuple(cfg['block'])
    assert model.count_param() == cpu.count_param()
    ids = t['ids'].to(DEV)
    assert_fp32_close(model(ids).logits, t['logits_full'], 1e-4, 'from_pretrained logits_full')
    cache = model.create_cache()
    pre = model(ids[:, :75], cache=cache).logits
    steps = torch.cat([model(ids[:, i:i + 1], cache=cache).logits for i in range(75, 80)], 1)
    assert_fp32_close(pre, t['logits_pre'], 1e-4, 'from_pretrained logits_pre')
    assert_fp32_close(steps, t['logits_steps'], 1e-4, 'from_pretrained logits_steps')


@torch.no_grad()
def test_save_pretrained_round_trip_bf16(tmp_path):
    from motif.model.motif import MotifChordModel
    from support import assert_bf16_layer_close
    cfg, t, cpu, path = _reference_layout_file(tmp_path)
    first = MotifChordModel.from_pretrained(path)
    again = os.path.join(tmp_path, 'tiny_saved.safetensors')
    info = first.save_pretrained(again)
    assert info['dropped'] == ['lm_head.weight'] or not cfg.get('tied_weight', True)
    model = MotifChordModel.from_pretrained(again).to(DEV, torch.bfloat16).eval()
    for (k, a), b in zip(cpu.state_dict().items(), model.state_dict().values()):
        assert torch.equal(a.to(torch.bfloat16), b.cpu()), k
    ids = t['ids'].to(DEV)
    got = model(ids).logits
    r64, r16 = _oracle_runs(model, cfg, ids.cpu())
    assert_bf16_layer_close(got, r64, r16, 'save_pretrained round trip, bf16 logits')
