'''The decoder's GatedDelta prefill step (motif.block.decoder._prefill_step): the layer's
o_proj and the MLP's down projection as one GEMM over [y | s], the sum accumulated in
fp32 and rounded once, against the reference's form (two GEMMs, each rounded, then
added; the layer forward followed by SwiGLU.forward_residual) at the 172M model's shapes.

- f_h is within one bf16 rounding of the float64 sum of the same two products (the
  reference's form is three roundings away);
- the layer cache the step updates (state and conv tails, from zero and carried on
  from a first chunk) equals the layer forward's bit for bit;
- inside a whole model prefill (config-3 model, T = 1024) every GatedDelta decoder's
  step passes the first check on the inputs it saw.
'''
import pytest
import torch

from support import gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _model():
    from motif.model.motif import MotifChordModel
    from motif.model.presets import config_172m, init_random
    return init_random(MotifChordModel(config_172m()), seed=0).to(DEV, torch.bfloat16).eval()


def _exact(decoder, x, m):
    '''float64 [y | s] [W_o | W_down]^T from the same kernels' y and s.'''
    from motif.ops.epilogue import swiglu
    attn, mlp = decoder.attn, decoder.mlp
    B, L, _ = x.shape
    y = torch.empty(B, L, attn.o_proj.in_features, dtype=x.dtype, device=x.device)
    assert attn.prefill_core(x, None, y)
    s = swiglu(torch.nn.functional.linear(m, mlp.gate_up_proj.weight))
    return (y.double() @ attn.o_proj.weight.double().t()) + (s.double() @ mlp.down_proj.weight.double().t())


def _check_one(decoder, x, m, f, what):
    f64 = _exact(decoder, x, m)
    d = (f.double() - f64).abs()
    bound = 2.0 ** -8 * f64.abs() + 1e-5 * f64.abs().max()
    assert bool((d <= bound).all()), f'{what}: f_h off by {(d - bound).max().item():.3e} past one rounding'
    attn_out = decoder.attn(hidden_states=x).output
    f_ref, _ = decoder.mlp.forward_residual(m, attn_out, None)
    e_fused, e_ref = d.mean().item(), (f_ref.double() - f64).abs().mean().item()
    print(f'{what}: mean |f_h - exact| fused {e_fused:.3e}, two roundings then add {e_ref:.3e}', flush=True)
    assert e_fused <= e_ref, what


@torch.no_grad()
@pytest.mark.parametrize('L', [4096, 1000])
def test_prefill_step_one_decoder(L):
    from motif.block.decoder import _prefill_step
    model = _model()
    dec = model.blocks[0].features[1]
    g = gen(3)
    x = torch.randn(1, L, 768, generator=g).to(DEV, torch.bfloat16)
    m = torch.randn(1, L, 768, generator=g).to(DEV, torch.bfloat16)
    f = _prefill_step(dec, x, m, None)
    _check_one(dec, x, m, f, f'one decoder, L={L}')


@torch.no_grad()
def test_prefill_step_cache_equals_layer_forward():
    from motif.block.decoder import _prefill_step
    from motif.model.cache import GatedDeltaAttentionLayerCache
    model = _model()
    dec = model.blocks[1].features[0]
    g = gen(4)
    xs = [torch.randn(1, n, 768, generator=g).to(DEV, torch.bfloat16) for n in (700, 333)]
    ms = [torch.randn(1, n, 768, generator=g).to(DEV, torch.bfloat16) for n in (700, 333)]
    c_step, c_layer = GatedDeltaAttentionLayerCache(), GatedDeltaAttentionLayerCache()
    for i, (x, m) in enumerate(zip(xs, ms)):
        assert _prefill_step(dec, x, m, c_step) is not None
        dec.attn(hidden_states=x, past_key_value=c_layer)
        assert torch.equal(c_step.state, c_layer.state), f'chunk {i}: state'
        assert all(torch.equal(a, b) for a, b in zip(c_step.conv_state, c_layer.conv_state)), f'chunk {i}: tails'


@torch.no_grad()
def test_prefill_step_inside_a_model_prefill():
    import motif.block.decoder as decmod
    model = _model()
    ids = torch.randint(0, model.config.vocab_size, (1, 1024), generator=gen(6)).to(DEV)
    calls = []
    real = decmod._prefill_step

    def record(decoder, x, m, layer_cache):
        out = real(decoder, x, m, layer_cache)
        if out is not None:
            calls.append((decoder, x.clone(), m.clone(), out))
        return out
    decmod._prefill_step = record
    try:
        model(ids)
    finally:
        decmod._prefill_step = real
    assert len(calls) == 12, 'every GatedDelta decoder prefills through the step'
    for i, (decoder, x, m, f) in enumerate(calls):
        _check_one(decoder, x, m, f, f'model prefill, GatedDelta decoder {i}')
