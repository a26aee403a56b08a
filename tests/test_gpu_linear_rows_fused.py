'''The decoder's batched decode projections against the launches they replace:

- motif_linear_rows_pair (attention input projection + MLP gate/up with SwiGLU in one
  launch) equals the two motif_linear_rows calls bit for bit;
- motif_linear_rows_dual (o_proj -- gated for Chord -- + MLP down projection + the
  residual fold) equals motif_linear_rows with the gate / no epilogue followed by the
  resid epilogue bit for bit, and the float64 formula within the bf16 bar;
- a decode step of the 172M model through the split step (pair, core, dual) equals
  the same step run layer by layer, logits and caches bit for bit.

motif_linear_rows itself is pinned to the float64 formula by test_gpu_linear_rows.py.'''
import pytest
import torch

from support import assert_bf16_close, gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _bf(*shape, seed, scale=0.5):
    return (torch.randn(*shape, generator=gen(seed)) * scale).to(DEV, torch.bfloat16)


@pytest.mark.parametrize('M', [1, 17, 64])
@pytest.mark.parametrize('N1,epi1', [(4632, 'none'), (2304, 'none'), (3072, 'swiglu')])
@torch.no_grad()
def test_pair_equals_two_launches(M, N1, epi1):
    from motif.ops.linear_rows import linear_rows, linear_rows_pair
    K = 768
    x1, x2 = _bf(M, K, seed=1), _bf(M, K, seed=2)
    w1, w2 = _bf(N1, K, seed=3, scale=0.05), _bf(4096, K, seed=4, scale=0.05)
    y1, y2 = linear_rows_pair(x1, w1, x2, w2, epi1)
    assert torch.equal(y1, linear_rows(x1, w1, epi1))
    assert torch.equal(y2, linear_rows(x2, w2, 'swiglu'))


@torch.no_grad()
def test_pair_keeps_leading_shape_and_strided_rows():
    from motif.ops.linear_rows import linear_rows, linear_rows_pair
    base = _bf(64, 1, 1024, seed=5)
    x1 = base[..., :768]                      # row stride 1024
    x2 = _bf(64, 1, 768, seed=6)
    w1, w2 = _bf(2304, 768, seed=7, scale=0.05), _bf(4096, 768, seed=8, scale=0.05)
    y1, y2 = linear_rows_pair(x1, w1, x2, w2)
    assert y1.shape == (64, 1, 2304) and y2.shape == (64, 1, 2048)
    assert torch.equal(y1, linear_rows(x1.contiguous(), w1))
    assert torch.equal(y2, linear_rows(x2, w2, 'swiglu'))


@pytest.mark.parametrize('M', [1, 5, 64])
@pytest.mark.parametrize('K1', [1536, 768])
@pytest.mark.parametrize('gated', [False, True])
@pytest.mark.parametrize('with_sum', [False, True])
@torch.no_grad()
def test_dual_equals_two_launches(M, K1, gated, with_sum):
    from motif.ops.linear_rows import linear_rows, linear_rows_dual
    N, K2 = 768, 2048
    x1, x2 = _bf(M, K1, seed=11), _bf(M, K2, seed=12)
    w1, w2 = _bf(N, K1, seed=13, scale=0.03), _bf(N, K2, seed=14, scale=0.03)
    gate = _bf(M, N, seed=15, scale=2.0) if gated else None
    prev = _bf(M, N, seed=16) if with_sum else None
    f, p = linear_rows_dual(x1, w1, x2, w2, gate=gate, aux2=prev)
    u = linear_rows(x1, w1, 'gate', aux=gate) if gated else linear_rows(x1, w1)
    if with_sum:
        f_ref, p_ref = linear_rows(x2, w2, 'resid', aux=u, aux2=prev)
        assert torch.equal(p, p_ref)
    else:
        f_ref, p = linear_rows(x2, w2, 'resid', aux=u), p
        assert p is None
    assert torch.equal(f, f_ref), (f.float() - f_ref.float()).abs().max().item()
    # the formula in float64
    e = x1.double() @ w1.double().T
    if gated:
        e = e * torch.sigmoid(gate.double())
    e = e + x2.double() @ w2.double().T
    assert_bf16_close(f, e, what='dual vs float64')


@torch.no_grad()
def test_dual_gate_as_strided_view():
    '''Chord hands the gate over as a column slice of its projection output.'''
    from motif.ops.linear_rows import linear_rows, linear_rows_dual
    proj = _bf(64, 1, 2304 + 768, seed=21)
    gate = proj[..., 2304:]
    x1, x2 = _bf(64, 1, 768, seed=22), _bf(64, 1, 2048, seed=23)
    w1, w2 = _bf(768, 768, seed=24, scale=0.03), _bf(768, 2048, seed=25, scale=0.03)
    f, p = linear_rows_dual(x1, w1, x2, w2, gate=gate)
    u = linear_rows(x1, w1, 'gate', aux=gate.contiguous())
    assert p is None and torch.equal(f, linear_rows(x2, w2, 'resid', aux=u))


@torch.no_grad()
def test_split_decode_step_equals_layer_by_layer(monkeypatch):
    import motif.block.decoder as dec
    from motif.model.cache import ModelCache
    from motif.model.motif import MotifChordModel
    from motif.model.presets import config_172m, init_random
    model = init_random(MotifChordModel(config_172m()), seed=3).to(DEV, torch.bfloat16).eval()
    n_decoders = sum(isinstance(mod, dec.Decoder) for mod in model.modules())
    B, n_pre, n_dec = 64, 40, 3
    ids = torch.randint(0, model.config.vocab_size, (B, n_pre + n_dec), generator=gen(4)).to(DEV)
    calls = []
    real = dec._split_step

    def counted(*a, **k):
        r = real(*a, **k)
        calls.append(r is not None)
        return r

    def run(split):
        monkeypatch.setattr(dec, '_split_step', counted if split else (lambda *a, **k: None))
        cache = ModelCache.for_decode(model, B, n_pre + n_dec + 8, DEV, torch.bfloat16)
        model(ids[:, :n_pre], cache=cache)
        logits = torch.cat([model(ids[:, i:i + 1], cache=cache).logits for i in range(n_pre, n_pre + n_dec)], 1)
        states = [lc.state.clone() if hasattr(lc, 'state') else lc._slab[0][:, :, :n_pre + n_dec].clone()
                  for lc in cache.layer_caches()]
        return logits, states

    split = run(True)
    assert sum(calls) == n_dec * n_decoders, 'every decode step of every decoder should take the split step'
    plain = run(False)
    assert torch.equal(split[0], plain[0]), (split[0].float() - plain[0].float()).abs().max().item()
    for a, b in zip(split[1], plain[1]):
        assert torch.equal(a, b)
