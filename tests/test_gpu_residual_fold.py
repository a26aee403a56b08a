'''The residual fold (motif_residual_fold) and the model prefill around it:

- the kernel equals the reference's separate ops bit for bit (the Chord output gate
  a * sigmoid(g), f_h = that + the MLP output, then one add per running-sum addend, in
  order, each rounded to the dtype): bf16 and fp32, with and without the gate, 0 to 8
  addends, the sum of addends alone, operands that are column views of wider rows (fp32
  with the gate within 1e-6: the fp32 sigmoid may differ from torch's in the last bit);
- a model prefill with the running-sum adds of the GatedDelta decoders put off and
  folded into the Chord decoder's pass equals, bit for bit, the same prefill with one
  add per decoder and the Chord output gate as its own pass (config-3 model, T = 1024,
  two batch rows; and a 2-block model of 3 GatedDelta + 1 Chord decoders whose last
  decoder is a GatedDelta one, so partial_block sums the put-off adds itself).
'''
import pytest
import torch

from support import gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _ref(a, g, b, chain):
    f = None
    if a is not None:
        f = (a if g is None else a * torch.sigmoid(g)) + b
    p = None
    if chain:
        p = chain[0]
        for c in list(chain[1:]) + ([f] if f is not None else []):
            p = p + c
    return f, p


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@pytest.mark.parametrize('gate', [True, False])
@pytest.mark.parametrize('n', [0, 1, 2, 5, 8])
@torch.no_grad()
def test_fold_equals_separate_ops(dtype, gate, n):
    from motif.ops.epilogue import residual_fold
    g = gen(n + 10 * gate)
    M, N = 1000, 768
    wide = (torch.randn(M, 3 * N, generator=g) * 4).to(DEV, dtype)   # a and the gate as column views
    a, gt = wide[:, :N], wide[:, 2 * N:]
    b = torch.randn(M, N, generator=g).to(DEV, dtype)
    chain = [(torch.randn(M, N, generator=g) * 10 ** (j % 3 - 1)).to(DEV, dtype) for j in range(n)]
    f, p = residual_fold(a, b, gate=gt if gate else None, chain=chain)
    f_ref, p_ref = _ref(a, gt if gate else None, b, chain)
    assert (p is None) == (n == 0)
    if gate and dtype == torch.float32:
        # fp32 sigmoid: torch's kernel and 1 / (1 + expf(-g)) may differ in the last bit
        torch.testing.assert_close(f, f_ref, rtol=1e-6, atol=1e-6)
        if n:
            torch.testing.assert_close(p, p_ref, rtol=1e-6, atol=1e-5)
        return
    assert torch.equal(f, f_ref)
    if n:
        assert torch.equal(p, p_ref)


@pytest.mark.parametrize('n', [2, 3, 8])
@torch.no_grad()
def test_fold_of_addends_only(n):
    from motif.ops.epilogue import residual_fold
    g = gen(40 + n)
    chain = [(torch.randn(2, 333, 768, generator=g) * 3).to(DEV, torch.bfloat16) for _ in range(n)]
    f, p = residual_fold(None, None, chain=chain)
    assert f is None and torch.equal(p, _ref(None, None, None, chain)[1])


def _both_ways(model, ids):
    '''Logits and block outputs of a prefill with the put-off adds and the fused Chord
    pass, then without them (one add per decoder, the gate as its own pass).'''
    import motif.block.decoder as decmod
    from motif.model.cache import AttnResCache
    outs = []
    for lazy in (True, False):
        blocks = []
        hooks = [b.register_forward_hook(lambda mod, inp, out: blocks.append(out.hidden_states.clone()))
                 for b in model.blocks]
        real_step, real_upd = decmod._chord_prefill_step, AttnResCache.update_increment
        if not lazy:
            decmod._chord_prefill_step = lambda *a, **k: None
            AttnResCache.update_increment = lambda self, f, partial=None, defer=False: real_upd(self, f, partial)
        try:
            logits = model(ids).logits
        finally:
            decmod._chord_prefill_step, AttnResCache.update_increment = real_step, real_upd
            for h in hooks:
                h.remove()
        outs.append((logits, blocks))
    return outs


@torch.no_grad()
def test_model_prefill_equals_add_per_decoder():
    from motif.model.motif import MotifChordModel
    from motif.model.presets import config_172m, init_random
    model = init_random(MotifChordModel(config_172m()), seed=0).to(DEV, torch.bfloat16).eval()
    ids = torch.randint(0, model.config.vocab_size, (2, 1024), generator=gen(9)).to(DEV)
    import motif.block.decoder as decmod
    calls = []
    real = decmod._chord_prefill_step

    def count(*a, **k):
        out = real(*a, **k)
        calls.append(out is not None)
        return out
    decmod._chord_prefill_step = count
    try:
        (lz, lz_blocks), (eg, eg_blocks) = _both_ways(model, ids)
    finally:
        decmod._chord_prefill_step = real
    assert calls[:4] == [True] * 4, 'every Chord decoder takes the fused pass'
    assert len(lz_blocks) == len(eg_blocks) == 4
    for i, (a, b) in enumerate(zip(lz_blocks, eg_blocks)):
        assert torch.equal(a, b), f'block {i}'
    assert torch.equal(lz, eg)


@torch.no_grad()
def test_block_ending_in_gated_delta_sums_put_off_adds():
    from motif.model.config import MotifChordConfig
    from motif.model.motif import MotifChordModel
    from motif.model.presets import init_random
    cfg = MotifChordConfig(vocab_size=32000, model_dim=768, num_heads=12, num_kv_heads=3, head_k_dim=64,
                           block=('gdn', 'chord', 'gdn', 'gdn'), block_n=2)
    model = init_random(MotifChordModel(cfg), seed=1).to(DEV, torch.bfloat16).eval()
    ids = torch.randint(0, cfg.vocab_size, (1, 700), generator=gen(10)).to(DEV)
    (lz, lz_blocks), (eg, eg_blocks) = _both_ways(model, ids)
    for i, (a, b) in enumerate(zip(lz_blocks, eg_blocks)):
        assert torch.equal(a, b), f'block {i}'
    assert torch.equal(lz, eg)


@torch.no_grad()
def test_fold_edge_shapes():
    '''Empty rows, rows the kernel does not serve (a width that is not a multiple of 16
    bytes: the torch ops run), and nine addends (past the kernel's eight: torch ops) all
    give the separate ops' values.'''
    from motif.ops.epilogue import residual_fold
    g = gen(50)
    for M, N, n in ((0, 768, 3), (37, 100, 2), (64, 768, 9)):
        a, b, gt = ((torch.randn(M, N, generator=g) * 2).to(DEV, torch.bfloat16) for _ in range(3))
        chain = [torch.randn(M, N, generator=g).to(DEV, torch.bfloat16) for _ in range(n)]
        f, p = residual_fold(a, b, gate=gt, chain=chain)
        f_ref, p_ref = _ref(a, gt, b, chain)
        assert torch.equal(f, f_ref) and torch.equal(p, p_ref), (M, N, n)


@torch.no_grad()
def test_elementwise_stages_take_empty_rows():
    from motif.ops.epilogue import add_fold, mul_sigmoid, swiglu
    e = torch.empty(1, 0, 768, dtype=torch.bfloat16, device=DEV)
    assert swiglu(torch.empty(1, 0, 1536, dtype=torch.bfloat16, device=DEV)).shape == (1, 0, 768)
    assert mul_sigmoid(e, e).shape == e.shape
    f, p = add_fold(e, e, e)
    assert f.shape == p.shape == e.shape
