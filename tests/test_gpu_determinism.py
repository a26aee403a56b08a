'''Run-to-run determinism of this build's own kernels at the benchmark shapes: every
hot-path op is launched twice on identical inputs and must return identical bits.
None of the kernels uses atomics or inter-workgroup communication (partial results are
summed in a fixed order), so any difference would mean a read of memory the launch did
not write first, or a race between launches.

- the fused GatedDelta prefill (conv, gates, chunk kernels, GatedRMSNorm) at B=64,
  T=4096 on raw projection rows, with and without incoming state and conv tails;
- Chord prefill at B=64, T=4096 (H=12, Hkv=3);
- the decode step of the 172M-shape model at B=64 over fixed-capacity caches after a
  4096-position prefill (decode projections, attention-residual reads, the GatedDelta
  decode kernel, the Chord cursor decode with its split-K merge, the vocabulary
  projection), run three times from the same cache contents.

The library GEMMs of the prefill projections are not this build's kernels and are not
covered here.'''
import pytest
import torch

from support import chord_inputs, gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _say(msg):
    print(f'[determinism] {msg}', flush=True)


@torch.no_grad()
@pytest.mark.parametrize('carry', [False, True])
def test_gdn_fused_prefill_repeats_bit_for_bit(carry):
    from motif.ops import gdn_prefill_fused
    B, T, H, dk, dv = 64, 4096, 12, 64, 128
    ncols = 2 * H * dk + 2 * H * dv + 2 * H
    g = torch.Generator(device=DEV).manual_seed(11)   # inputs made on the device (1.2 G elements)

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g, device=DEV) * scale).to(torch.bfloat16)

    proj = rnd(B, T, ncols, scale=0.5)
    offs = (0, H * dk, 2 * H * dk, 2 * H * dk + H * dv, 2 * H * dk + 2 * H * dv, 2 * H * dk + 2 * H * dv + H)
    conv = tuple(rnd(c, 1, 4, scale=0.3) for c in (H * dk, H * dk, H * dv))
    tails = tuple(rnd(B, c, 3, scale=0.5) for c in (H * dk, H * dk, H * dv)) if carry else (None, None, None)
    S = torch.randn(B, H, dk, dv, generator=g, device=DEV) * 0.1 if carry else None
    a_log, dt = rnd(H), rnd(H)
    nw = (1 + 0.1 * torch.randn(dv, generator=g, device=DEV)).to(torch.bfloat16)
    args = (proj, offs, conv, tails, a_log, dt, dk ** -0.5, nw, 1e-6, S, H, dk, dv)
    first = gdn_prefill_fused(*args)
    assert first is not None, 'the fused prefill must serve the model shape'
    for rep in range(2):
        again = gdn_prefill_fused(*args)
        assert torch.equal(first[0], again[0]), f'output, repeat {rep}'
        assert torch.equal(first[1], again[1]), f'final state, repeat {rep}'
        assert all(torch.equal(a, b) for a, b in zip(first[2], again[2])), f'conv tails, repeat {rep}'
    _say(f'gdn fused prefill B={B} T={T} carry={carry}: 3 launches, identical bits')


@torch.no_grad()
def test_chord_prefill_repeats_bit_for_bit():
    from motif.ops import apply_chord_attention
    B, H, Hkv, T = 64, 12, 3, 4096
    g = torch.Generator(device=DEV).manual_seed(12)
    q = (torch.randn(B, H, T, 64, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    k, v = ((torch.randn(B, Hkv, T, 64, generator=g, device=DEV) * 0.5).to(torch.bfloat16) for _ in range(2))
    _, _, _, alpha, beta, mu, ssmax = chord_inputs(1, H, 1, 1, 1, seed=12)
    log_n = torch.log(torch.arange(1, T + 1, dtype=torch.float32))[None].expand(B, T).contiguous()
    dev = [q, k, v] + [t.to(DEV) for t in (alpha, beta, mu, ssmax, log_n)]
    first = apply_chord_attention(*dev, q_start=0)
    for rep in range(2):
        assert torch.equal(first, apply_chord_attention(*dev, q_start=0)), f'repeat {rep}'
    _say(f'chord prefill B={B} T={T}: 3 launches, identical bits')


@torch.no_grad()
def test_model_decode_step_repeats_bit_for_bit():
    from motif.model.cache import ModelCache, StaticKVLayerCache
    from motif.model.motif import MotifChordModel
    from motif.model.presets import config_172m, init_random
    cfg = config_172m()
    model = init_random(MotifChordModel(cfg), seed=0).to(DEV, torch.bfloat16).eval()
    B, T = 64, 4096
    ids = torch.randint(0, cfg.vocab_size, (B, T + 1), generator=gen(2)).to(DEV)
    cache = ModelCache.for_decode(model, B, T + 8, DEV, torch.bfloat16)
    model(ids[:, :T], cache=cache, logits=False)
    saved = []
    for lc in cache.layer_caches():
        if isinstance(lc, StaticKVLayerCache):
            saved.append((lc.length_dev, lc.length_dev.clone()))
        else:
            saved += [(lc.state, lc.state.clone())] + [(t, t.clone()) for t in lc.conv_state]
    lengths = [lc.length for lc in cache.layer_caches()]
    seqs = [b.attn_res.seq_len for b in cache.blocks]

    def rewind():
        for dst, src in saved:
            dst.copy_(src)
        for lc, n in zip(cache.layer_caches(), lengths):
            lc.length = n
        for b, n in zip(cache.blocks, seqs):
            b.attn_res.seq_len = n

    first = model(ids[:, T:T + 1], cache=cache).logits.clone()
    for rep in range(2):
        rewind()
        again = model(ids[:, T:T + 1], cache=cache).logits
        assert torch.equal(first, again), f'decode step, repeat {rep}: {(first - again).abs().max().item()}'
    _say(f'decode step B={B} after a {T}-position prefill: 3 steps from the same caches, identical logits')
