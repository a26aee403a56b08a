'''The prefill's second stream (motif.block.decoder._Fork): while a graph is captured each
decoder's MLP branch runs on a second stream beside the attention layer.  A captured
config-3-shaped prefill, replayed several times with eager forwards (no fork) between the
replays, gives the eager logits bit for bit on every replay, and every decoder's step
forked during the capture.
'''
import pytest
import torch

from support import gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'


@pytest.mark.parametrize('B,T', [(1, 1024), (2, 384)])
@torch.no_grad()
def test_captured_prefill_with_fork_equals_eager(B, T):
    import motif.block.decoder as decmod
    from motif.model.motif import MotifChordModel
    from motif.model.presets import config_172m, init_random
    model = init_random(MotifChordModel(config_172m()), seed=2).to(DEV, torch.bfloat16).eval()
    ids = torch.randint(0, model.config.vocab_size, (B, T), generator=gen(12)).to(DEV)
    eager = model(ids).logits.clone()
    forks = []
    real = decmod._Fork

    class Counted(real):
        def __init__(self, device):
            super().__init__(device)
            forks.append(self.on)
    decmod._Fork = Counted
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            model(ids)  # warm-up outside the capture (no fork: not capturing)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        assert forks and not any(forks)
        forks.clear()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = model(ids)
    finally:
        decmod._Fork = real
    assert len(forks) == 16 and all(forks), forks
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.logits, eager), f'replay {i}'
        assert torch.equal(model(ids).logits, eager), f'eager after replay {i}'
        torch.cuda.synchronize()


@torch.no_grad()
def test_fork_is_joined_when_a_step_bails_out():
    '''A prefill step that forks and then finds its layer route unserved joins the side
    stream before returning None: the capture around it ends cleanly.'''
    import motif.block.decoder as decmod
    from motif.model.cache import AttnResCache
    from motif.model.motif import MotifChordModel
    from motif.model.presets import config_172m, init_random
    model = init_random(MotifChordModel(config_172m()), seed=3).to(DEV, torch.bfloat16).eval()
    gdn, chord = model.blocks[0].features[0], model.blocks[0].features[3]
    g = gen(13)
    x = torch.randn(1, 256, 768, generator=g).to(DEV, torch.bfloat16)
    m = torch.randn(1, 256, 768, generator=g).to(DEV, torch.bfloat16)
    gdn.attn.prefill_core = lambda *a, **k: False
    chord.attn.prefill_parts = lambda *a, **k: None
    try:
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            assert decmod._prefill_step(gdn, x, m, None) is None
            assert decmod._chord_prefill_step(chord, x, m, None, None, 0, AttnResCache()) is None
        graph.replay()
        torch.cuda.synchronize()
    finally:
        del gdn.attn.prefill_core, chord.attn.prefill_parts
