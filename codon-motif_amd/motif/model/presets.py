'''Model shapes and synthetic inputs of the benchmark configurations.

- `config_172m`: the published model shape (d=768, 4 blocks x (3 GatedDelta + 1
  Chord), 12 heads, GDN dk=64 / dv=128, Chord D=64 with 3 kv heads, SwiGLU 2048) at
  a chosen vocabulary (32000 in the benchmark configurations).
- `init_random`: random initialisation of a model with no checkpoint, wholly
  determined by the seed: every Linear / Embedding / Conv1d weight ~ N(0, std) and
  the GatedDelta decay parameters (A_log, dt_bias: their constructor distributions)
  from one seeded CPU generator; the other semantic parameters (theta_*, ssmax_s,
  pseudo-queries, norms) keep their constant constructor values, so the recurrence
  stays in its designed regime.  (The constructor draws A_log / dt_bias from the
  global RNG, whose seed differs from process to process.)
- `packed_lengths`: the sequence lengths of the packed prefill configuration
  (uniform in [lo, hi], seeded).
'''
from typing import List

import torch
import torch.nn as nn

from motif.model.config import MotifChordConfig


def config_172m(vocab_size: int = 32000) -> MotifChordConfig:
    return MotifChordConfig(vocab_size=vocab_size, model_dim=768, num_heads=12, num_kv_heads=3, head_k_dim=64,
                            block=('gdn', 'gdn', 'gdn', 'chord'), block_n=4)


def init_random(model: nn.Module, std: float = 0.02, seed: int = 0) -> nn.Module:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, (nn.Linear, nn.Embedding, nn.Conv1d)):
                m.weight.copy_(torch.randn(m.weight.shape, generator=g) * std)
            elif hasattr(m, 'init_gates'):
                m.init_gates(g)
    return model


def packed_lengths(n: int = 16, lo: int = 512, hi: int = 8192, seed: int = 0) -> List[int]:
    g = torch.Generator().manual_seed(seed)
    return [int(x) for x in torch.randint(lo, hi + 1, (n,), generator=g)]


def cu_seqlens_of(lengths: List[int]) -> torch.Tensor:
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return torch.tensor(cu, dtype=torch.int32)
