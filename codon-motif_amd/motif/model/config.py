'''Model hyper-parameters; same fields and defaults as the reference's
motif/model/config.py:5-39.'''
from dataclasses import dataclass
from typing import Literal, Optional, Tuple


@dataclass
class MotifChordConfig:
    vocab_size: int = 5 * (2 ** 13)
    model_dim: int = 768
    num_heads: int = 12
    num_kv_heads: Optional[int] = 3
    head_k_dim: Optional[int] = 64
    tied_weight: bool = True
    block: Tuple[Literal['chord', 'gdn'], ...] = ('gdn', 'gdn', 'gdn', 'chord')
    block_n: int = 4
