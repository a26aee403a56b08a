'''AttentionOutput and BasicAttention with the reference interface
(motif/block/attention/base.py:10-118).'''
from dataclasses import dataclass
from typing import Any, Optional

import torch
import torch.nn as nn

from motif.model.cache import BasicLayerCache


@dataclass
class AttentionOutput:
    output: torch.Tensor
    attention_weights: Optional[torch.Tensor] = None
    past_key_value: Optional[Any] = None
    payload: Optional[dict] = None


class BasicAttention(nn.Module):
    '''Head layout shared by the attention layers.'''

    def __init__(self, hidden_size: int, num_heads: int, num_kv_heads: Optional[int] = None, **kwargs):
        super().__init__()
        num_kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        assert hidden_size % num_heads == 0, \
            f'hidden_size {hidden_size} must be divisible by num_heads {num_heads}'
        assert num_heads % num_kv_heads == 0, \
            f'num_heads {num_heads} must be divisible by num_kv_heads {num_kv_heads}'
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = hidden_size // num_heads
        self.kv_dim = num_kv_heads * self.head_dim
        self.num_kv_queries = num_heads // num_kv_heads

    @classmethod
    def cache_type(cls):
        return BasicLayerCache

    def reshape_q(self, q, q_len, batch_size):
        return q.view(batch_size, q_len, self.num_heads, self.head_dim).transpose(1, 2)

    def reshape_kv(self, x, kv_len, batch_size):
        return x.view(batch_size, kv_len, self.num_kv_heads, self.head_dim).transpose(1, 2)
