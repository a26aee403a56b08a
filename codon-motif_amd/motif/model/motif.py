'''MotifChordModel: the integration harness for the full-model configurations.

Same module tree and parameter names as the reference (motif/model/motif.py:154-630:
embed, blocks, norm, tied lm_head) and the same forward contract
(input_ids, cache, labels, mask, position) -> ModelOutput.  Generation,
sampling and checkpoint IO are outside this build.
'''
from dataclasses import dataclass
from typing import Optional, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from motif.block.decoder import DecoderBlock
from motif.model.cache import ModelCache, build_cache
from motif.model.config import MotifChordConfig
from motif.ops import RMSNorm


@dataclass
class ModelOutput:
    hidden_states: torch.Tensor
    logits: Optional[torch.Tensor] = None
    loss: Optional[torch.Tensor] = None
    cache: Optional[ModelCache] = None

    @property
    def last_logits(self):
        return None if self.logits is None else self.logits[:, -1, :]

    def next_token(self) -> Optional[torch.Tensor]:
        '''Greedy next token [B, 1].'''
        return None if self.logits is None else self.logits[:, -1, :].argmax(dim=-1, keepdim=True)


class MotifChordModel(nn.Module):
    def __init__(self, config: MotifChordConfig):
        super().__init__()
        self.config = config
        self.embed = nn.Embedding(config.vocab_size, config.model_dim)
        self.blocks = nn.ModuleList([DecoderBlock(config) for _ in range(config.block_n)])
        self.norm = RMSNorm(config.model_dim)
        self.lm_head = nn.Linear(config.model_dim, config.vocab_size, bias=False)
        if config.tied_weight:
            self.embed.weight = self.lm_head.weight

    def count_param(self) -> int:
        return sum(p.numel() for p in {id(p): p for p in self.parameters()}.values())

    def cache_types(self):
        return [[d.cache_type for d in b.features] for b in self.blocks]

    def create_cache(self, use_attn: Optional[bool] = None, functional: bool = False,
                     wide_kv: bool = False) -> ModelCache:
        return build_cache(self, use_attn=use_attn, functional=functional, wide_kv=wide_kv)

    def forward(self, input_ids: torch.Tensor, cache: Optional[ModelCache] = None,
                labels: Optional[torch.Tensor] = None, mask: Optional[torch.Tensor] = None,
                position: Optional[Union[int, torch.Tensor]] = None,
                cu_seqlens: Optional[torch.Tensor] = None, logits: bool = True) -> ModelOutput:
        '''Run the model over [B, T] ids.

        `cu_seqlens` (new): packed sequences, B == 1 -- every sequence starts from
        empty state.  `logits=False` skips the vocabulary projection.'''
        cached = cache.seq_len if cache is not None else 0
        if mask is not None:
            width = cached + input_ids.shape[1]
            if mask.dim() != 2:
                raise ValueError(f'mask must be [B, T], got {tuple(mask.shape)}')
            if mask.shape != (input_ids.shape[0], width):
                raise ValueError(f'mask {tuple(mask.shape)} does not cover the {width} keys of a '
                                 f'{cached}-position cache plus {input_ids.shape[1]} inputs')
            mask = mask[:, None, None, :]
        x = self.embed(input_ids)
        if cache is None:
            cache = self.create_cache(use_attn=False if cu_seqlens is not None else None)
        for i, block in enumerate(self.blocks):
            out = block(x, cache[i], mask, 0 if position is None else position, cu_seqlens=cu_seqlens)
            x = out.hidden_states
        x = self.norm(x)
        out_logits = self.lm_head(x) if (logits or labels is not None) else None
        loss = None
        if labels is not None:
            loss = F.cross_entropy(out_logits.view(-1, out_logits.size(-1)), labels.view(-1), ignore_index=-100)
        return ModelOutput(hidden_states=x, logits=out_logits, loss=loss, cache=cache)
