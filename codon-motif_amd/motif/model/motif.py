'''MotifChordModel: the integration harness for the full-model configurations.

Same module tree and parameter names as the reference (motif/model/motif.py:154-630:
embed, blocks, norm, tied lm_head) and the same forward contract
(input_ids, cache, labels, mask, position) -> ModelOutput, and the checkpoint
entry points `from_pretrained` / `save_pretrained` (motif/model/motif.py:237-380
over motif/model/checkpoint.py).  Generation and sampling are outside this build.
'''
import dataclasses
import os
from dataclasses import dataclass
from typing import Dict, Optional, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from motif.block.decoder import DecoderBlock
from motif.model.cache import ModelCache, build_cache
from motif.model.config import MotifChordConfig
from motif.ops import RMSNorm
from motif.ops.packed import PackedSeqs


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

    @classmethod
    def from_pretrained(cls, path: str, config: Optional[Union[MotifChordConfig, Dict, str]] = None,
                        map_location: Union[str, torch.device] = 'cpu',
                        device: Optional[Union[str, torch.device]] = None, strict: bool = False,
                        verbose: bool = True, **overrides) -> 'MotifChordModel':
        '''Build the model a checkpoint describes and load its weights (eval mode).

        The config comes from `config` (a MotifChordConfig, a mapping or a JSON file
        path), else from the file, else from the tensor shapes
        (`config_from_state_dict`); `**overrides` replace fields of the result.  A
        tied model whose file lacks `lm_head.weight` takes it from `embed.weight`.
        `strict` fails on missing / unexpected keys instead of reporting them.
        '''
        from motif.model.checkpoint import _as_config, config_from_state_dict, load_checkpoint
        loaded = load_checkpoint(path, map_location=map_location)
        sd = dict(loaded.state_dict)
        if isinstance(config, str):
            with open(config, 'r', encoding='utf-8') as fh:
                import json
                config = json.load(fh)
        cfg = _as_config(config) if config is not None else None
        if config is not None and cfg is None:
            raise TypeError(f'config must be a MotifChordConfig, a mapping or a JSON path, got {type(config).__name__}')
        cfg = cfg or loaded.config or config_from_state_dict(sd)
        if overrides:
            known = {f.name for f in dataclasses.fields(MotifChordConfig)}
            unknown = sorted(set(overrides) - known)
            if unknown:
                raise TypeError(f'unknown MotifChordConfig override(s): {unknown}')
            cfg = dataclasses.replace(cfg, **overrides)
        model = cls(cfg)
        if cfg.tied_weight and 'lm_head.weight' not in sd and 'embed.weight' in sd:
            sd['lm_head.weight'] = sd['embed.weight']
        try:
            report = model.load_state_dict(sd, strict=False)
        except RuntimeError as exc:
            raise RuntimeError(f'{os.fspath(path)!r} does not match the model built from {cfg!r}: {exc}') from exc
        if strict and (report.missing_keys or report.unexpected_keys):
            raise RuntimeError(f'{os.fspath(path)!r}: missing {report.missing_keys}, '
                               f'unexpected {report.unexpected_keys}')
        if verbose:
            print(f'[motif] {loaded.source} {os.fspath(path)}: {len(sd)} tensors, '
                  f'{len(report.missing_keys)} missing, {len(report.unexpected_keys)} unexpected')
        if device is not None:
            model = model.to(device)
        return model.eval()

    def save_pretrained(self, path: str, metadata: Optional[Dict] = None) -> Dict:
        '''Write the weights and config to one `.safetensors` file.'''
        from motif.model.checkpoint import save_safetensors
        return save_safetensors(self, path, self.config, metadata)

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
        empty state; an int tensor (its host-side metadata is then built once, one read
        back from the device) or a motif.ops.packed.PackedSeqs built beforehand (the
        forward then reads nothing back and can be captured in a graph).  `logits=False`
        skips the vocabulary projection.'''
        cached = cache.seq_len if cache is not None else 0
        if cu_seqlens is not None:
            cu_seqlens = PackedSeqs.of(cu_seqlens, input_ids.shape[1], input_ids.device)
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
