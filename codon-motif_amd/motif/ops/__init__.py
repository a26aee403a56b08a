'''Public op surface, named as the reference's motif/ops/__init__.py:1-10.

`HAS_TRITON` keeps its name because the layers read it as "the fast backend
is present"; here it is True when libmotif_hip.so loaded and a ROCm device is
visible.
'''
from . import _lib
from .rms_norm import RMSNorm, GatedRMSNorm
from .swiglu import SwiGLU
from .chord_attention import apply_chord_attention, apply_chord_attention_varlen
from .gated_deltanet import (
    recurrent_gated_delta_rule,
    chunk_gated_delta_rule,
    chunk_gated_delta_rule_triton,
    chunk_gated_delta_rule_varlen,
    chunk_gated_delta_rule_gated_norm,
    gdn_prefill_fused,
)
from .short_conv import short_conv_silu, short_conv_silu_multi, short_conv_silu_varlen
from .attn_res import apply_block_attn_res, attn_res_read, attn_res_read_norms
from .gdn_decode import gdn_decode_fused
from .linear_rows import cat_weights, linear_rows, project, rows_eligible

HAS_TRITON = _lib.available()
HAS_HIP = HAS_TRITON

__all__ = [
    'RMSNorm', 'GatedRMSNorm', 'SwiGLU',
    'apply_chord_attention', 'apply_chord_attention_varlen',
    'recurrent_gated_delta_rule', 'chunk_gated_delta_rule',
    'chunk_gated_delta_rule_triton', 'chunk_gated_delta_rule_varlen', 'chunk_gated_delta_rule_gated_norm',
    'gdn_prefill_fused',
    'short_conv_silu', 'short_conv_silu_multi', 'short_conv_silu_varlen',
    'apply_block_attn_res', 'attn_res_read', 'attn_res_read_norms', 'gdn_decode_fused',
    'cat_weights', 'linear_rows', 'project', 'rows_eligible',
    'HAS_TRITON', 'HAS_HIP',
]
