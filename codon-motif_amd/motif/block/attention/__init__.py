from motif.block.attention.base import AttentionOutput, BasicAttention
from motif.block.attention.chord_attn import ChordAttention
from motif.block.attention.gdn_attn import GatedDeltaAttention

__all__ = ['AttentionOutput', 'BasicAttention', 'ChordAttention', 'GatedDeltaAttention']
