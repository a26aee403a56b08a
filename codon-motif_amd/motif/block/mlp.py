'''Decoder MLP: down_proj(values * SiLU(gate)) with the fused gate/up projection
(reference motif/block/mlp.py:7-63); the gated width is ceil(8 D / 3) rounded
up to a multiple of 128.'''
import torch.nn as nn

from motif.ops import SwiGLU as SwiGLUOp


class SwiGLU(nn.Module):
    def __init__(self, in_features: int, hidden_features: int = None, out_features: int = None, bias: bool = False):
        super().__init__()
        if hidden_features is None:
            h = int(in_features * 8 / 3)
            hidden_features = (h + 127) // 128 * 128
        out_features = out_features or in_features
        self.hidden_features = hidden_features
        self.gate_up_proj = nn.Linear(in_features, 2 * hidden_features, bias=bias)
        self.down_proj = nn.Linear(hidden_features, out_features, bias=bias)
        self.act = SwiGLUOp(dim=-1)

    def forward(self, x):
        return self.down_proj(self.act(self.gate_up_proj(x)))
