'''Decoder MLP: down_proj(values * SiLU(gate)) with the fused gate/up projection
(reference motif/block/mlp.py:7-63); the gated width is ceil(8 D / 3) rounded
up to a multiple of 128.'''
import torch.nn as nn

from motif.ops import SwiGLU as SwiGLUOp
from motif.ops.epilogue import add_fold, usable
from motif.ops.linear_rows import linear_rows, rows_eligible


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

    def _fused(self, x):
        '''Decode-sized bf16 input: SwiGLU fused into the gate/up projection kernel.'''
        return (self.gate_up_proj.bias is None and self.down_proj.bias is None
                and rows_eligible(x, self.gate_up_proj.weight) and x.shape[-1] == self.gate_up_proj.in_features)

    def forward(self, x):
        if self._fused(x):
            return linear_rows(linear_rows(x, self.gate_up_proj.weight, 'swiglu'), self.down_proj.weight)
        return self.down_proj(self.act(self.gate_up_proj(x)))

    def forward_residual(self, x, residual, partial=None):
        '''(f, p) with f = residual + forward(x) and p = partial + f (None when `partial`
        is None, or when the adds took the torch fallback: the caller then folds f
        itself).  Decode-sized inputs run both adds in the down projection's epilogue,
        larger ones in one elementwise kernel.'''
        if (self._fused(x) and residual.dtype == x.dtype and residual.shape[:-1] == x.shape[:-1]
                and residual.stride(-1) == 1
                and (partial is None or (partial.shape == residual.shape and partial.dtype == x.dtype
                                         and partial.stride(-1) == 1))):
            h = linear_rows(x, self.gate_up_proj.weight, 'swiglu')
            if partial is None:
                return linear_rows(h, self.down_proj.weight, 'resid', aux=residual), None
            return linear_rows(h, self.down_proj.weight, 'resid', aux=residual, aux2=partial)
        out = self.forward(x)
        if residual.shape == out.shape and usable(residual, out) and (
                partial is None or (partial.shape == out.shape and usable(partial))):
            return add_fold(residual, out, partial)
        return residual + out, None
