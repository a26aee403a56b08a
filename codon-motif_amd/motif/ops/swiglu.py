'''SwiGLU activation module (adjacent to the hot path).

values * SiLU(gate) over the two halves of the split dimension, as the
reference's motif/ops/swiglu.py:184-253.  On ROCm tensors (last dimension, no
autograd) it is one HIP pass (`motif_swiglu`); otherwise the torch formula.
'''
import torch
import torch.nn as nn
import torch.nn.functional as F


class SwiGLU(nn.Module):
    def __init__(self, dim: int = -1, use_triton: bool = True):
        super().__init__()
        self.dim = dim
        self.use_triton = False

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.dim in (-1, x.dim() - 1) and x.shape[-1] % 2 == 0:
            from .epilogue import swiglu, usable
            if usable(x):
                return swiglu(x)
        out, gate = torch.split(x, x.size(self.dim) // 2, dim=self.dim)
        return out * F.silu(gate)
