'''SwiGLU activation module (adjacent to the hot path; PyTorch-ROCm).

values * SiLU(gate) over the two halves of the split dimension, as the
reference's motif/ops/swiglu.py:184-253.
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
        out, gate = torch.split(x, x.size(self.dim) // 2, dim=self.dim)
        return out * F.silu(gate)
