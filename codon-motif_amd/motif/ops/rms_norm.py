'''RMSNorm / GatedRMSNorm modules (adjacent to the hot path; PyTorch-ROCm).

Same parameters and formulas as the reference (motif/ops/rms_norm.py:419-553):
RMSNorm y = x / sqrt(mean(x^2) + eps) * weight; GatedRMSNorm takes
[values || gate] and returns rms_norm(values) * SiLU(gate).
'''
import torch
import torch.nn as nn
import torch.nn.functional as F


def _rms(x, weight, eps):
    if x.is_cuda and weight is not None and weight.numel() == x.shape[-1]:
        return F.rms_norm(x, (x.shape[-1],), weight, eps)
    x_f = x.float()
    y = (x_f * torch.rsqrt(x_f.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)
    return y * weight if weight is not None else y


class RMSNorm(nn.Module):
    '''Root-mean-square normalisation over the last dimension.'''

    def __init__(self, dim, eps=1e-6, elementwise_affine=True, use_triton=True):
        super().__init__()
        self.dim = dim
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            self.weight = nn.Parameter(torch.ones(dim))
        else:
            self.register_parameter('weight', None)
        self.use_triton = False

    def forward(self, x):
        return _rms(x, self.weight, self.eps)


class GatedRMSNorm(nn.Module):
    '''RMSNorm of the value half of [values || gate], gated by SiLU(gate).'''

    def __init__(self, dim, eps=1e-6, elementwise_affine=True, use_triton=True):
        super().__init__()
        self.dim = dim
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            self.weight = nn.Parameter(torch.ones(dim))
        else:
            self.register_parameter('weight', None)
        self.use_triton = False

    def forward(self, x):
        x_in, gate = x.split(self.dim, dim=-1)
        x_f = x_in.float()
        y = (x_f * torch.rsqrt(x_f.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype)
        if self.weight is not None:
            y = y * self.weight
        return y * F.silu(gate)
