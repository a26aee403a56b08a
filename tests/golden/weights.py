'''Deterministic parameter values keyed by parameter name.

Used by make_layer_fixtures.py (on the reference modules) and by the parity
tests (on this build's modules): both module trees use the same parameter
names, so filling them with this function gives identical weights without
storing them in the fixtures.
'''
import math

import torch


def fill_params(module: torch.nn.Module, seed: int, std: float = 0.05) -> None:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in sorted(module.named_parameters()):
            shape = p.shape
            if name.endswith('A_log'):
                val = torch.empty(shape).uniform_(1, 16, generator=g).log()
            elif name.endswith('dt_bias'):
                dt = torch.exp(torch.rand(shape, generator=g) * (math.log(0.1) - math.log(0.001)) + math.log(0.001))
                val = dt + torch.log(-torch.expm1(-dt))
            elif name.endswith('theta_alpha') or name.endswith('theta_beta'):
                val = 0.3 * torch.randn(shape, generator=g)
            elif name.endswith('theta_mu'):
                val = torch.zeros(shape)
            elif name.endswith('ssmax_s'):
                val = 1.0 + 0.2 * torch.randn(shape, generator=g)
            elif 'pseudo_queries' in name:
                val = 0.3 * torch.randn(shape, generator=g)
            elif '_conv.weight' in name:
                val = 0.3 * torch.randn(shape, generator=g)
            elif 'norm' in name and name.endswith('weight'):
                val = 1.0 + 0.1 * torch.randn(shape, generator=g)
            else:
                val = std * torch.randn(shape, generator=g)
            p.copy_(val.to(p.dtype))
