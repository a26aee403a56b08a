'''Decode-sized projections on the HIP kernel `motif_linear_rows`: y = x W^T for
at most a few dozen activation rows (bf16, fp32 accumulation), with the
elementwise op that follows the projection fused into its epilogue.  Prefill-sized
inputs keep the library GEMM (`F.linear`), which is compute-bound there.

Epilogues (each intermediate rounded to bf16 where the reference's separate ops
round):
  'none'    y = x W^T
  'gate'    y = (x W^T) * sigmoid(aux)           ChordAttention: o_proj(out) * G
  'resid'   y = (x W^T) + aux; y2 = aux2 + y     decoder: f_h = attn + mlp, block sum
  'swiglu'  y = (x W_a^T) * SiLU(x W_b^T)        SwiGLU MLP, W = [W_a; W_b] (gate_up_proj)
'''
import torch
import torch.nn.functional as F

from . import _lib
from .autograd_path import wants_grad

EPILOGUES = {'none': 0, 'gate': 1, 'resid': 2, 'swiglu': 3}

# Row counts up to this take the HIP kernel.
MAX_ROWS = 64

def _rows2d(t):
    '''[..., K] -> ([M, K] view with unit feature stride, leading shape) or None.'''
    lead = t.shape[:-1]
    if t.stride(-1) != 1:
        return None, lead
    try:
        return t.view(-1, t.shape[-1]), lead
    except RuntimeError:
        return None, lead


def rows_eligible(x, weight, bias=None):
    '''True when `linear_rows` serves this call: a bf16 ROCm input of at most
    MAX_ROWS rows, no bias, no autograd, and 16-byte aligned rows.'''
    if bias is not None or not x.is_cuda or x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        return False
    if wants_grad(x, weight):
        return False
    K = x.shape[-1]
    if K % 32 or weight.dim() != 2 or weight.shape[1] != K or weight.stride(1) != 1 or weight.stride(0) % 8:
        return False
    M = x.numel() // K if K else 0
    if M == 0 or M > MAX_ROWS:
        return False
    x2, _ = _rows2d(x)
    if x2 is None or x2.stride(0) % 8 or x2.data_ptr() % 16 or weight.data_ptr() % 16:
        return False
    return True


def linear_rows(x, weight, epilogue='none', aux=None, aux2=None, out=None, out2=None):
    '''Fused decode projection (see the module docstring).

    Args:
        x: [..., K] bf16 rows.  weight: [N, K] bf16 (nn.Linear layout).
        aux: [..., Nout] for 'gate' (pre-sigmoid gate) and 'resid' (residual).
        aux2: [..., Nout] running sum for 'resid' (optional); out2 receives aux2 + y.

    Returns:
        y [..., Nout] (and y2 for 'resid' with aux2).
    '''
    code = EPILOGUES[epilogue]
    if wants_grad(x, weight, aux, aux2):
        return _torch_form(x, weight, code, aux, aux2)
    x2, lead = _rows2d(x)
    if x2 is None:
        x2 = x.reshape(-1, x.shape[-1]).contiguous()
    M, K = x2.shape
    N = weight.shape[0]
    nout = N // 2 if code == 3 else N
    dev = x.device
    y = out if out is not None else torch.empty(*lead, nout, dtype=x.dtype, device=dev)
    y2d = y.view(-1, nout)

    def flat(t):
        if t is None:
            return None
        t2, _ = _rows2d(t)
        if t2 is None or t2.shape != (M, nout):
            raise ValueError(f'linear_rows: epilogue operand must be [..., {nout}] row-major, got {tuple(t.shape)}')
        if t2.dtype != torch.bfloat16:
            raise ValueError('linear_rows: epilogue operands must be bf16')
        return t2

    a1, a2 = flat(aux), flat(aux2)
    y2 = None
    if code == 2 and a2 is not None:
        y2 = out2 if out2 is not None else torch.empty(*lead, nout, dtype=x.dtype, device=dev)
    y22 = None if y2 is None else y2.view(-1, nout)
    rc = _lib.lib().motif_linear_rows(
        x2.data_ptr(), x2.stride(0), weight.data_ptr(), weight.stride(0), y2d.data_ptr(), y2d.stride(0),
        M, N, K, code,
        _lib.ptr(a1), 0 if a1 is None else a1.stride(0),
        _lib.ptr(a2), 0 if a2 is None else a2.stride(0),
        _lib.ptr(y22), 0 if y22 is None else y22.stride(0),
        _lib.stream_ptr(dev))
    _lib.check(rc, 'motif_linear_rows')
    return (y, y2) if code == 2 and a2 is not None else y


def _torch_form(x, weight, code, aux, aux2):
    '''The projection and its epilogue as torch ops (differentiable).'''
    y = F.linear(x, weight)
    if code == 1:
        return y * torch.sigmoid(aux)
    if code == 2:
        y = aux + y
        return y if aux2 is None else (y, aux2 + y)
    if code == 3:
        out, gate = y.chunk(2, dim=-1)
        return out * F.silu(gate)
    return y


def project(x, weight, bias=None):
    '''F.linear, on the decode kernel when `rows_eligible`.'''
    if rows_eligible(x, weight, bias):
        return linear_rows(x, weight)
    return torch.nn.functional.linear(x, weight, bias)


def cat_weights(owner, name, linears):
    '''Row-concatenated weight (and bias) of several nn.Linear, so their projections
    of one input run as one GEMM.  Cached on `owner` under `name` and rebuilt when a
    weight is replaced or updated in place (version counters); rebuilt per call while
    autograd records, so gradients reach the original parameters.'''
    has_bias = linears[0].bias is not None
    params = [m.weight for m in linears] + ([m.bias for m in linears] if has_bias else [])
    if torch.is_grad_enabled() and any(p.requires_grad for p in params):
        w = torch.cat([m.weight for m in linears])
        return w, (torch.cat([m.bias for m in linears]) if has_bias else None)
    key = tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in params)
    cached = owner.__dict__.get(name)
    if cached is None or cached[0] != key:
        with torch.no_grad():
            w = torch.cat([m.weight for m in linears])
            b = torch.cat([m.bias for m in linears]) if has_bias else None
        cached = (key, w, b)
        owner.__dict__[name] = cached
    return cached[1], cached[2]
