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


def _rows_of(t, what):
    t2, lead = _rows2d(t)
    if t2 is None or t2.dtype != torch.bfloat16 or not t2.is_cuda:
        raise ValueError(f'{what}: bf16 ROCm rows with unit feature stride required, got {tuple(t.shape)}')
    return t2, lead


def linear_rows_pair(x1, w1, x2, w2, epilogue1='none'):
    '''(linear_rows(x1, w1, epilogue1), linear_rows(x2, w2, 'swiglu')) in one launch: the
    decoder's attention input projection and its MLP gate/up projection.  Equal to the
    two separate calls bit for bit.  K of both a multiple of 64, at most MAX_ROWS rows.'''
    code = EPILOGUES[epilogue1]
    if wants_grad(x1, w1, x2, w2):
        return _torch_form(x1, w1, code, None, None), _torch_form(x2, w2, 3, None, None)
    a, lead1 = _rows_of(x1, 'linear_rows_pair')
    b, lead2 = _rows_of(x2, 'linear_rows_pair')
    M, K = a.shape
    if b.shape[0] != M:
        raise ValueError('linear_rows_pair: both inputs need the same rows')
    N1, N2 = w1.shape[0], w2.shape[0]
    y1 = torch.empty(*lead1, N1 // 2 if code == 3 else N1, dtype=x1.dtype, device=x1.device)
    y2 = torch.empty(*lead2, N2 // 2, dtype=x2.dtype, device=x2.device)
    y1d, y2d = y1.view(M, -1), y2.view(M, -1)
    rc = _lib.lib().motif_linear_rows_pair(
        a.data_ptr(), a.stride(0), w1.data_ptr(), w1.stride(0), y1d.data_ptr(), y1d.stride(0), N1, K, code,
        b.data_ptr(), b.stride(0), w2.data_ptr(), w2.stride(0), y2d.data_ptr(), y2d.stride(0), N2, b.shape[1],
        M, _lib.stream_ptr(x1.device))
    _lib.check(rc, 'motif_linear_rows_pair')
    return y1, y2


def linear_rows_dual(x1, w1, x2, w2, gate=None, aux2=None):
    '''The decoder's output side in one launch: u = x1 W1^T (times sigmoid(gate) when
    given: Chord's gated o_proj), f = u + x2 W2^T (the MLP's down projection), and
    p = aux2 + f when aux2 is given (the block's running sum).  Returns (f, p or None);
    equal bit for bit to linear_rows(x1, w1, 'gate' / 'none') followed by
    linear_rows(x2, w2, 'resid', aux=u, aux2=aux2).'''
    if wants_grad(x1, w1, x2, w2, gate, aux2):
        u = F.linear(x1, w1)
        if gate is not None:
            u = u * torch.sigmoid(gate)
        f = u + F.linear(x2, w2)
        return f, (None if aux2 is None else aux2 + f)
    a, lead = _rows_of(x1, 'linear_rows_dual')
    b, _ = _rows_of(x2, 'linear_rows_dual')
    M, N = a.shape[0], w1.shape[0]
    if b.shape[0] != M or w2.shape[0] != N:
        raise ValueError('linear_rows_dual: the two products must have the same rows and columns')
    g = _rows_of(gate, 'linear_rows_dual')[0] if gate is not None else None
    p = _rows_of(aux2, 'linear_rows_dual')[0] if aux2 is not None else None
    for t in (g, p):
        if t is not None and tuple(t.shape) != (M, N):
            raise ValueError(f'linear_rows_dual: gate / aux2 must be [..., {N}]')
    f = torch.empty(*lead, N, dtype=x1.dtype, device=x1.device)
    y2 = torch.empty_like(f) if p is not None else None
    fd = f.view(M, N)
    y2d = None if y2 is None else y2.view(M, N)
    rc = _lib.lib().motif_linear_rows_dual(
        a.data_ptr(), a.stride(0), w1.data_ptr(), w1.stride(0), a.shape[1],
        b.data_ptr(), b.stride(0), w2.data_ptr(), w2.stride(0), b.shape[1],
        _lib.ptr(g), 0 if g is None else g.stride(0), _lib.ptr(p), 0 if p is None else p.stride(0),
        fd.data_ptr(), fd.stride(0), _lib.ptr(y2d), 0 if y2d is None else y2d.stride(0), M, N,
        _lib.stream_ptr(x1.device))
    _lib.check(rc, 'motif_linear_rows_dual')
    return f, y2


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


def sum_weights(owner, name, linears):
    '''Column-concatenated weight [N, K1 + K2 + ...] of several bias-free nn.Linear of
    one output width: x W^T over inputs laid side by side, [x1 | x2 | ...], is the sum
    of their projections in one GEMM (accumulated in fp32 and rounded once).  Cached
    like cat_weights; None under autograd or when a Linear has a bias.'''
    params = [m.weight for m in linears]
    if any(m.bias is not None for m in linears) or (
            torch.is_grad_enabled() and any(p.requires_grad for p in params)):
        return None
    key = tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in params)
    cached = owner.__dict__.get(name)
    if cached is None or cached[0] != key:
        with torch.no_grad():
            cached = (key, torch.cat(params, dim=1))
        owner.__dict__[name] = cached
    return cached[1]
