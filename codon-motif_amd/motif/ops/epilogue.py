'''Prefill-size elementwise stages on HIP kernels (csrc/epilogue.hip), each one pass
over HBM, rounding to the activation dtype where the reference's separate ops round:

- `gated_rms_norm_heads`: GatedRMSNorm of the GDN layer output per head, from o and
  the gate directly (the reference concatenates [o || gate] first;
  motif/block/attention/gdn_attn.py:206-209, motif/ops/rms_norm.py:530-553).
- `swiglu`: out * SiLU(gate) of the fused gate/up projection (motif/ops/swiglu.py:252-253).
- `add_fold`: f = a + b and p' = p + f, the decoder's f_h and the block's running sum
  (motif/block/decoder.py:208-213).
- `residual_fold`: the same with the Chord output gate on a and the running sum's
  put-off adds folded in: f = a * sigmoid(g) + b, p = ((c_0 + c_1) + ..) + f.

`usable(*tensors)` says whether the kernels serve a call (ROCm, bf16/fp32, 16-byte
aligned rows, no autograd); callers keep the torch formula otherwise.  Each wrapper
also computes its torch formula itself when any input or weight needs a gradient
(the kernels are forward-only), so no caller can drop a gradient by accident.
'''
import ctypes

import torch
import torch.nn.functional as F

from . import _lib
from .autograd_path import wants_grad


def usable(*ts):
    t0 = ts[0]
    if not t0.is_cuda or t0.dtype not in (torch.bfloat16, torch.float32):
        return False
    if torch.is_grad_enabled() and any(t.requires_grad for t in ts):
        return False
    vec = 16 // t0.element_size()
    for t in ts:
        if t.dtype != t0.dtype or t.stride(-1) != 1 or t.data_ptr() % 16:
            return False
        if any(s % vec for s in t.stride()[:-1]) or t.shape[-1] % vec:
            return False
    return True


def gated_rms_norm_heads(o, gate, weight, eps):
    '''y [B, L, H*dv] = GatedRMSNorm over the head rows o[b, h, t, :] with the gate
    gate[b, t, h*dv:(h+1)*dv] (o: [B, H, L, dv] any strides with unit feature stride;
    gate: [B, L, H*dv]).'''
    B, H, L, dv = o.shape
    dt = o.dtype
    if wants_grad(o, gate, weight):
        of = o.float()
        y = (of * torch.rsqrt(of.pow(2).mean(-1, keepdim=True) + eps)).to(dt) * weight.to(dt)
        return (y.transpose(1, 2) * F.silu(gate.reshape(B, L, H, dv))).reshape(B, L, H * dv)
    w = weight.detach().to(dt).contiguous()
    y = torch.empty(B, L, H * dv, dtype=dt, device=o.device)
    if y.numel() == 0:
        return y
    rc = _lib.lib().motif_gated_rms_norm(
        o.data_ptr(), o.stride(0), o.stride(1), o.stride(2), gate.data_ptr(), gate.stride(0), gate.stride(1),
        w.data_ptr(), float(eps), y.data_ptr(), y.stride(0), y.stride(1), B, L, H, dv,
        _lib.dtype_code(dt), _lib.stream_ptr(o.device))
    _lib.check(rc, 'motif_gated_rms_norm')
    return y


def swiglu(x, out=None):
    '''x [..., 2I] -> x[..., :I] * SiLU(x[..., I:]); written into `out` (a [B, L, I]
    view of x's dtype with unit feature stride and 16-byte aligned rows, e.g. the right
    columns of a wider buffer) when given.'''
    if wants_grad(x):
        if out is not None:
            raise ValueError('swiglu: out= is forward-only')
        val, gate = x.chunk(2, dim=-1)
        return val * F.silu(gate)
    x2 = x.reshape(-1, x.shape[-1])
    M, I = x2.shape[0], x.shape[-1] // 2
    if out is None:
        y = torch.empty(*x.shape[:-1], I, dtype=x.dtype, device=x.device)
        y_rs = I
    else:
        if (out.dim() != 3 or tuple(out.shape) != (*x.shape[:-1], I) or out.dtype != x.dtype
                or out.stride(-1) != 1 or out.stride(0) != out.shape[1] * out.stride(1) or not usable(out)):
            raise ValueError(f'swiglu: out must be a {x.dtype} [..., {I}] view of rows with one stride')
        y, y_rs = out, out.stride(1)
    if M == 0:
        return y
    rc = _lib.lib().motif_swiglu(x2.data_ptr(), x2.stride(0), y.data_ptr(), y_rs, M, I, _lib.dtype_code(x.dtype),
                                 _lib.stream_ptr(x.device))
    _lib.check(rc, 'motif_swiglu')
    return y


def add_fold(a, b, p=None):
    '''(f, p') with f = a + b and p' = p + f (p' is None when p is None); a, b, p of one
    shape [..., N].'''
    if wants_grad(a, b, p):
        f = a + b
        return f, (None if p is None else p + f)
    N = a.shape[-1]
    a2, b2 = a.reshape(-1, N), b.reshape(-1, N)
    f = torch.empty_like(a, memory_format=torch.contiguous_format)
    f2 = f.view(-1, N)
    p2 = po = po2 = None
    if p is not None:
        p2 = p.reshape(-1, N)
        po = torch.empty_like(f)
        po2 = po.view(-1, N)
    if f.numel() == 0:
        return f, po
    rc = _lib.lib().motif_add_fold(a2.data_ptr(), a2.stride(0), b2.data_ptr(), b2.stride(0), _lib.ptr(p2),
                                   0 if p2 is None else p2.stride(0), f2.data_ptr(), N, _lib.ptr(po2),
                                   0 if po2 is None else N, a2.shape[0], N, _lib.dtype_code(a.dtype),
                                   _lib.stream_ptr(a.device))
    _lib.check(rc, 'motif_add_fold')
    return f, po


MAX_CHAIN = 8


def _fold_torch(a, g, b, chain):
    '''residual_fold as torch ops: each op rounds to the dtype as the reference's do.'''
    f = None
    if a is not None:
        f = (a if g is None else a * torch.sigmoid(g)) + b
    if not chain:
        return f, None
    p = chain[0]
    for c in list(chain[1:]) + ([f] if f is not None else []):
        p = p + c
    return f, p


def _row_view(t):
    '''[M, N] view of t's rows (unit feature stride), or None when there is none.'''
    if t.stride(-1) != 1:
        return None
    try:
        return t.view(-1, t.shape[-1])
    except RuntimeError:
        return None


def residual_fold(a, b, gate=None, chain=()):
    '''(f, p) with f = a * sigmoid(gate) + b (a + b without a gate) and
    p = ((chain[0] + chain[1]) + ..) + f, one add and one rounding each in that order
    (None without a chain); with a and b None, p sums the chain only.  Every operand
    [..., N] of one shape and dtype (row views allowed); at most MAX_CHAIN addends.
    Calls the kernel does not serve (autograd, other dtypes, unaligned rows) take the
    same ops in torch.'''
    chain = list(chain)
    ops = [t for t in (a, gate, b) if t is not None] + chain
    if not ops:
        raise ValueError('residual_fold: nothing to sum')
    if a is None and (gate is not None or b is not None or len(chain) < 2):
        raise ValueError('residual_fold: a and b together, or a chain of two or more addends')
    if (a is None) != (b is None):
        raise ValueError('residual_fold: a and b together')
    shape = ops[0].shape
    N = shape[-1]
    rows = [_row_view(t) for t in ops]
    if (len(chain) > MAX_CHAIN or wants_grad(*ops) or any(t.shape != shape for t in ops)
            or any(r is None for r in rows) or not usable(*rows)):
        return _fold_torch(a, gate, b, chain)
    M = rows[0].shape[0]
    dev, dt = ops[0].device, ops[0].dtype
    it = iter(rows)
    a2 = next(it) if a is not None else None
    g2 = next(it) if gate is not None else None
    b2 = next(it) if b is not None else None
    c2 = list(it)
    f = torch.empty(shape, dtype=dt, device=dev) if a is not None else None
    p = torch.empty(shape, dtype=dt, device=dev) if chain else None
    if M == 0:
        return f, p
    n = len(c2)
    ptrs = (ctypes.c_void_p * max(n, 1))(*[t.data_ptr() for t in c2])
    rs = (ctypes.c_int64 * max(n, 1))(*[t.stride(0) for t in c2])
    rc = _lib.lib().motif_residual_fold(
        _lib.ptr(a2), 0 if a2 is None else a2.stride(0), _lib.ptr(g2), 0 if g2 is None else g2.stride(0),
        _lib.ptr(b2), 0 if b2 is None else b2.stride(0), ptrs, rs, n,
        _lib.ptr(f), N, _lib.ptr(p), N, M, N, _lib.dtype_code(dt), _lib.stream_ptr(dev))
    _lib.check(rc, 'motif_residual_fold')
    return f, p


def gdn_gates(a, b, a_log, dt_bias):
    '''(beta, g) [B, H, L] from the a / b projections [B, L, H] (column views allowed):
    beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias) -- one kernel instead of
    the reference's six elementwise ops (motif/block/attention/gdn_attn.py:193-195).'''
    B, L, H = a.shape
    dt = a.dtype
    if wants_grad(a, b, a_log, dt_bias):
        g = -a_log.exp() * F.softplus(a + dt_bias)
        return torch.sigmoid(b).transpose(1, 2), g.transpose(1, 2)
    al = a_log.detach().to(dt).contiguous()
    db = dt_bias.detach().to(dt).contiguous()
    beta = torch.empty(B, H, L, dtype=dt, device=a.device)
    g = torch.empty(B, H, L, dtype=dt, device=a.device)
    if beta.numel() == 0:
        return beta, g
    rc = _lib.lib().motif_gdn_gates(a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(), b.stride(0), b.stride(1),
                                    al.data_ptr(), db.data_ptr(), beta.data_ptr(), g.data_ptr(),
                                    beta.stride(0), beta.stride(1), beta.stride(2), B, L, H,
                                    _lib.dtype_code(dt), _lib.stream_ptr(a.device))
    _lib.check(rc, 'motif_gdn_gates')
    return beta, g


def mul_sigmoid(x, g):
    '''x * sigmoid(g) (both [..., N], row-major views).'''
    if wants_grad(x, g):
        return x * torch.sigmoid(g)
    N = x.shape[-1]
    x2, g2 = x.reshape(-1, N), g.reshape(-1, N)
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if y.numel() == 0:
        return y
    rc = _lib.lib().motif_mul_sigmoid(x2.data_ptr(), x2.stride(0), g2.data_ptr(), g2.stride(0), y.data_ptr(), N,
                                      x2.shape[0], N, _lib.dtype_code(x.dtype), _lib.stream_ptr(x.device))
    _lib.check(rc, 'motif_mul_sigmoid')
    return y
