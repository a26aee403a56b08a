'''Intra-block attention-residual read (adjacent to the hot path).

Softmax over the block's sources of <query, RMSNorm(source)>, then the weighted
sum of the raw sources: the reference's fused read (motif/ops/attn_res.py:22-55,
:94-186) and eager read (:588-593), and `apply_block_attn_res` (:596-622).  On
CUDA tensors it runs as one HIP kernel (`motif_attn_res_read`, fp32 arithmetic,
every source read once).  The torch formula serves CPU tensors, calls that need
gradients (the kernel is forward-only) and reads of more than MAX_SRC sources (with
one warning, as the reference's reader warns when it leaves its kernel,
motif/ops/attn_res.py:570-586).
'''
import ctypes
import warnings

import torch

from . import _lib
from .autograd_path import wants_grad

MAX_SRC = 8
_warned_many = False


def attn_res_torch(sources, query, norm):
    '''The read in torch ops (differentiable): scores <query, norm(x_n)> in the sources'
    dtype, softmax over the sources, weighted sum of the raw sources.'''
    V = torch.stack(list(sources), dim=0)                      # [N, B, T, D]
    K = norm(V)
    logits = torch.matmul(K, query.to(K.dtype))                # [N, B, T]
    alpha = logits.softmax(dim=0)
    w = alpha.permute(1, 2, 0).unsqueeze(-2)                   # [B, T, 1, N]
    return torch.matmul(w, V.permute(1, 2, 0, 3).contiguous()).squeeze(-2)


def _torch_route(sources, query, norm, *more) -> bool:
    '''The read takes the torch formula: CPU tensors, gradients, too many sources.'''
    global _warned_many
    if not sources[0].is_cuda or wants_grad(sources, query, norm, *more):
        return True
    if len(sources) > MAX_SRC:
        if not _warned_many:
            _warned_many = True
            warnings.warn(f'attention-residual read of {len(sources)} sources: the HIP kernel takes at most '
                          f'{MAX_SRC}; computing it with torch ops', RuntimeWarning)
        return True
    return False


def attn_res_read(sources, query, norm):
    '''h = sum_n softmax_n(<query, norm(x_n)>) x_n over sources x_n [B, T, D].'''
    sources = list(sources)
    x0 = sources[0]
    if _torch_route(sources, query, norm):
        return attn_res_torch(sources, query, norm)
    if not _lib.available():
        raise RuntimeError('attn_res_read: the HIP kernel library is not loaded')
    B, T, D = x0.shape
    dt = x0.dtype
    if dt not in (torch.bfloat16, torch.float32):
        raise NotImplementedError(f'attn_res_read: dtype {dt}')
    srcs = [s if s.stride(-1) == 1 else s.contiguous() for s in sources]
    for s in srcs:
        if s.shape != x0.shape or s.dtype != dt:
            raise ValueError('attn_res_read: sources must share shape and dtype')
    weight = norm.weight
    if weight is None:
        weight = torch.ones(D, dtype=dt, device=x0.device)
    q = query.to(dt).contiguous()
    w = weight.to(dt).contiguous()
    out = torch.empty(B, T, D, dtype=dt, device=x0.device)
    n = len(srcs)
    ptrs = (ctypes.c_void_p * n)(*[s.data_ptr() for s in srcs])
    sb = (ctypes.c_int64 * n)(*[s.stride(0) for s in srcs])
    st = (ctypes.c_int64 * n)(*[s.stride(1) for s in srcs])
    rc = _lib.lib().motif_attn_res_read(ptrs, sb, st, n, q.data_ptr(), w.data_ptr(), float(norm.eps),
                                        out.data_ptr(), out.stride(0), out.stride(1), B, T, D,
                                        _lib.dtype_code(dt), _lib.stream_ptr(x0.device))
    _lib.check(rc, 'attn_res_read')
    return out


def attn_res_read_norms(sources, query, norm, norm_a, norm_b):
    '''(norm_a(h), norm_b(h)) for h = attn_res_read(sources, query, norm), in one HIP
    kernel that never writes h: the decoder's attn_norm / mlp_norm inputs.  RMSNorm
    as the reference computes it on the stored h: T(h * rsqrt(mean(h^2) + eps)) * w.
    Needs ROCm tensors, both norms with weights and one eps; reads the torch route
    would serve (see attn_res_read) are computed as attn_res_read then the two norms.'''
    sources = list(sources)
    x0 = sources[0]
    if _torch_route(sources, query, norm, norm_a, norm_b):
        h = attn_res_read(sources, query, norm) if len(sources) > 1 else sources[0]
        return norm_a(h), norm_b(h)
    B, T, D = x0.shape
    dt = x0.dtype
    if dt not in (torch.bfloat16, torch.float32):
        raise NotImplementedError(f'attn_res_read_norms: dtype {dt}')
    if norm_a.weight is None or norm_b.weight is None or norm_a.eps != norm_b.eps:
        raise NotImplementedError('attn_res_read_norms: needs weighted norms with one eps')
    srcs = [s if s.stride(-1) == 1 else s.contiguous() for s in sources]
    for s in srcs:
        if s.shape != x0.shape or s.dtype != dt:
            raise ValueError('attn_res_read_norms: sources must share shape and dtype')
    dev = x0.device
    weight = norm.weight if norm.weight is not None else torch.ones(D, dtype=dt, device=dev)
    q = query.to(dt).contiguous()
    w = weight.to(dt).contiguous()
    wa, wb = norm_a.weight.to(dt).contiguous(), norm_b.weight.to(dt).contiguous()
    ya = torch.empty(B, T, D, dtype=dt, device=dev)
    yb = torch.empty(B, T, D, dtype=dt, device=dev)
    n = len(srcs)
    ptrs = (ctypes.c_void_p * n)(*[s.data_ptr() for s in srcs])
    sb = (ctypes.c_int64 * n)(*[s.stride(0) for s in srcs])
    st = (ctypes.c_int64 * n)(*[s.stride(1) for s in srcs])
    nw = (ctypes.c_void_p * 2)(wa.data_ptr(), wb.data_ptr())
    no = (ctypes.c_void_p * 2)(ya.data_ptr(), yb.data_ptr())
    nsb = (ctypes.c_int64 * 2)(ya.stride(0), yb.stride(0))
    nst = (ctypes.c_int64 * 2)(ya.stride(1), yb.stride(1))
    rc = _lib.lib().motif_attn_res_read_norms(ptrs, sb, st, n, q.data_ptr(), w.data_ptr(), float(norm.eps),
                                              None, 0, 0, 2, nw, no, nsb, nst, float(norm_a.eps),
                                              B, T, D, _lib.dtype_code(dt), _lib.stream_ptr(dev))
    _lib.check(rc, 'attn_res_read_norms')
    return ya, yb


def apply_block_attn_res(cache, query, norm):
    sources = cache.aligned_values()
    if len(sources) == 1:
        return sources[0]
    return attn_res_read(sources, query, norm)
