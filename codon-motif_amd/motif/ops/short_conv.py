'''Short causal depthwise conv + SiLU on the HIP kernel.

Replaces the body of the reference's `GatedDeltaAttention._conv`
(motif/block/attention/gdn_attn.py:116-136): xc = [cache || x] on the time
axis, y = SiLU(depthwise_conv1d(xc)), new cache = the last K-1 pre-activation
inputs of xc.  Inputs stay in the [B, L, D] layout the projections produce (no
transposes); the cache keeps the reference layout [B, D, K-1].
'''
import ctypes

import torch

from . import _lib
from .packed import PackedSeqs
from .autograd_path import short_conv_silu_torch, wants_grad


def _conv_call(x, w, cache, new_cache, y, cu, nseq, max_len, head_dim, scale):
    B, L, D = x.shape
    K = w.shape[-1]
    L_ = _lib.lib()
    args = (x.data_ptr(), x.stride(0), x.stride(1), w.data_ptr(), _lib.ptr(cache), _lib.ptr(new_cache),
            y.data_ptr(), y.stride(0), y.stride(1), B, L, D, K, _lib.ptr(cu), nseq, max_len)
    if head_dim:
        rc = L_.motif_short_conv_silu_l2norm(*args, int(head_dim), float(scale), _lib.dtype_code(x.dtype),
                                             _lib.stream_ptr(x.device))
    else:
        rc = L_.motif_short_conv_silu(*args, _lib.dtype_code(x.dtype), _lib.stream_ptr(x.device))
    _lib.check(rc, 'motif_short_conv_silu')


def short_conv_silu(x, weight, cache=None, y=None, new_cache=None, head_dim=None, scale=1.0):
    '''Causal depthwise conv + SiLU.

    Args:
        x: [B, L, D] (fp32 or bf16, feature axis unit-stride).
        weight: nn.Conv1d weight [D, 1, K] (any float dtype; cast to x's).
        cache: [B, D, K-1] tail of the previous chunk, or None (zeros).
        y: optional preallocated [B, L, D] output.
        new_cache: optional preallocated [B, D, K-1] tail output; may be `cache`
            itself (in-place update).
        head_dim: if set (16, 32 or 64), every head_dim channels of each timestep
            are then L2-normalised (F.normalize, eps 1e-12) and multiplied by
            `scale` -- the GDN q / k front end (gdn_attn.py:190-191).

    Returns:
        (y [B, L, D], new_cache [B, D, K-1])
    '''
    if wants_grad(x, weight, cache):
        # forward-only kernel: training takes the differentiable torch form
        y_, tail = short_conv_silu_torch(x, weight, cache, head_dim, scale)
        if new_cache is not None:
            new_cache.copy_(tail.detach())
            tail = new_cache
        return y_, tail
    if not x.is_cuda:
        raise ValueError('short_conv_silu: x must live on the ROCm device')
    B, L, D = x.shape
    K = weight.shape[-1]
    if weight.numel() != D * K:
        raise ValueError(f'short_conv_silu: weight must hold [D, 1, K] = [{D}, 1, {K}]')
    if x.stride(-1) != 1:
        x = x.contiguous()
    w = weight.detach().reshape(D, K).to(x.dtype).contiguous()
    if cache is not None:
        if cache.shape != (B, D, K - 1):
            raise ValueError(f'short_conv_silu: cache must be [B, D, K-1] = {(B, D, K - 1)}')
        if cache.dtype != x.dtype or not cache.is_contiguous():
            cache = cache.to(x.dtype).contiguous()
    if y is None:
        y = torch.empty(B, L, D, dtype=x.dtype, device=x.device)
    if new_cache is None:
        new_cache = torch.empty(B, D, K - 1, dtype=x.dtype, device=x.device)
    _conv_call(x, w, cache, new_cache, y, None, B, L, head_dim, scale)
    return y, new_cache


def short_conv_silu_varlen(x, weight, cu_seqlens, max_seqlen=None, head_dim=None, scale=1.0):
    '''Packed-sequence conv (B == 1): every sequence starts from a zero tail.

    Returns:
        (y [1, T, D], tails [nseq, D, K-1])
    '''
    if wants_grad(x, weight):
        # per sequence in the differentiable torch form (training)
        cu = PackedSeqs.of(cu_seqlens, x.shape[1]).cu_host.tolist()
        parts = [short_conv_silu_torch(x[:, cu[i]:cu[i + 1]], weight, None, head_dim, scale)
                 for i in range(len(cu) - 1)]
        return torch.cat([p[0] for p in parts], 1), torch.cat([p[1] for p in parts], 0)
    if not x.is_cuda:
        raise ValueError('short_conv_silu_varlen: x must live on the ROCm device')
    B, L, D = x.shape
    if B != 1:
        raise ValueError('short_conv_silu_varlen: packed sequences need B == 1')
    K = weight.shape[-1]
    if x.stride(-1) != 1:
        x = x.contiguous()
    w = weight.detach().reshape(D, K).to(x.dtype).contiguous()
    ps = PackedSeqs.of(cu_seqlens, L, x.device)
    nseq = ps.nseq
    if max_seqlen is None:
        max_seqlen = ps.max_len
    cu_dev = ps.cu
    y = torch.empty(B, L, D, dtype=x.dtype, device=x.device)
    tails = torch.empty(nseq, D, K - 1, dtype=x.dtype, device=x.device)
    _conv_call(x, w, None, tails, y, cu_dev, nseq, int(max_seqlen), head_dim, scale)
    return y, tails


def short_conv_silu_multi(xs, weights, caches, head_dims, scales, cu_seqlens=None, max_seqlen=None):
    '''Several conv + SiLU problems over the same tokens in one launch (the GDN q, k, v
    front ends; no reference counterpart).  Problem i is
    `short_conv_silu(xs[i], weights[i], caches[i], head_dim=head_dims[i], scale=scales[i])`
    (or the `_varlen` form when `cu_seqlens` is given).

    Returns the list of (y, new_cache) pairs, or None when the single-launch kernel does
    not serve these inputs (the caller then makes the separate calls).
    '''
    n = len(xs)
    x0 = xs[0]
    if wants_grad(xs, weights, caches):
        return None
    if not 1 <= n <= 3 or not x0.is_cuda or x0.dtype not in (torch.bfloat16, torch.float32):
        return None
    B, L = x0.shape[0], x0.shape[1]
    K = weights[0].shape[-1]
    if L < 1 or any(x.shape[:2] != (B, L) or x.dtype != x0.dtype or x.stride(-1) != 1 for x in xs):
        return None
    if any(w.shape[-1] != K or w.numel() != x.shape[-1] * K for w, x in zip(weights, xs)):
        return None
    dev, dt = x0.device, x0.dtype
    ws = [w.detach().reshape(x.shape[-1], K).to(dt).contiguous() for w, x in zip(weights, xs)]
    if cu_seqlens is None:
        nseq, max_len, cu_dev = B, L, None
        cs = []
        for c, x in zip(caches, xs):
            if c is not None and (c.shape != (B, x.shape[-1], K - 1) or c.dtype != dt or not c.is_contiguous()):
                return None
            cs.append(c)
    else:
        if B != 1:
            return None
        ps = PackedSeqs.of(cu_seqlens, L, dev)
        nseq = ps.nseq
        if nseq < 1:
            return None
        max_len = int(max_seqlen) if max_seqlen is not None else ps.max_len
        if max_len < 1:
            return None
        cu_dev = ps.cu
        cs = [None] * n
    ys = [torch.empty(B, L, x.shape[-1], dtype=dt, device=dev) for x in xs]
    tails = [torch.empty(nseq, x.shape[-1], K - 1, dtype=dt, device=dev) for x in xs]
    arr = lambda ct, vals: (ct * n)(*vals)
    rc = _lib.lib().motif_short_conv_silu_multi(
        n, arr(ctypes.c_void_p, [x.data_ptr() for x in xs]),
        arr(ctypes.c_int64, [x.stride(0) for x in xs]), arr(ctypes.c_int64, [x.stride(1) for x in xs]),
        arr(ctypes.c_void_p, [w.data_ptr() for w in ws]), arr(ctypes.c_void_p, [_lib.ptr(c) for c in cs]),
        arr(ctypes.c_void_p, [t.data_ptr() for t in tails]), arr(ctypes.c_void_p, [y.data_ptr() for y in ys]),
        arr(ctypes.c_int64, [y.stride(0) for y in ys]), arr(ctypes.c_int64, [y.stride(1) for y in ys]),
        arr(ctypes.c_int, [x.shape[-1] for x in xs]), arr(ctypes.c_int, [int(h or 0) for h in head_dims]),
        arr(ctypes.c_float, [float(sc) for sc in scales]),
        B, L, K, _lib.ptr(cu_dev), nseq, max_len, _lib.dtype_code(dt), _lib.stream_ptr(dev))
    if rc == _lib.ERR_UNSUPPORTED:
        return None
    _lib.check(rc, 'motif_short_conv_silu_multi')
    return list(zip(ys, tails))

