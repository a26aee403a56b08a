'''Short causal depthwise conv + SiLU on the HIP kernel.

Replaces the body of the reference's `GatedDeltaAttention._conv`
(motif/block/attention/gdn_attn.py:116-136): xc = [cache || x] on the time
axis, y = SiLU(depthwise_conv1d(xc)), new cache = the last K-1 pre-activation
inputs of xc.  Inputs stay in the [B, L, D] layout the projections produce (no
transposes); the cache keeps the reference layout [B, D, K-1].
'''
import torch

from . import _lib


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
    if not x.is_cuda:
        raise ValueError('short_conv_silu_varlen: x must live on the ROCm device')
    B, L, D = x.shape
    if B != 1:
        raise ValueError('short_conv_silu_varlen: packed sequences need B == 1')
    K = weight.shape[-1]
    if x.stride(-1) != 1:
        x = x.contiguous()
    w = weight.detach().reshape(D, K).to(x.dtype).contiguous()
    cu_host = cu_seqlens.detach().to('cpu', torch.int64)
    nseq = int(cu_host.numel()) - 1
    lens = cu_host[1:] - cu_host[:-1]
    if max_seqlen is None:
        max_seqlen = int(lens.max()) if nseq > 0 else 0
    cu_dev = cu_host.to(device=x.device, dtype=torch.int32)
    y = torch.empty(B, L, D, dtype=x.dtype, device=x.device)
    tails = torch.empty(nseq, D, K - 1, dtype=x.dtype, device=x.device)
    _conv_call(x, w, None, tails, y, cu_dev, nseq, int(max_seqlen), head_dim, scale)
    return y, tails
