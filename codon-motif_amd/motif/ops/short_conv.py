'''Short causal depthwise conv + SiLU on the HIP kernel.

Replaces the body of the reference's `GatedDeltaAttention._conv`
(motif/block/attention/gdn_attn.py:116-136): xc = [cache || x] on the time
axis, y = SiLU(depthwise_conv1d(xc)), new cache = the last K-1 pre-activation
inputs of xc.  Inputs stay in the [B, L, D] layout the projections produce (no
transposes); the cache keeps the reference layout [B, D, K-1].
'''
import torch

from . import _lib


def short_conv_silu(x, weight, cache=None, y=None, new_cache=None):
    '''Causal depthwise conv + SiLU.

    Args:
        x: [B, L, D] (fp32 or bf16, feature axis unit-stride).
        weight: nn.Conv1d weight [D, 1, K] (any float dtype; cast to x's).
        cache: [B, D, K-1] tail of the previous chunk, or None (zeros).
        y: optional preallocated [B, L, D] output.
        new_cache: optional preallocated [B, D, K-1] tail output; may be `cache`
            itself (in-place update).

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
    rc = _lib.lib().motif_short_conv_silu(
        x.data_ptr(), x.stride(0), x.stride(1), w.data_ptr(), _lib.ptr(cache), new_cache.data_ptr(),
        y.data_ptr(), y.stride(0), y.stride(1), B, L, D, K, None, B, L,
        _lib.dtype_code(x.dtype), _lib.stream_ptr(x.device))
    _lib.check(rc, 'motif_short_conv_silu')
    return y, new_cache


def short_conv_silu_varlen(x, weight, cu_seqlens, max_seqlen=None):
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
    rc = _lib.lib().motif_short_conv_silu(
        x.data_ptr(), x.stride(0), x.stride(1), w.data_ptr(), None, tails.data_ptr(),
        y.data_ptr(), y.stride(0), y.stride(1), B, L, D, K, cu_dev.data_ptr(), nseq, int(max_seqlen),
        _lib.dtype_code(x.dtype), _lib.stream_ptr(x.device))
    _lib.check(rc, 'motif_short_conv_silu')
    return y, tails
