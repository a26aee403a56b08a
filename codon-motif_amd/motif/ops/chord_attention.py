'''Chord attention (GGD-biased causal softmax) on the gfx950 HIP kernels.

`apply_chord_attention` keeps the reference signature, defaults, validation
messages and exception types (motif/ops/chord_attention.py:1557-1625 with
`_check_tensors` :966-1011 and `_check_params` :1448-1472).  The launcher
picks the bf16 MFMA flash kernel for prefill shapes and the split-K vector
kernel when a kv head serves at most 8 query rows (GQA group x L), which is
the reference's long-KV / short-Q split path (:1128-1229).  fp32 inputs run on
the vector kernel for every shape (fp32 FMA throughout, the accuracy mode).
`apply_chord_attention_varlen` adds packed sequences (new) and
`chord_decode_cursor` the decode step over a fixed-capacity cache whose length
lives on the device (new; the graph-replayable form of the decode call).
Calls that need gradients run `ChordFunction` (bf16, head dim 64, padded batch): the
forward kernel with its log-sum-exp, then the backward kernels (motif_chord_bwd: dq, dk,
dv and the four per-head parameter gradients, the reference's custom backward
:1348-1554).  Other gradient calls take the differentiable torch forms
(motif/ops/autograd_path.py).
'''
from typing import Optional

import torch

from . import _lib
from .packed import PackedSeqs
from .autograd_path import chord_attention_torch, chord_attention_varlen_torch, wants_grad

HEAD_DIM = 64                  # the model's head dim: bf16 runs on the MFMA kernels
HEAD_DIMS = (16, 32, 64, 128)  # head dims the kernels serve (fp32 / fp16 / other D: the vector kernel)


def serves_head_dim(D: int) -> bool:
    '''Head dims apply_chord_attention takes: the kernels' own (HEAD_DIMS) and every
    size between them (zero-padded to the next one).'''
    return HEAD_DIMS[0] <= D <= HEAD_DIMS[-1]


def _grad_kernels_serve(q, k, v, alpha, beta, mu, ssmax, log_n, q_start):
    '''The backward kernels take bf16 q / k / v with head dim 64 on a GPU, fp32 [H]
    parameters and no gradient into log_n (as the reference's backward).'''
    if not (q.is_cuda and q.dtype == torch.bfloat16 and k.dtype == q.dtype and v.dtype == q.dtype
            and q.dim() == 4 and q.shape[-1] == HEAD_DIM and k.shape == v.shape and k.shape[-1] == HEAD_DIM
            and _lib.available()):
        return False
    if log_n.requires_grad or any(t.dtype != torch.float32 or t.dim() != 1 for t in (alpha, beta, mu, ssmax)):
        return False
    S, L = k.shape[2], q.shape[2]
    qs = S - L if q_start is None else int(q_start)
    return 0 <= qs and qs + L <= S and log_n.dtype == torch.float32 and log_n.shape == (q.shape[0], L)


class ChordFunction(torch.autograd.Function):
    '''Chord attention with the HIP forward (which also writes the base-2 log-sum-exp)
    and the HIP backward (motif_chord_bwd), the reference's `_TritonChordFunction`
    (motif/ops/chord_attention.py:1475-1554): gradients for q, k, v, alpha, beta, mu and
    ssmax; none for log_n.'''

    @staticmethod
    def forward(ctx, q, k, v, alpha, beta, mu, ssmax, log_n, q_start, scale, eps):
        B, H, L, D = q.shape
        q, k, v = _aligned(q.contiguous()), _aligned(k.contiguous()), _aligned(v.contiguous())
        params = [t.detach().contiguous() for t in (alpha, beta, mu, ssmax)]
        ln = log_n.detach().contiguous()
        out = torch.empty((B, H, L, D), dtype=q.dtype, device=q.device)
        lse = torch.empty((B, H, L), dtype=torch.float32, device=q.device)
        if L > 0:
            _launch(q, k, v, *params, ln, q_start, scale, eps, out, lse)
        ctx.save_for_backward(q, k, v, out, lse, *params, ln)
        ctx.q_start, ctx.scale, ctx.eps = q_start, scale, eps
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse, alpha, beta, mu, ssmax, ln = ctx.saved_tensors
        B, H, L, D = q.shape
        Hkv, S = k.shape[1], k.shape[2]
        dout = _aligned(dout.contiguous())
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        lib = _lib.lib()
        d_params = torch.empty((4, H), dtype=torch.float32, device=q.device)
        nbytes = int(lib.motif_chord_bwd_workspace_bytes(B, H, Hkv, L, S, int(ctx.q_start)))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        rc = lib.motif_chord_bwd(
            *_lib.t4(q), *_lib.t4(k), *_lib.t4(v), *_lib.t4(out), *_lib.t4(dout),
            lse.data_ptr(), alpha.data_ptr(), beta.data_ptr(), mu.data_ptr(), ssmax.data_ptr(),
            ln.data_ptr(), ln.stride(0), ln.stride(1),
            *_lib.t4(dq), *_lib.t4(dk), *_lib.t4(dv), d_params.data_ptr(),
            B, H, Hkv, L, S, D, int(ctx.q_start), float(ctx.scale), float(ctx.eps),
            ws.data_ptr(), ws.numel(), _lib.chord_dtype_code(q.dtype), _lib.stream_ptr(q.device))
        _lib.check(rc, 'motif_chord_bwd')
        needs = ctx.needs_input_grad
        grads = [dq, dk, dv] + list(d_params.unbind(0))
        grads = [g if needs[i] else None for i, g in enumerate(grads)]
        return (*grads, None, None, None, None)


def _check_tensors(q, k, v, log_n):
    for name, t in (('q', q), ('k', k), ('v', v)):
        if not t.is_cuda:
            raise ValueError(f'{name} must live on CUDA')
        if t.dim() != 4:
            raise ValueError(f'{name} must be 4-D [B, H, L, D], got {tuple(t.shape)}')
        if t.stride(-1) != 1:
            raise ValueError(f'{name} must be contiguous along the last dimension (stride(-1) == 1)')
        if t.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError(f'{name} has unsupported dtype {t.dtype} (only fp16 / bf16 / fp32)')
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError('q / k / v must all have the same dtype')
    if k.shape != v.shape:
        raise ValueError(f'k / v must have the same shape, got {tuple(k.shape)} vs {tuple(v.shape)}')
    B, H, L, D = q.shape
    Bk, Hkv, S, Dk = k.shape
    if B != Bk or D != Dk:
        raise ValueError(f'q {tuple(q.shape)} and k {tuple(k.shape)} disagree on B / D')
    if H % Hkv != 0:
        raise ValueError(f'num_heads {H} must be divisible by num_kv_heads {Hkv}')
    if D < 16:
        raise ValueError(f'head_dim {D} is too small (>= 16 required)')
    if log_n.shape != (B, L):
        raise ValueError(f'log_n must be [B, q_len] = {(B, L)}, got {tuple(log_n.shape)}')
    if log_n.dtype != torch.float32:
        raise ValueError(f'log_n must be fp32, got {log_n.dtype}')
    if log_n.stride(-1) != 1:
        raise ValueError('log_n must be contiguous along the last dimension')
    return B, H, L, D, Hkv, S


def _check_params(alpha, beta, mu, ssmax, num_heads):
    for name, t in (('alpha', alpha), ('beta', beta), ('mu', mu), ('ssmax', ssmax)):
        if not t.is_cuda:
            raise ValueError(f'{name} must live on CUDA')
        if t.dtype != torch.float32:
            raise ValueError(f'{name} must be fp32, got {t.dtype}')
        if t.shape != (num_heads,):
            raise ValueError(f'{name} must be [{num_heads}], got {tuple(t.shape)}')
        if not t.is_contiguous():
            raise ValueError(f'{name} must be contiguous')


def _aligned(t):
    '''Rows must start on 16-byte boundaries for the vector loads.'''
    per16 = 16 // t.element_size()
    ok = t.data_ptr() % 16 == 0 and all(s % per16 == 0 for s in t.stride()[:-1])
    return t if ok else t.contiguous()


def _check_out(out, shape, dtype, device):
    '''A caller's destination: the output's shape, dtype and device, unit feature stride,
    rows on 16-byte boundaries (the kernels' vector stores).'''
    if tuple(out.shape) != tuple(shape) or out.dtype != dtype or out.device != device:
        raise ValueError(f'out must be {tuple(shape)} {dtype} on {device}, got {tuple(out.shape)} {out.dtype} '
                         f'on {out.device}')
    per16 = 16 // out.element_size()
    if out.stride(-1) != 1 or out.data_ptr() % 16 or any(s % per16 for s in out.stride()[:-1]):
        raise ValueError('out must have unit feature stride and 16-byte aligned rows')
    return out


def _out_for(out, q):
    '''The kernel's destination: the caller's `out` (checked) or a new [B, H, L, D].'''
    if out is None:
        return torch.empty(q.shape, dtype=q.dtype, device=q.device)
    return _check_out(out, q.shape, q.dtype, q.device)


def _launch(q, k, v, alpha, beta, mu, ssmax, log_n, q_start, scale, eps, out, lse=None,
            cu_dev=None, nseq=None, max_seqlen=None, cu_host=None):
    B, H, L, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    if D not in HEAD_DIMS:
        # a head dim between the kernels' sizes: q, k, v zero-padded to the next one (the
        # extra features add nothing to q.k and give zero output columns), output cut back
        Dp = next((d for d in HEAD_DIMS if d > D), None)
        if Dp is None or lse is not None:
            raise NotImplementedError(f'apply_chord_attention: head_dim {D} unsupported (16 to 128)')
        pad = lambda t: torch.nn.functional.pad(t, (0, Dp - D))
        out_p = torch.empty((B, H, L, Dp), dtype=out.dtype, device=out.device)
        _launch(pad(q), pad(k), pad(v), alpha, beta, mu, ssmax, log_n, q_start, scale, eps, out_p,
                cu_dev=cu_dev, nseq=nseq, max_seqlen=max_seqlen, cu_host=cu_host)
        out.copy_(out_p[..., :D])
        return out
    if cu_dev is not None and (q.dtype != torch.bfloat16 or D != HEAD_DIM):
        # the packed kernel serves bf16 at head dim 64; other packed inputs run sequence
        # by sequence (each one causal from position 0) on the same kernels
        cu = [int(x) for x in cu_host]
        for a, b in zip(cu[:-1], cu[1:]):
            if b > a:
                _launch(q[:, :, a:b], k[:, :, a:b], v[:, :, a:b], alpha, beta, mu, ssmax, log_n[:, a:b], 0,
                        scale, eps, out[:, :, a:b])
        return out
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    lib = _lib.lib()
    if cu_dev is None:
        nseq, max_seqlen = B, L
    nbytes = lib.motif_chord_workspace_bytes(B, H, Hkv, L, S, D, None)
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=q.device)
    rc = lib.motif_chord_fwd(
        *_lib.t4(q), *_lib.t4(k), *_lib.t4(v),
        alpha.data_ptr(), beta.data_ptr(), mu.data_ptr(), ssmax.data_ptr(),
        log_n.data_ptr(), log_n.stride(0), log_n.stride(1),
        *_lib.t4(out), _lib.ptr(lse),
        B, H, Hkv, L, S, D, int(q_start), float(scale), float(eps),
        _lib.ptr(cu_dev), int(nseq), int(max_seqlen),
        ws.data_ptr(), ws.numel(), _lib.chord_dtype_code(q.dtype), _lib.stream_ptr(q.device))
    _lib.check(rc, 'motif_chord_fwd')
    return out


def apply_chord_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    alpha: torch.Tensor,
    beta: torch.Tensor,
    mu: torch.Tensor,
    ssmax: torch.Tensor,
    log_n: torch.Tensor,
    q_start: Optional[int] = None,
    softmax_scale: Optional[float] = None,
    eps: float = 1e-5,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    '''Chord attention forward on the HIP kernels.

    logits = (softmax_scale * q.k + bias) * ssmax_h * log_n[b, i] with the GGD
    bias -alpha_h (|j - (q_start + i) - mu_h| + eps) ** beta_h, causal over
    keys j <= q_start + i, softmax over keys, times v.

    Args:
        q: [B, H, L, D];  k, v: [B, H_kv, S, D] (fp16, bf16 or fp32; 16 <= D <= 128).
        alpha, beta, mu, ssmax: [H] fp32 contiguous.
        log_n: [B, L] fp32.
        q_start: absolute position of the first query; defaults to S - L.
        softmax_scale: defaults to D ** -0.5.
        eps: GGD epsilon.
        out: optional [B, H, L, D] destination in q's dtype with unit feature stride (a
            strided view, e.g. the transpose of a [B, L, H, D] buffer, so the heads come
            out already merged); not a reference argument.

    Returns:
        [B, H, L, D] in q's dtype (`out` when given).

    Raises:
        ValueError: on unsupported inputs or a negative q_start.
        NotImplementedError: for a head dim above 128 (inputs requiring grad take the
            differentiable torch form).
        RuntimeError: when the HIP library is unavailable or a launch fails.
    '''
    if wants_grad(q, k, v, alpha, beta, mu, ssmax, log_n):
        if q_start is not None and int(q_start) < 0:
            raise ValueError(f'q_start must not be negative, got {q_start}')
        if _grad_kernels_serve(q, k, v, alpha, beta, mu, ssmax, log_n, q_start):
            scale = q.shape[-1] ** -0.5 if softmax_scale is None else float(softmax_scale)
            qs = k.shape[2] - q.shape[2] if q_start is None else int(q_start)
            res = ChordFunction.apply(q, k, v, alpha, beta, mu, ssmax, log_n, qs, scale, float(eps))
        else:
            res = chord_attention_torch(q, k, v, alpha, beta, mu, ssmax, log_n, q_start, softmax_scale, eps)
        return res if out is None else _check_out(out, res.shape, res.dtype, res.device).copy_(res)
    if not _lib.available():
        raise RuntimeError('there is no usable HIP backend in the current environment')
    B, H, L, D, Hkv, S = _check_tensors(q, k, v, log_n)
    _check_params(alpha, beta, mu, ssmax, H)
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    if q_start is None:
        q_start = S - L
    q_start = int(q_start)
    if q_start < 0:
        raise ValueError(f'q_start must not be negative, got {q_start}')
    out = _out_for(out, q)
    if L == 0:
        return out
    return _launch(q, k, v, alpha, beta, mu, ssmax, log_n, q_start, softmax_scale, eps, out)


def apply_chord_attention_varlen(q, k, v, alpha, beta, mu, ssmax, log_n, cu_seqlens,
                                 softmax_scale=None, eps=1e-5, out=None):
    '''Packed-sequence Chord attention (no reference counterpart).

    B == 1; q [1, H, T, D], k/v [1, H_kv, T, D] hold the sequences back to back,
    sequence i covering rows [cu_seqlens[i], cu_seqlens[i+1]).  Each sequence is
    causal on its own with positions restarting at 0; log_n [1, T] is read at
    the packed row (log(1 .. len_i) per sequence reproduces separate runs).
    `cu_seqlens` is an int tensor or a motif.ops.packed.PackedSeqs (whose host-side
    metadata then spares the call every read back from the device).
    Calls that need gradients run the sequences separately: through the HIP forward /
    backward pair (`ChordFunction`) where it serves, else as differentiable torch runs.
    `out` is an optional destination, as for apply_chord_attention.
    '''
    if wants_grad(q, k, v, alpha, beta, mu, ssmax, log_n):
        if (q.shape[0] == 1 and q.shape[2] > 0 and k.shape[2] == q.shape[2]
                and _grad_kernels_serve(q, k, v, alpha, beta, mu, ssmax, log_n, 0)):
            cu = PackedSeqs.of(cu_seqlens, q.shape[2], q.device).cu_host.tolist()
            outs = [apply_chord_attention(q[:, :, a:b], k[:, :, a:b], v[:, :, a:b], alpha, beta, mu, ssmax,
                                          log_n[:, a:b], q_start=0, softmax_scale=softmax_scale, eps=eps)
                    for a, b in zip(cu[:-1], cu[1:]) if b > a]
            res = torch.cat(outs, dim=2)
        else:
            cu_t = cu_seqlens.cu_host if isinstance(cu_seqlens, PackedSeqs) else cu_seqlens
            res = chord_attention_varlen_torch(q, k, v, alpha, beta, mu, ssmax, log_n, cu_t, softmax_scale, eps)
        return res if out is None else _check_out(out, res.shape, res.dtype, res.device).copy_(res)
    if not _lib.available():
        raise RuntimeError('there is no usable HIP backend in the current environment')
    B, H, L, D, Hkv, S = _check_tensors(q, k, v, log_n)
    _check_params(alpha, beta, mu, ssmax, H)
    if B != 1 or S != L:
        raise ValueError('apply_chord_attention_varlen: needs B == 1 and packed q / k of equal length')
    ps = PackedSeqs.of(cu_seqlens, L, q.device)
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    out = _out_for(out, q)
    if L == 0:
        return out
    return _launch(q, k, v, alpha, beta, mu, ssmax, log_n, 0, softmax_scale, eps, out,
                   cu_dev=ps.cu, nseq=ps.nseq, max_seqlen=ps.max_len, cu_host=ps.cu_host)


def chord_decode_workspace(B, H, Hkv, L, capacity, D, dtype, device) -> torch.Tensor:
    '''A workspace for chord_decode_cursor at these sizes.'''
    n = _lib.lib().motif_chord_decode_workspace_bytes(B, H, Hkv, L, capacity, D, _lib.chord_dtype_code(dtype), None)
    return torch.empty(max(int(n), 1), dtype=torch.uint8, device=device)


def chord_decode_step_serves(proj, H, Hkv, D) -> bool:
    '''Whether chord_decode_step serves a decode of these projection rows: bf16, head
    dim 64, at most 16 query rows per kv head, 16-byte aligned rows.'''
    return (proj.is_cuda and proj.dtype == torch.bfloat16 and proj.dim() == 3 and proj.stride(-1) == 1
            and D == HEAD_DIM and H % Hkv == 0 and (H // Hkv) * proj.shape[1] <= 16
            and proj.data_ptr() % 16 == 0 and proj.stride(0) % 8 == 0 and proj.stride(1) % 8 == 0
            and _lib.available())


def chord_decode_step_workspace(B, H, Hkv, L, capacity, device) -> torch.Tensor:
    '''A zeroed workspace for chord_decode_step at these sizes (its arrival counters must
    start at zero; every call leaves them zero).'''
    n = int(_lib.lib().motif_chord_decode_step_workspace_bytes(B, H, Hkv, L, capacity))
    return torch.zeros(max(n, 1), dtype=torch.uint8, device=device)


def chord_decode_step(proj, offsets, q_norm_weight, k_norm_weight, norm_eps, k_cache, v_cache, length_dev, alpha,
                      beta, mu, ssmax, log_table, num_heads, softmax_scale, eps, workspace):
    '''A Chord decode step at the device cursor in one launch (new; the reference's
    motif/block/attention/chord_attn.py:255-265 q / k norms and v, the cache append
    motif/model/cache.py:170-215 and the decode call of apply_chord_attention): from the
    projection rows proj [B, L, ncols] (q, k, v at column `offsets`), appends the
    normalised keys and the values at length_dev, attends over length_dev + L keys with
    q_start = length_dev and log_n = log_table[q_start + i], advances length_dev by L.
    Returns out [B, H, L, 64], the same bits as chord_qkv_prep followed by
    chord_decode_cursor.'''
    B, L = proj.shape[0], proj.shape[1]
    Hkv, cap, D = k_cache.shape[1], k_cache.shape[2], k_cache.shape[3]
    out = torch.empty(B, num_heads, L, D, dtype=proj.dtype, device=proj.device)
    rc = _lib.lib().motif_chord_decode_step(
        proj.data_ptr(), proj.stride(0), proj.stride(1), *[int(o) for o in offsets],
        q_norm_weight.data_ptr(), k_norm_weight.data_ptr(), float(norm_eps),
        *_lib.t4(k_cache), *_lib.t4(v_cache), length_dev.data_ptr(), cap,
        alpha.data_ptr(), beta.data_ptr(), mu.data_ptr(), ssmax.data_ptr(), log_table.data_ptr(), log_table.numel(),
        *_lib.t4(out), B, num_heads, Hkv, L, D, float(softmax_scale), float(eps),
        workspace.data_ptr(), workspace.numel(), _lib.stream_ptr(proj.device))
    _lib.check(rc, 'motif_chord_decode_step')
    return out


def chord_decode_cursor(q, k_cache, v_cache, length_dev, alpha, beta, mu, ssmax, log_table, softmax_scale=None,
                        eps=1e-5, log_n=None, workspace=None, library_scratch=False):
    '''Chord attention of L new queries over a fixed-capacity cache (new).

    k_cache / v_cache [B, Hkv, capacity, D] hold `length_dev[0]` cached positions and
    the L new keys / values right after them.  Attends over length_dev + L keys with
    q_start = length_dev (the cached length), log_n[b, i] = log_table[q_start + i]
    unless `log_n` [B, L] is given, then advances length_dev by L -- on the device, so
    a captured launch replays token after token.  Returns [B, H, L, D].
    `library_scratch=True` takes the allocation-free entry point
    (motif_chord_decode_noalloc: the library's own per-device scratch, no workspace).
    '''
    B, H, L, D = q.shape
    Hkv, cap = k_cache.shape[1], k_cache.shape[2]
    if length_dev.dtype != torch.int32 or length_dev.device != q.device:
        raise ValueError('chord_decode_cursor: length_dev must be a device int32 tensor')
    if log_table.dtype != torch.float32 or log_table.numel() < cap:
        raise ValueError('chord_decode_cursor: log_table must be fp32 with at least `capacity` entries')
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    q = _aligned(q)
    out = torch.empty((B, H, L, D), dtype=q.dtype, device=q.device)
    ln_sb, ln_st = (log_n.stride(0), log_n.stride(1)) if log_n is not None else (0, 0)
    if library_scratch:
        rc = _lib.lib().motif_chord_decode_noalloc(
            *_lib.t4(q), *_lib.t4(k_cache), *_lib.t4(v_cache), length_dev.data_ptr(), cap,
            alpha.data_ptr(), beta.data_ptr(), mu.data_ptr(), ssmax.data_ptr(),
            _lib.ptr(log_n), ln_sb, ln_st, log_table.data_ptr(), log_table.numel(),
            *_lib.t4(out), B, H, Hkv, L, D, float(softmax_scale), float(eps),
            _lib.chord_dtype_code(q.dtype), _lib.stream_ptr(q.device))
        _lib.check(rc, 'motif_chord_decode_noalloc')
        return out
    if workspace is None:
        workspace = chord_decode_workspace(B, H, Hkv, L, cap, D, q.dtype, q.device)
    rc = _lib.lib().motif_chord_decode(
        *_lib.t4(q), *_lib.t4(k_cache), *_lib.t4(v_cache), length_dev.data_ptr(), cap,
        alpha.data_ptr(), beta.data_ptr(), mu.data_ptr(), ssmax.data_ptr(),
        _lib.ptr(log_n), ln_sb, ln_st, log_table.data_ptr(), log_table.numel(),
        *_lib.t4(out), B, H, Hkv, L, D, float(softmax_scale), float(eps),
        workspace.data_ptr(), workspace.numel(), _lib.chord_dtype_code(q.dtype), _lib.stream_ptr(q.device))
    _lib.check(rc, 'motif_chord_decode')
    return out
