'''Gated delta rule (GDN) ops on the gfx950 HIP kernels.

Same public functions and argument meaning as the reference's
motif/ops/gated_deltanet.py (`recurrent_gated_delta_rule` :26-59,
`chunk_gated_delta_rule` :287-321, `chunk_gated_delta_rule_triton` :796-834),
plus `chunk_gated_delta_rule_varlen` for packed sequences (new).

Differences that do not change results beyond rounding:
- the recurrent state is carried and returned in fp32 whatever the input dtype
  (inputs may be fp32 or bf16; q/k/v/beta/g of mixed dtypes are computed in fp32);
- `chunk_size` is rounded down to one of the kernel chunk lengths
  {16, 32, 64} (values >= 64 use 64); the chunk length only changes the order
  of floating-point operations, not the recurrence.
Gradients: `chunk_gated_delta_rule` runs its HIP forward inside `GDNChunkFunction`
(motif/ops/gdn_grad.py), whose backward uses the HIP fp32 scans, and the packed form
runs each sequence through it; the recurrent form and shapes the scans do not take
differentiate through the torch form of the chunked rule
(motif/ops/autograd_path.py:gdn_chunk_torch).
'''
import functools

import torch

from . import _lib
from .packed import PackedSeqs
from .autograd_path import gdn_chunk_torch, wants_grad as _needs_grad
from .gdn_grad import GDNChunkFunction, scans_serve

__all__ = [
    'gdn_prefill_fused',
    'recurrent_gated_delta_rule',
    'chunk_gated_delta_rule',
    'chunk_gated_delta_rule_triton',
    'chunk_gated_delta_rule_varlen',
]

_KERNEL_CHUNKS = (64, 32, 16)


def _kernel_chunk(chunk_size: int) -> int:
    for c in _KERNEL_CHUNKS:
        if chunk_size >= c:
            return c
    return 16


def _prepare(q, k, v, beta, g, name):
    '''Validate GDN inputs and return them in one kernel dtype.'''
    for n, t in (('q', q), ('k', k), ('v', v)):
        if t.dim() != 4:
            raise ValueError(f'{name}: {n} must be 4-D [B, H, L, D], got {tuple(t.shape)}')
    for n, t in (('beta', beta), ('g', g)):
        if t.dim() != 3:
            raise ValueError(f'{name}: {n} must be 3-D [B, H, L], got {tuple(t.shape)}')
    B, H, L, Dk = q.shape
    if k.shape != q.shape:
        raise ValueError(f'{name}: k {tuple(k.shape)} must match q {tuple(q.shape)}')
    if v.shape[:3] != (B, H, L):
        raise ValueError(f'{name}: v {tuple(v.shape)} disagrees with q on [B, H, L]')
    if beta.shape != (B, H, L) or g.shape != (B, H, L):
        raise ValueError(f'{name}: beta / g must be [B, H, L] = {(B, H, L)}')
    ts = (q, k, v, beta, g)
    if not all(t.is_cuda for t in ts):
        raise ValueError(f'{name}: inputs must live on the ROCm device (the HIP kernels have no CPU path)')
    if len({t.device for t in ts}) != 1:
        raise ValueError(f'{name}: inputs must share one device')
    # calls that need gradients never get here: the public functions route them to
    # the torch form first
    dts = {t.dtype for t in ts}
    if not dts <= {torch.float32, torch.bfloat16}:
        raise NotImplementedError(f'{name}: dtypes {sorted(map(str, dts))} unsupported (float32 / bfloat16)')
    cdt = torch.bfloat16 if dts == {torch.bfloat16} else torch.float32
    out = []
    for i, t in enumerate(ts):
        t = t.to(cdt)
        if i < 3 and t.stride(-1) != 1:  # feature axis of q / k / v must be unit-stride
            t = t.contiguous()
        out.append(t)
    return out, cdt


def _state_in(S, B, H, Dk, Dv, device, name):
    if S is None:
        return None
    if S.shape != (B, H, Dk, Dv):
        raise ValueError(f'{name}: S must be [B, H, Dk, Dv] = {(B, H, Dk, Dv)}, got {tuple(S.shape)}')
    return S.to(device=device, dtype=torch.float32).contiguous()


def recurrent_gated_delta_rule(q, k, v, beta, g, S=None):
    '''Token-by-token gated delta rule on the HIP recurrence kernel.

    Per step: S <- S * exp(g_t); S <- S + k_t (beta_t (v_t - k_t^T S))^T;
    o_t = S^T q_t (reference motif/ops/gated_deltanet.py:26-59).

    Args:
        q, k: [B, H, L, Dk];  v: [B, H, L, Dv];  beta, g: [B, H, L].
        S: optional [B, H, Dk, Dv] initial state (zeros when None).

    Returns:
        (o [B, H, L, Dv] in q's dtype, S [B, H, Dk, Dv] fp32)
    '''
    name = 'recurrent_gated_delta_rule'
    if _needs_grad(q, k, v, beta, g, S):
        return gdn_chunk_torch(q, k, v, beta, g, S)
    (qc, kc, vc, bc, gc), cdt = _prepare(q, k, v, beta, g, name)
    B, H, L, Dk = qc.shape
    Dv = vc.shape[-1]
    S_in = _state_in(S, B, H, Dk, Dv, qc.device, name)
    o = torch.empty(B, H, L, Dv, dtype=cdt, device=qc.device)
    S_out = torch.empty(B, H, Dk, Dv, dtype=torch.float32, device=qc.device)
    gdn_recurrent_into(qc, kc, vc, bc, gc, S_in, S_out, o)
    return o.to(q.dtype), S_out


def gdn_recurrent_into(q, k, v, beta, g, S_in, S_out, o):
    '''Launch the recurrence writing into preallocated `S_out` and `o`.

    `S_out` may be `S_in` (in-place state update, used by the decode step);
    no allocation happens here, so the launch can be captured in a hipGraph.
    '''
    B, H, L, Dk = q.shape
    Dv = v.shape[-1]
    code = _lib.dtype_code(q.dtype)
    rc = _lib.lib().motif_gdn_recurrent_fwd(
        *_lib.t4(q), *_lib.t4(k), *_lib.t4(v), *_lib.t4(beta), *_lib.t4(g),
        _lib.ptr(S_in), S_out.data_ptr(), *_lib.t4(o),
        B, H, L, Dk, Dv, code, _lib.dtype_code(o.dtype), _lib.stream_ptr(q.device))
    _lib.check(rc, 'motif_gdn_recurrent_fwd')


def _chunk_call(qc, kc, vc, bc, gc, S_in, C, cu=None, nseq=None, norm=None):
    '''One chunk launch.  With `norm` = (gate [B, L, H*Dv], weight [Dv], eps) the
    output is the GatedRMSNorm y [B, L, H*Dv] of the head outputs, fused into the
    output pass (o is not stored); returns None when that fusion does not apply.'''
    B, H, L, Dk = qc.shape
    Dv = vc.shape[-1]
    dev = qc.device
    if cu is None:
        nseq = B
        total = B * ((L + C - 1) // C)
        cu_dev = coff_dev = None
    else:
        ps = PackedSeqs.of(cu, L, dev)
        nseq = ps.nseq
        coff_dev, total = ps.chunk_offsets(C)
        cu_dev = ps.cu
    S_out = torch.empty(nseq, H, Dk, Dv, dtype=torch.float32, device=dev)
    nbytes = _lib.lib().motif_gdn_chunk_workspace_bytes(H, Dk, Dv, C, max(total, 1))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    code = _lib.dtype_code(qc.dtype)
    if norm is not None:
        gate, weight, eps = norm
        y = torch.empty(B, L, H * Dv, dtype=qc.dtype, device=dev)
        rc = _lib.lib().motif_gdn_chunk_fwd_gated(
            *_lib.t4(qc), *_lib.t4(kc), *_lib.t4(vc), *_lib.t4(bc), *_lib.t4(gc),
            _lib.ptr(S_in), S_out.data_ptr(), 0, 0, 0, 0,
            B, H, L, Dk, Dv, C,
            _lib.ptr(cu_dev), _lib.ptr(coff_dev), nseq, total,
            ws.data_ptr(), ws.numel(),
            gate.data_ptr(), gate.stride(0), gate.stride(1), weight.data_ptr(), float(eps),
            y.data_ptr(), y.stride(0), y.stride(1), code, _lib.stream_ptr(dev))
        if rc == _lib.ERR_UNSUPPORTED:
            return None
        _lib.check(rc, 'motif_gdn_chunk_fwd_gated')
        return y, S_out
    o = torch.empty(B, H, L, Dv, dtype=qc.dtype, device=dev)
    rc = _lib.lib().motif_gdn_chunk_fwd(
        *_lib.t4(qc), *_lib.t4(kc), *_lib.t4(vc), *_lib.t4(bc), *_lib.t4(gc),
        _lib.ptr(S_in), S_out.data_ptr(), *_lib.t4(o),
        B, H, L, Dk, Dv, C,
        _lib.ptr(cu_dev), _lib.ptr(coff_dev), nseq, total,
        ws.data_ptr(), ws.numel(), code, code, _lib.stream_ptr(dev))
    _lib.check(rc, 'motif_gdn_chunk_fwd')
    return o, S_out


def chunk_gated_delta_rule(q, k, v, beta, g, S=None, chunk_size=64):
    '''Chunked gated delta rule on the HIP chunk kernels.

    Same result as the reference's pure-torch chunk loop
    (motif/ops/gated_deltanet.py:287-321) up to rounding.

    Args:
        q, k: [B, H, L, Dk];  v: [B, H, L, Dv];  beta, g: [B, H, L].
        S: optional [B, H, Dk, Dv] initial state (zeros when None).
        chunk_size: chunk length (rounded down to 16, 32 or 64).

    Returns:
        (o [B, H, L, Dv] in q's dtype, S [B, H, Dk, Dv] fp32)
    '''
    C = _kernel_chunk(int(chunk_size))
    if _needs_grad(q, k, v, beta, g, S):
        if q.is_cuda and _lib.available() and q.dtype in (torch.float32, torch.bfloat16) \
                and scans_serve(q.shape[-1], v.shape[-1], C):
            fwd = functools.partial(_chunk_fwd, chunk=C)
            return GDNChunkFunction.apply(q, k, v, beta, g, S, C, fwd)
        return gdn_chunk_torch(q, k, v, beta, g, S, chunk_size)
    return _chunk_fwd(q, k, v, beta, g, S, C)


def _chunk_fwd(q, k, v, beta, g, S, chunk):
    name = 'chunk_gated_delta_rule'
    (qc, kc, vc, bc, gc), _ = _prepare(q, k, v, beta, g, name)
    B, H, L, Dk = qc.shape
    S_in = _state_in(S, B, H, Dk, vc.shape[-1], qc.device, name)
    o, S_out = _chunk_call(qc, kc, vc, bc, gc, S_in, chunk)
    return o.to(q.dtype), S_out


def chunk_gated_delta_rule_gated_norm(q, k, v, beta, g, gate, norm_weight, norm_eps, S=None, chunk_size=64,
                                      cu_seqlens=None):
    '''The chunk rule with the GatedDeltaAttention output norm fused into its output
    pass (no reference counterpart; replaces the chunk call plus the GatedRMSNorm of
    motif/block/attention/gdn_attn.py:198-209).

    Returns (y [B, L, H*Dv], S) where y = GatedRMSNorm(o; gate, norm_weight, norm_eps)
    per head, or None when the fused kernel does not serve these inputs (bf16 MFMA
    path only); the caller then runs the two steps separately.  `cu_seqlens` (a tensor
    or a motif.ops.packed.PackedSeqs) selects the packed-sequence form (S then
    [nseq, H, Dk, Dv]).
    '''
    name = 'chunk_gated_delta_rule_gated_norm'
    if q.dtype != torch.bfloat16 or gate.dtype != torch.bfloat16 or not q.is_cuda:
        return None
    if _needs_grad(q, k, v, beta, g, gate, norm_weight, S):
        return None
    (qc, kc, vc, bc, gc), _ = _prepare(q, k, v, beta, g, name)
    B, H, L, Dk = qc.shape
    Dv = vc.shape[-1]
    if gate.shape != (B, L, H * Dv) or gate.stride(-1) != 1:
        return None
    w = norm_weight.detach().to(torch.bfloat16).contiguous()
    if cu_seqlens is None:
        S_in = _state_in(S, B, H, Dk, Dv, qc.device, name)
        return _chunk_call(qc, kc, vc, bc, gc, S_in, _kernel_chunk(int(chunk_size)), norm=(gate, w, norm_eps))
    nseq = cu_seqlens.nseq if isinstance(cu_seqlens, PackedSeqs) else int(cu_seqlens.numel()) - 1
    if B != 1 or nseq < 1 or S is not None:
        return None
    ps = PackedSeqs.of(cu_seqlens, L, qc.device)
    return _chunk_call(qc, kc, vc, bc, gc, None, _kernel_chunk(int(chunk_size)), ps, nseq, norm=(gate, w, norm_eps))


def chunk_gated_delta_rule_triton(q, k, v, beta, g, S=None, chunk_size=64):
    '''The fast-backend entry of the reference (motif/ops/gated_deltanet.py:796-834).

    Raises NotImplementedError when the HIP backend is unavailable or
    `chunk_size < 16`, as the reference does for a missing Triton or a chunk
    below the dot-product minimum; otherwise identical to
    `chunk_gated_delta_rule`.
    '''
    if not _lib.available():
        raise NotImplementedError('the HIP backend is not available for the GatedDeltaNet chunk scan.')
    if int(chunk_size) < 16:
        raise NotImplementedError('chunk_size must be >= 16')
    return chunk_gated_delta_rule(q, k, v, beta, g, S, chunk_size)


def chunk_gated_delta_rule_varlen(q, k, v, beta, g, cu_seqlens, S=None, chunk_size=64):
    '''Packed-sequence chunked gated delta rule (no reference counterpart).

    B must be 1; sequence i covers tokens [cu_seqlens[i], cu_seqlens[i+1]) and
    runs independently from its own initial state S[i] (zeros when S is None).
    `cu_seqlens` is an int tensor or a motif.ops.packed.PackedSeqs (whose host-side
    metadata then spares the call every read back from the device).

    Returns:
        (o [1, H, L, Dv] in q's dtype, S [nseq, H, Dk, Dv] fp32)
    '''
    name = 'chunk_gated_delta_rule_varlen'
    for n, t in (('q', q), ('v', v)):
        if t.dim() != 4:
            raise ValueError(f'{name}: {n} must be 4-D [B, H, L, D], got {tuple(t.shape)}')
    B, H, L, Dk = q.shape
    Dv = v.shape[-1]
    if B != 1:
        raise ValueError(f'{name}: packed sequences need B == 1, got B={B}')
    ps = cu_seqlens if isinstance(cu_seqlens, PackedSeqs) else None
    nseq = ps.nseq if ps is not None else int(cu_seqlens.numel()) - 1
    if nseq < 1:
        raise ValueError(f'{name}: cu_seqlens needs at least two entries')
    if S is not None and S.shape != (nseq, H, Dk, Dv):
        raise ValueError(f'{name}: S must be [nseq, H, Dk, Dv] = {(nseq, H, Dk, Dv)}')
    ps = PackedSeqs.of(cu_seqlens, L, q.device)
    if _needs_grad(q, k, v, beta, g, S):
        cu = ps.cu_host.tolist()
        outs, states = [], []
        for i in range(len(cu) - 1):
            # each sequence through the chunk op's own gradient route (HIP scans where they
            # serve); an empty one passes its state through
            sl = slice(cu[i], cu[i + 1])
            if cu[i + 1] == cu[i]:
                B_, H_, _, Dk_ = q.shape
                o_i = q.new_empty(B_, H_, 0, v.shape[-1])
                S_i = (S[i:i + 1].float() if S is not None
                       else torch.zeros(1, H_, Dk_, v.shape[-1], dtype=torch.float32, device=q.device))
            else:
                o_i, S_i = chunk_gated_delta_rule(q[:, :, sl], k[:, :, sl], v[:, :, sl], beta[:, :, sl],
                                                  g[:, :, sl], None if S is None else S[i:i + 1], chunk_size)
            outs.append(o_i)
            states.append(S_i)
        return torch.cat(outs, 2), torch.cat(states, 0)
    (qc, kc, vc, bc, gc), _ = _prepare(q, k, v, beta, g, name)
    S_in = None if S is None else S.to(device=qc.device, dtype=torch.float32).contiguous()
    o, S_out = _chunk_call(qc, kc, vc, bc, gc, S_in, _kernel_chunk(int(chunk_size)), ps, nseq)
    return o.to(q.dtype), S_out


# Packed sequences (cu_seqlens) take the separate conv / gates / chunk kernels: the
# packed form of the fused front end is switched off.  A 16-sequence, 73364-token model
# prefill through it did not finish within its test's time limit and the cause is not
# established; small packed inputs (tests/test_gpu_gdn_prefill_fused.py) matched the
# separate kernels bit for bit.
PACKED_FRONT = False


def gdn_prefill_fused(proj, offsets, conv_weights, tails, a_log, dt_bias, q_scale, norm_weight, norm_eps, S=None,
                      heads=None, dk=None, dv=None, cu_seqlens=None, y=None):
    '''A GatedDeltaAttention prefill from its input projections to the o_proj input, in
    three kernels (no reference counterpart as one call; replaces
    motif/block/attention/gdn_attn.py:183-209: the q / k / v short conv + SiLU, the q / k
    L2 norm, the gates, the chunked delta rule and the GatedRMSNorm).

    proj [B, L, ncols] bf16 with columns (q, k, v, gate, a, b) at `offsets`;
    conv_weights (wq, wk, wv) nn.Conv1d weights [C, 1, 4]; tails (tq, tk, tv) incoming
    conv tails [B, C, 3] or Nones; S [B, H, dk, dv] fp32 or None; cu_seqlens (B == 1)
    for packed sequences (zero tails and states); y (optional) a [B, L, H*dv] bf16 view
    with unit feature stride to write the output into (e.g. the left columns of a wider
    buffer).  Returns (y [B, L, H*dv], S_out [B|nseq, H, dk, dv], (tq, tk, tv) outgoing
    tails), or None, before anything ran, when the fused kernels do not serve these
    inputs (the caller then runs the separate steps).
    '''
    if cu_seqlens is not None and not PACKED_FRONT:
        return None
    if proj.dtype != torch.bfloat16 or not proj.is_cuda or proj.dim() != 3 or _needs_grad(
            proj, a_log, dt_bias, norm_weight, S, *conv_weights, *[t for t in tails if t is not None]):
        return None
    if conv_weights[0].shape[-1] != 4 or proj.stride(-1) != 1:
        return None
    B, L, _ = proj.shape
    H = heads
    dev = proj.device
    C = (H * dk, H * dk, H * dv)
    ws_ = [w.detach().reshape(c, 4).to(torch.bfloat16).contiguous() for w, c in zip(conv_weights, C)]
    tin = [None if t is None else t.detach().to(torch.bfloat16).contiguous() for t in tails]
    if any(t is not None for t in tin) and (cu_seqlens is not None or not all(t is not None for t in tin)):
        return None
    if cu_seqlens is None:
        nseq, total, cu_dev, coff_dev = B, B * ((L + 63) // 64), None, None
        if S is not None and (S.shape != (B, H, dk, dv) or S.dtype != torch.float32 or not S.is_contiguous()):
            return None
    else:
        if B != 1 or S is not None:
            return None
        ps = PackedSeqs.of(cu_seqlens, L, dev)
        nseq = ps.nseq
        coff_dev, total = ps.chunk_offsets(64)
        cu_dev = ps.cu
    if L == 0 or nseq == 0:
        return None
    if y is None:
        y = torch.empty(B, L, H * dv, dtype=torch.bfloat16, device=dev)
    elif (tuple(y.shape) != (B, L, H * dv) or y.dtype != torch.bfloat16 or y.device != dev
          or y.stride(-1) != 1):
        raise ValueError(f'gdn_prefill_fused: y must be a bf16 [{B}, {L}, {H * dv}] view with unit feature stride')
    S_out = torch.empty(nseq, H, dk, dv, dtype=torch.float32, device=dev)
    tout = [torch.empty(nseq, c, 3, dtype=torch.bfloat16, device=dev) for c in C]
    nbytes = _lib.lib().motif_gdn_chunk_workspace_bytes(H, dk, dv, 64, max(total, 1))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    al = a_log.detach().to(torch.bfloat16).contiguous()
    db = dt_bias.detach().to(torch.bfloat16).contiguous()
    nw = norm_weight.detach().to(torch.bfloat16).contiguous()
    rc = _lib.lib().motif_gdn_prefill_fused(
        proj.data_ptr(), proj.stride(0), proj.stride(1), *[int(o) for o in offsets],
        ws_[0].data_ptr(), ws_[1].data_ptr(), ws_[2].data_ptr(), 4,
        *[_lib.ptr(t) for t in tin], *[t.data_ptr() for t in tout],
        al.data_ptr(), db.data_ptr(), float(q_scale), nw.data_ptr(), float(norm_eps),
        _lib.ptr(S), S_out.data_ptr(), y.data_ptr(), y.stride(0), y.stride(1),
        B, H, L, dk, dv, _lib.ptr(cu_dev), _lib.ptr(coff_dev), nseq, total,
        ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    if rc == _lib.ERR_UNSUPPORTED:
        return None
    _lib.check(rc, 'motif_gdn_prefill_fused')
    return y, S_out, tuple(tout)
