'''Fused single-token GatedDeltaAttention step on the HIP kernel
(`motif_gdn_decode_fused`): conv + SiLU, q / k L2 normalisation, gates, the
delta-rule state update and the GatedRMSNorm, from the layer's input
projections to the input of o_proj.  The reference runs these as separate ops in
the L == 1 path of motif/block/attention/gdn_attn.py:183-209.
'''
import torch

from . import _lib


def gdn_decode_fused(proj, offsets, conv_weights, tails, a_log, dt_bias, norm_weight, norm_eps, state,
                     H, dk, dv, tails_out=None, state_out=None):
    '''One decode step.

    Args:
        proj: [B, ncols] projections of the new token (row-contiguous features).
        offsets: column offsets (q, k, v, gate, a, b) inside proj.
        conv_weights: (wq, wk, wv) nn.Conv1d weights [C, 1, K].
        tails: (tq, tk, tv) conv tails [B, C, K-1], contiguous.
        a_log, dt_bias: [H];  norm_weight: [dv].
        state: [B, H, dk, dv] fp32 contiguous.
        tails_out, state_out: where the shifted tails and the new state go (default:
            `tails` / `state` themselves, i.e. an in-place update).

    Returns:
        y [B, H * dv] (GatedRMSNorm output, the input of o_proj).
    '''
    B = proj.shape[0]
    dt = proj.dtype
    if proj.stride(-1) != 1:
        proj = proj.contiguous()
    K = conv_weights[0].shape[-1]
    ws = [w.detach().reshape(w.shape[0], K).to(dt).contiguous() for w in conv_weights]
    for t in tails:
        if t.dtype != dt or not t.is_contiguous():
            raise ValueError('gdn_decode_fused: conv tails must be contiguous and in the activation dtype')
    tails_out = tails if tails_out is None else tails_out
    state_out = state if state_out is None else state_out
    for t, o in zip(tails, tails_out):
        if o.shape != t.shape or o.dtype != dt or not o.is_contiguous():
            raise ValueError('gdn_decode_fused: output tails must match the input tails')
    for t in (state, state_out):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.shape != (B, H, dk, dv):
            raise ValueError('gdn_decode_fused: state must be contiguous fp32 [B, H, dk, dv]')
    al = a_log.detach().to(dt).contiguous()
    db = dt_bias.detach().to(dt).contiguous()
    nw = norm_weight.detach().to(dt).contiguous()
    y = torch.empty(B, H * dv, dtype=dt, device=proj.device)
    rc = _lib.lib().motif_gdn_decode_fused(
        proj.data_ptr(), proj.stride(0), *[int(o) for o in offsets],
        ws[0].data_ptr(), ws[1].data_ptr(), ws[2].data_ptr(),
        tails[0].data_ptr(), tails[1].data_ptr(), tails[2].data_ptr(),
        tails_out[0].data_ptr(), tails_out[1].data_ptr(), tails_out[2].data_ptr(),
        al.data_ptr(), db.data_ptr(), nw.data_ptr(), float(norm_eps),
        state.data_ptr(), state_out.data_ptr(), y.data_ptr(), y.stride(0), B, H, dk, dv, K,
        _lib.dtype_code(dt), _lib.stream_ptr(proj.device))
    _lib.check(rc, 'motif_gdn_decode_fused')
    return y
