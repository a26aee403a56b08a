'''GatedDeltaAttention with the reference interface (motif/block/attention/gdn_attn.py:19-219).

Same constructor arguments, parameter names / shapes / initialisation, cache
type and forward contract.  The six input projections (q, k, v, gate, a, b) run
as one GEMM against their concatenated weights.  The sequence mixing runs on the
HIP kernels:
  * prefill (L > 1): one call from the projections to the o_proj input
    (motif_gdn_prefill_fused: the chunk-preparation kernel computes the conv + SiLU,
    the q / k L2 norm and the gates itself; the output pass applies the GatedRMSNorm);
    shapes it does not serve run conv (motif_short_conv_silu_multi), gates and the
    chunked rule (motif_gdn_chunk_fwd_gated) as separate kernels;
  * decode (L == 1 with a cache): one fused kernel from the projections to the
    GatedRMSNorm output (motif_gdn_decode_fused).  It writes the new recurrent
    state and conv tails to fresh tensors that replace the cache's (the reference's
    update semantics, motif/model/cache.py:332-356), or, for an in-place cache (the
    graph-captured decode step), over the cache's own storage.
Calls that need gradients take the differentiable torch forms inside the ops.

Precision: the reference casts q/k/v/beta/g to fp32 before the delta rule
(:197).  Those tensors are produced in the activation dtype, so casting is
exact; this layer hands them to the kernel in that dtype and the kernel
computes in fp32 with an fp32 state, which yields the same inputs to the
recurrence.  The returned state is fp32.
'''
import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from motif.block.attention.base import AttentionOutput, BasicAttention
from motif.model.cache import GatedDeltaAttentionLayerCache
from motif.ops.autograd_path import wants_grad
from motif.ops.epilogue import gated_rms_norm_heads, gdn_gates, usable
from motif.ops.packed import PackedSeqs
from motif.ops import (
    GatedRMSNorm,
    cat_weights,
    project,
    HAS_TRITON,
    chunk_gated_delta_rule,
    gdn_decode_fused,
    recurrent_gated_delta_rule,
    short_conv_silu,
    short_conv_silu_varlen,
    chunk_gated_delta_rule_varlen,
    chunk_gated_delta_rule_gated_norm,
    gdn_prefill_fused,
    short_conv_silu_multi,
)


class GatedDeltaAttention(BasicAttention):
    '''Gated delta-net attention (GDN) layer.'''

    def __init__(
        self,
        hidden_size: int,
        num_heads: int,
        head_k_dim: Optional[int] = None,
        expand_v: float = 2.0,
        conv_size: int = 4,
        chunk_size: int = 64,
        bias: bool = False,
        dropout: float = 0.0,
        use_triton: bool = True,
        **kwargs,
    ):
        super().__init__(hidden_size=hidden_size, num_heads=num_heads, num_kv_heads=num_heads)
        self.dk = head_k_dim or self.head_dim
        self.dv = int(self.dk * expand_v)
        self.conv_size = conv_size
        self.chunk_size = chunk_size
        self.bias = bias
        self.dropout = dropout
        self.use_triton = bool(use_triton and HAS_TRITON)
        dk_all = self.num_heads * self.dk
        dv_all = self.num_heads * self.dv

        self.q_proj = nn.Linear(hidden_size, dk_all, bias=bias)
        self.k_proj = nn.Linear(hidden_size, dk_all, bias=bias)
        self.v_proj = nn.Linear(hidden_size, dv_all, bias=bias)
        self.a_proj = nn.Linear(hidden_size, self.num_heads, bias=bias)
        self.b_proj = nn.Linear(hidden_size, self.num_heads, bias=bias)
        self.g_proj = nn.Linear(hidden_size, dv_all, bias=bias)
        self.o_proj = nn.Linear(dv_all, hidden_size, bias=bias)

        self.q_conv = nn.Conv1d(dk_all, dk_all, conv_size, groups=dk_all, bias=False)
        self.k_conv = nn.Conv1d(dk_all, dk_all, conv_size, groups=dk_all, bias=False)
        self.v_conv = nn.Conv1d(dv_all, dv_all, conv_size, groups=dv_all, bias=False)

        self.A_log = nn.Parameter(torch.empty(self.num_heads))
        self.dt_bias = nn.Parameter(torch.empty(self.num_heads))
        self.init_gates()

        self.o_norm = GatedRMSNorm(self.dv)

    @torch.no_grad()
    def init_gates(self, generator: Optional[torch.Generator] = None) -> None:
        '''The decay parameters' initial values: A ~ U(1, 16) stored as log A, dt
        log-uniform in [1e-3, 1e-1] stored as softplus^-1(dt) (motif/block/attention/
        gdn_attn.py:99-104).  Drawn from `generator`, or from the global RNG as the
        reference's constructor does.'''
        n = self.num_heads
        A = torch.rand(n, generator=generator) * 15 + 1
        dt = torch.exp(torch.rand(n, generator=generator) * (math.log(0.1) - math.log(0.001)) + math.log(0.001))
        self.A_log.copy_(A.log().to(self.A_log))
        self.dt_bias.copy_((dt + torch.log(-torch.expm1(-dt))).to(self.dt_bias))

    @classmethod
    def cache_type(cls) -> type:
        return GatedDeltaAttentionLayerCache

    def _proj_weight(self):
        '''[q | k | v | gate | a | b] projection weight and bias as one matrix.'''
        return cat_weights(self, '_proj_cat', (self.q_proj, self.k_proj, self.v_proj, self.g_proj,
                                                self.a_proj, self.b_proj))

    def _proj_offsets(self):
        '''Column offsets of q, k, v, gate, a, b in the fused projection.'''
        hk, hv, H = self.num_heads * self.dk, self.num_heads * self.dv, self.num_heads
        return (0, hk, 2 * hk, 2 * hk + hv, 2 * hk + 2 * hv, 2 * hk + 2 * hv + H)

    def _project(self, hidden_states):
        '''All six projections -> (q, k, v, gate, a, b) views of one [B, L, ncols] result.'''
        w, b = self._proj_weight()
        proj = project(hidden_states, w, b)
        offs = self._proj_offsets()
        ends = offs[1:] + (proj.shape[-1],)
        return proj, tuple(proj[..., s:e] for s, e in zip(offs, ends))

    def _gates(self, a, b):
        if a.is_cuda and a.dtype in (torch.bfloat16, torch.float32) and b.dtype == a.dtype:
            return gdn_gates(a, b, self.A_log, self.dt_bias)  # torch form inside when grad is needed
        beta = torch.sigmoid(b).transpose(1, 2)
        g = -self.A_log.exp() * F.softplus(a + self.dt_bias)
        return beta, g.transpose(1, 2)

    def _heads(self, q, k, v, B, L, normalized=False):
        q = q.view(B, L, self.num_heads, self.dk).transpose(1, 2)
        k = k.view(B, L, self.num_heads, self.dk).transpose(1, 2)
        v = v.view(B, L, self.num_heads, self.dv).transpose(1, 2)
        if not normalized:
            q = F.normalize(q, dim=-1) * (self.dk ** -0.5)
            k = F.normalize(k, dim=-1)
        return q, k, v

    def _qkv(self, xs, tails, B, L, cu_seqlens=None, max_len=None):
        '''q / k / v projections `xs` through conv + SiLU; q and k then L2-normalised per
        head (q also scaled by dk^-1/2), inside the conv kernel when dk <= 64.'''
        fused = self.dk in (16, 32, 64)
        hd = self.dk if fused else None
        ws = (self.q_conv.weight, self.k_conv.weight, self.v_conv.weight)
        opts = ((hd, self.dk ** -0.5), (hd, 1.0), (None, 1.0))
        outs = None
        if xs[0].is_cuda and not wants_grad(xs, ws, tails):
            outs = short_conv_silu_multi(xs, ws, tails, [o[0] for o in opts], [o[1] for o in opts],
                                         cu_seqlens, max_len)
        if outs is not None:
            q, k, v = self._heads(outs[0][0], outs[1][0], outs[2][0], B, L, normalized=fused)
            return q, k, v, tuple(o[1] for o in outs)
        outs = []
        for i in range(3):
            if cu_seqlens is None:
                outs.append(short_conv_silu(xs[i], ws[i], tails[i], head_dim=opts[i][0], scale=opts[i][1]))
            else:
                outs.append(short_conv_silu_varlen(xs[i], ws[i], cu_seqlens, max_len,
                                                   head_dim=opts[i][0], scale=opts[i][1]))
        q, k, v = self._heads(outs[0][0], outs[1][0], outs[2][0], B, L, normalized=fused)
        return q, k, v, tuple(o[1] for o in outs)

    def _output(self, o, gate, B, L):
        '''GatedRMSNorm of [o || gate] per head, then o_proj.  One HIP pass over o and the
        gate (no concatenation) when the kernel serves the tensors.'''
        o = o.to(gate.dtype)
        if self.o_norm.weight is not None and usable(o, gate) and not wants_grad(self.o_norm):
            y = gated_rms_norm_heads(o, gate, self.o_norm.weight, self.o_norm.eps)
            return project(y, self.o_proj.weight, self.o_proj.bias)
        o = o.transpose(1, 2)
        gate = gate.reshape(B, L, self.num_heads, self.dv)
        o = self.o_norm(torch.cat([o, gate], dim=-1)).reshape(B, L, -1)
        return project(o, self.o_proj.weight, self.o_proj.bias)

    def _prefill_fused(self, proj, tails, S0, cu_seqlens=None, y=None):
        '''The whole prefill after the projections in three kernels, or None when the
        fused kernels do not serve this layer / these inputs.'''
        if self.o_norm.weight is None or self.conv_size != 4 or wants_grad(proj, self):
            return None
        return gdn_prefill_fused(proj, self._proj_offsets(), (self.q_conv.weight, self.k_conv.weight,
                                                             self.v_conv.weight), tails, self.A_log, self.dt_bias,
                                 self.dk ** -0.5, self.o_norm.weight, self.o_norm.eps, S0, self.num_heads, self.dk,
                                 self.dv, cu_seqlens, y=y)

    def prefill_core(self, hidden_states, past_key_value, out):
        '''The prefill of forward() up to the o_proj input (no reference counterpart as
        one call): the projections, conv, gates, chunk rule and GatedRMSNorm, written into
        `out` (a bf16 [B, L, H dv] view with unit feature stride, e.g. the left columns of
        a wider buffer that another projection's input fills), with `past_key_value`
        (None, or a GatedDeltaAttentionLayerCache) updated as forward() updates it.
        Returns False, before anything ran, when the fused prefill kernels do not serve
        this call; the caller then runs forward().'''
        B, L, _ = hidden_states.shape
        if (L < 2 or self.o_norm.weight is None or self.conv_size != 4 or self.dk not in (32, 64)
                or self.dv not in (64, 128) or hidden_states.dtype != torch.bfloat16 or not hidden_states.is_cuda
                or wants_grad(hidden_states, self)):
            return False
        tails, S0 = (None, None, None), None
        if past_key_value is not None:
            if not isinstance(past_key_value, GatedDeltaAttentionLayerCache):
                return False
            if past_key_value.conv_state is not None:
                tails = past_key_value.conv_state
            S0 = past_key_value.state
        if S0 is not None and (S0.dtype != torch.float32 or not S0.is_contiguous()
                               or tuple(S0.shape) != (B, self.num_heads, self.dk, self.dv)):
            return False
        if any(t is None for t in tails) and any(t is not None for t in tails):
            return False
        proj, _ = self._project(hidden_states)
        whole = self._prefill_fused(proj, tails, S0, y=out)
        if whole is None:
            return False
        _, S, conv_tails = whole
        if past_key_value is not None:
            past_key_value.update(S, conv_tails, steps=L)
        return True

    def _decode_fusable(self, hidden_states, cache):
        '''True when one decode step can run as the fused kernel: one token, a cache whose
        state / tails (if present) are in the kernel's layout, inference only.'''
        B, L, _ = hidden_states.shape
        if L != 1 or not hidden_states.is_cuda or hidden_states.dtype not in (torch.float32, torch.bfloat16):
            return False
        if self.dk not in (16, 32, 64) or self.dv > 128 or not 2 <= self.conv_size <= 5:
            return False
        if self.o_norm.weight is None or wants_grad(hidden_states, self):
            return False
        S = cache.state
        if S is not None and (S.dtype != torch.float32 or not S.is_contiguous() or not S.is_cuda
                              or tuple(S.shape) != (B, self.num_heads, self.dk, self.dv)):
            return False
        if cache.conv_state is not None:
            chans = (self.num_heads * self.dk, self.num_heads * self.dk, self.num_heads * self.dv)
            for t, c in zip(cache.conv_state, chans):
                if (t is None or t.dtype != hidden_states.dtype or not t.is_contiguous() or not t.is_cuda
                        or tuple(t.shape) != (B, c, self.conv_size - 1)):
                    return False
        return True

    def _decode_step(self, hidden_states, cache):
        '''One token: the fused projection, the fused decode kernel, o_proj.'''
        B = hidden_states.shape[0]
        w, b = self._proj_weight()
        proj = project(hidden_states.view(B, -1), w, b)
        return project(self._decode_core(proj, cache), self.o_proj.weight, self.o_proj.bias)

    def _decode_core(self, proj, cache):
        '''The step from the projected token (proj [B, ncols] or [B, 1, ncols]) to the
        o_proj input [B, 1, H dv]: one fused kernel (conv, gates, recurrence, output
        norm).  An empty cache starts from zero state and tails; an in-place cache is
        updated over its own storage, any other receives new tensors.'''
        B = proj.shape[0]
        dev, dt = proj.device, proj.dtype
        H, K = self.num_heads, self.conv_size
        chans = (H * self.dk, H * self.dk, H * self.dv)
        state, tails = cache.state, cache.conv_state
        if state is None:
            state = torch.zeros(B, H, self.dk, self.dv, dtype=torch.float32, device=dev)
        if tails is None:
            tails = tuple(torch.zeros(B, c, K - 1, dtype=dt, device=dev) for c in chans)
        if cache.in_place:
            state_out, tails_out = state, tails
        else:
            state_out, tails_out = torch.empty_like(state), tuple(torch.empty_like(t) for t in tails)
        y = gdn_decode_fused(proj.view(B, -1), self._proj_offsets(),
                             (self.q_conv.weight, self.k_conv.weight, self.v_conv.weight),
                             tails, self.A_log, self.dt_bias, self.o_norm.weight, self.o_norm.eps,
                             state, H, self.dk, self.dv, tails_out=tails_out, state_out=state_out)
        cache.update(state_out, tails_out, steps=1)
        return y.view(B, 1, -1)

    def decode_split(self, hidden_states, cache):
        '''A decode step in three parts, for a caller that batches the projections with
        other launches: (W_in, core, W_out) or None when the fused decode does not serve
        this call.  The caller computes proj = hidden_states W_in^T, calls core(proj) --
        which runs the step, updates `cache` and returns (o, None) -- and applies
        o_proj as o W_out^T.  Together: what forward() computes for this step.'''
        if not isinstance(cache, GatedDeltaAttentionLayerCache) or not self._decode_fusable(hidden_states, cache):
            return None
        w, b = self._proj_weight()
        if b is not None or self.o_proj.bias is not None:
            return None
        return w, (lambda proj: (self._decode_core(proj, cache), None)), self.o_proj.weight

    def forward(self, hidden_states: torch.Tensor, past_key_value=None) -> AttentionOutput:
        '''Run the layer over [B, L, hidden]; continue from / update `past_key_value`.'''
        B, L, _ = hidden_states.shape
        use_cache = past_key_value is not None
        if use_cache:
            if not isinstance(past_key_value, GatedDeltaAttentionLayerCache):
                raise TypeError(f'GatedDeltaAttention requires GatedDeltaAttentionLayerCache, '
                                f'got {type(past_key_value).__name__}')
            tails = past_key_value.conv_state if past_key_value.conv_state is not None else (None, None, None)
            S0 = past_key_value.state
        else:
            tails = (None, None, None)
            S0 = None

        if use_cache and self._decode_fusable(hidden_states, past_key_value):
            output = self._decode_step(hidden_states, past_key_value)
            return AttentionOutput(output=output, past_key_value=past_key_value)

        proj, (xq, xk, xv, gate, xa, xb) = self._project(hidden_states)
        whole = self._prefill_fused(proj, tails, S0) if L > 1 else None
        if whole is not None:
            y, S, conv_tails = whole
            output = project(y, self.o_proj.weight, self.o_proj.bias)
            if use_cache:
                past_key_value.update(S, conv_tails, steps=L)
                return AttentionOutput(output=output, past_key_value=past_key_value)
            return AttentionOutput(output=output, payload={'state': S.detach(), 'conv_state': conv_tails})
        q, k, v, (cq, ck, cv) = self._qkv((xq, xk, xv), tails, B, L)
        beta, g = self._gates(xa, xb)

        fused = None
        if L > 1 and self.o_norm.weight is not None:
            fused = chunk_gated_delta_rule_gated_norm(q, k, v, beta, g, gate, self.o_norm.weight, self.o_norm.eps,
                                                      S0, self.chunk_size)
        if fused is not None:
            y, S = fused
            output = project(y, self.o_proj.weight, self.o_proj.bias)
        else:
            if L == 1:
                o, S = recurrent_gated_delta_rule(q, k, v, beta, g, S0)
            else:
                o, S = chunk_gated_delta_rule(q, k, v, beta, g, S0, self.chunk_size)
            output = self._output(o, gate, B, L)

        if use_cache:
            past_key_value.update(S, (cq, ck, cv), steps=L)
            return AttentionOutput(output=output, past_key_value=past_key_value)
        payload = {'state': S.detach(), 'conv_state': tuple(c.detach() for c in (cq, ck, cv))}
        return AttentionOutput(output=output, payload=payload)

    def forward_varlen(self, hidden_states: torch.Tensor, cu_seqlens) -> AttentionOutput:
        '''Packed sequences (B == 1): every sequence starts from zero state and zero
        conv tails.  `cu_seqlens` is an int tensor or a motif.ops.packed.PackedSeqs (then
        nothing is read back from the device).  Returns the output and a payload with
        the per-sequence final states [nseq, H, dk, dv] and conv tails [nseq, D, K-1].'''
        B, L, _ = hidden_states.shape
        if B != 1:
            raise ValueError('forward_varlen expects packed sequences with B == 1')
        cu_seqlens = PackedSeqs.of(cu_seqlens, L, hidden_states.device)
        max_len = cu_seqlens.max_len
        proj, (xq, xk, xv, gate, xa, xb) = self._project(hidden_states)
        whole = self._prefill_fused(proj, (None, None, None), None, cu_seqlens)
        if whole is not None:
            y, S, conv_tails = whole
            return AttentionOutput(output=project(y, self.o_proj.weight, self.o_proj.bias),
                                   payload={'state': S, 'conv_state': conv_tails})
        q, k, v, (cq, ck, cv) = self._qkv((xq, xk, xv), (None, None, None), B, L, cu_seqlens, max_len)
        beta, g = self._gates(xa, xb)
        fused = None
        if self.o_norm.weight is not None:
            fused = chunk_gated_delta_rule_gated_norm(q, k, v, beta, g, gate, self.o_norm.weight, self.o_norm.eps,
                                                      None, self.chunk_size, cu_seqlens=cu_seqlens)
        if fused is not None:
            y, S = fused
            output = project(y, self.o_proj.weight, self.o_proj.bias)
        else:
            o, S = chunk_gated_delta_rule_varlen(q, k, v, beta, g, cu_seqlens, None, self.chunk_size)
            output = self._output(o, gate, B, L)
        return AttentionOutput(output=output, payload={'state': S, 'conv_state': (cq, ck, cv)})
