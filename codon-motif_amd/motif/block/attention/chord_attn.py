'''ChordAttention: softmax attention with the per-head gated geometric-decay (GGD)
bias, behind the reference layer interface (motif/block/attention/chord_attn.py:59-379:
constructor, parameter names / shapes / initial values, cache type, forward
arguments and AttentionOutput contract).

How a call is served:
  * decode over a StaticKVLayerCache (the graph-captured step): one projection
    GEMM, one kernel for the q / k RMSNorms and the append at the device cursor,
    the device-cursor attention kernel (which also advances the cursor), the gated
    output projection -- no host value enters the launch sequence;
  * other inference calls on bf16 / fp32 ROCm tensors with head_dim 64: the HIP
    kernels with host positions (apply_chord_attention);
  * calls that need gradients: the differentiable torch form (inside
    apply_chord_attention);
  * an attention mask, a request for the attention weights, a tensor position
    (`embedding_start` as a tensor) or a shape the kernels do not serve (fp16,
    head_dim != 64): the explicit materialised-bias computation below, the
    reference's rule for leaving its kernel (chord_attn.py:295-298).
'''
import warnings
from typing import Optional, Union

import torch
import torch.nn as nn

from motif.block.attention.base import AttentionOutput, BasicAttention
from motif.model.cache import KVLayerCache, StaticKVLayerCache, expand_kv_heads
from motif.ops import RMSNorm, apply_chord_attention, apply_chord_attention_varlen
from motif.ops.packed import PackedSeqs
from motif.ops import _lib
from motif.ops.autograd_path import wants_grad
from motif.ops.chord_attention import (HEAD_DIMS, chord_decode_cursor, chord_decode_step, chord_decode_step_serves,
                                       chord_decode_step_workspace, chord_decode_workspace, serves_head_dim)
from motif.ops.epilogue import mul_sigmoid, usable
from motif.ops.linear_rows import cat_weights, linear_rows, project, rows_eligible

GGD_EPS = 1e-5
_KERNEL_DTYPES = (torch.bfloat16, torch.float32)  # the input kernel (norms, cache append)
_ATTN_DTYPES = (torch.bfloat16, torch.float32, torch.float16)  # the attention kernels
_DECODE_ROWS = 8  # (GQA group x L) up to this size is a decode-shaped call
# Cursor decode steps in one launch (motif_chord_decode_step) where it serves; False keeps
# the input kernel + decode kernels (the same bits, three launches).
FUSED_STEP = True


class LogPositions:
    '''ln(1), ln(2), ... in fp32, one table per device, grown in 4096-entry pages.
    The log_n factor of a query at absolute position p is table[p] = ln(p + 1)
    (motif/block/attention/chord_attn.py:21-43 with :274-283).'''

    _tables = {}

    @classmethod
    def get(cls, n: int, device) -> torch.Tensor:
        device = torch.device(device)
        t = cls._tables.get(device)
        if t is None or t.numel() < n:
            size = max(4096, -(-n // 4096) * 4096)
            t = torch.log(torch.arange(1, size + 1, dtype=torch.float32, device=device))
            cls._tables[device] = t
        return t

    @classmethod
    def at(cls, start: int, n: int, device) -> torch.Tensor:
        return cls.get(start + n, device)[start:start + n]


def ggd_bias(alpha: torch.Tensor, beta: torch.Tensor, mu: torch.Tensor, distance: torch.Tensor,
             eps: float = GGD_EPS) -> torch.Tensor:
    '''-alpha_h (|d - mu_h| + eps) ** beta_h for every head h and distance d = key -
    query position; alpha, beta, mu [H], distance any shape -> [H, *distance.shape].'''
    ex = (1,) * distance.dim()
    dist = distance.to(alpha.dtype)[None]
    return -alpha.view(-1, *ex) * ((dist - mu.view(-1, *ex)).abs() + eps) ** beta.view(-1, *ex)


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.float() if t.dtype in (torch.float16, torch.bfloat16) else t


class ChordAttention(BasicAttention):
    '''Softmax attention with the per-head gated geometric-decay (GGD) bias.'''

    def __init__(self, hidden_size: int, num_heads: int, num_kv_heads: Optional[int] = None, **kwargs):
        super().__init__(hidden_size=hidden_size, num_heads=num_heads, num_kv_heads=num_kv_heads)
        self.q_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.k_proj = nn.Linear(hidden_size, self.kv_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, self.kv_dim, bias=False)
        self.o_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.g_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.q_norm = RMSNorm(self.head_dim)
        self.k_norm = RMSNorm(self.head_dim)
        self.theta_alpha = nn.Parameter(torch.zeros(num_heads))
        self.theta_beta = nn.Parameter(torch.zeros(num_heads))
        self.theta_mu = nn.Parameter(torch.zeros(num_heads), requires_grad=False)
        self.ssmax_s = nn.Parameter(torch.ones(num_heads))
        self._warned = False

    @classmethod
    def cache_type(cls) -> type:
        return KVLayerCache

    # ------------------------------------------------------------------ parameters
    def ggd_params(self):
        '''(alpha, beta, mu, ssmax) in fp32: alpha = e^theta_alpha, beta = theta_beta,
        mu = e^theta_mu - e^-theta_mu, ssmax = ssmax_s (chord_attn.py:126-138).
        Inference reuses one contiguous copy until a parameter changes.'''
        thetas = (self.theta_alpha, self.theta_beta, self.theta_mu, self.ssmax_s)

        def compute():
            ta, tb, tm, ss = (_f32(t) for t in thetas)
            return tuple(t.contiguous() for t in (ta.exp(), tb, tm.exp() - (-tm).exp(), ss))

        if wants_grad(*thetas):
            return compute()
        key = tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in thetas)
        memo = self.__dict__.get('_ggd_memo')
        if memo is None or memo[0] != key:
            with torch.no_grad():
                memo = (key, compute())
            self.__dict__['_ggd_memo'] = memo
        return memo[1]

    @torch.no_grad()
    def relative_prior(self, max_distance: int, device=None, dtype=torch.float32) -> torch.Tensor:
        '''The GGD bias of every head at distances -max_distance .. max_distance:
        [num_heads, 2 * max_distance + 1].'''
        alpha, beta, mu, _ = self.ggd_params()
        device = self.theta_alpha.device if device is None else device
        d = torch.arange(-max_distance, max_distance + 1, device=device)
        return ggd_bias(alpha.to(device), beta.to(device), mu.to(device), d).to(dtype)

    # ------------------------------------------------------------------ routing
    def _kernel_serves(self, x: torch.Tensor) -> bool:
        '''Inputs the HIP kernels take; ROCm inputs they do not take go to the
        materialised path with a one-time warning.'''
        if not x.is_cuda:
            return False
        if x.dtype in _ATTN_DTYPES and serves_head_dim(self.head_dim) and _lib.available():
            return True
        if not self._warned:
            warnings.warn(f'ChordAttention: no HIP kernel for {x.dtype} / head_dim {self.head_dim}; '
                          'computing the attention with the materialised bias', RuntimeWarning)
            self._warned = True
        return False

    def _prep_fusable(self, x: torch.Tensor, cache) -> bool:
        '''The single input kernel (q / k RMSNorms, cache append) serves this call.'''
        if not x.is_cuda or x.dtype not in _KERNEL_DTYPES or not _lib.available():
            return False
        row_bytes = self.head_dim * x.element_size()
        if row_bytes % 16 or row_bytes > 512:
            return False
        if self.q_norm.weight is None or self.k_norm.weight is None or self.q_norm.eps != self.k_norm.eps:
            return False
        if cache is not None and (cache.wide or type(cache) not in (KVLayerCache, StaticKVLayerCache)):
            return False
        return not wants_grad(x, self)

    def _on_cursor(self, x, cache, q_start) -> bool:
        '''Decode over a static cache at its own position: the device-cursor path.'''
        L = x.shape[1]
        return (isinstance(cache, StaticKVLayerCache) and cache.capacity > 0 and not cache.wide
                and self.head_dim in HEAD_DIMS
                and q_start == cache.length and cache.length + L <= cache.capacity
                and cache.k.dtype == x.dtype and self.num_kv_queries * L <= _DECODE_ROWS
                and self._prep_fusable(x, cache))

    # ------------------------------------------------------------------ inputs
    def _fused_proj(self, x):
        w, b = cat_weights(self, '_proj_cat', (self.q_proj, self.k_proj, self.v_proj, self.g_proj))
        proj = project(x, w, b)
        return proj if proj.stride(-1) == 1 else proj.contiguous()

    def _prep(self, proj, q, k_dst, v_dst, length_dev, pos, capacity):
        B, L = proj.shape[0], proj.shape[1]
        hs, kd = self.hidden_size, self.kv_dim
        dt = proj.dtype
        rc = _lib.lib().motif_chord_qkv_prep(
            proj.data_ptr(), proj.stride(0), proj.stride(1), 0, hs, hs + kd,
            self.q_norm.weight.to(dt).contiguous().data_ptr(), self.k_norm.weight.to(dt).contiguous().data_ptr(),
            float(self.q_norm.eps), *_lib.t4(q), *_lib.t4(k_dst), *_lib.t4(v_dst),
            _lib.ptr(length_dev), pos, capacity, B, L, self.num_heads, self.num_kv_heads, self.head_dim,
            _lib.dtype_code(dt), _lib.stream_ptr(proj.device))
        _lib.check(rc, 'motif_chord_qkv_prep')

    def _inputs(self, hidden_states, kv_states, cache, fused: bool):
        '''(q [B, H, L, D], k / v [B, h, S, D] -- every cached position plus the new ones,
        gate pre-activation g [B, L, hidden]).  The fused form writes k / v straight
        into the cache's slab.'''
        B, L, _ = hidden_states.shape
        if fused:
            proj = self._fused_proj(hidden_states)
            hs, kd = self.hidden_size, self.kv_dim
            q = torch.empty(B, self.num_heads, L, self.head_dim, dtype=proj.dtype, device=proj.device)
            if cache is None:
                k = torch.empty(B, self.num_kv_heads, L, self.head_dim, dtype=proj.dtype, device=proj.device)
                v = torch.empty_like(k)
                self._prep(proj, q, k, v, None, 0, L)
            else:
                ks, vs, first = cache.append_slots(L, q.new_empty(B, self.num_kv_heads, 0, self.head_dim))
                length_dev = cache.length_dev if isinstance(cache, StaticKVLayerCache) else None
                self._prep(proj, q, ks, vs, length_dev, first, ks.shape[2])
                k, v = cache.k, cache.v
            return q, k, v, proj[..., hs + 2 * kd:]
        kv = hidden_states if kv_states is None else kv_states
        if kv is hidden_states:
            proj = self._fused_proj(hidden_states) if hidden_states.is_cuda else None
        else:
            proj = None
        if proj is not None:
            hs, kd = self.hidden_size, self.kv_dim
            xq, xk, xv, g = (proj[..., :hs], proj[..., hs:hs + kd], proj[..., hs + kd:hs + 2 * kd],
                             proj[..., hs + 2 * kd:])
        else:
            xq, xk, xv, g = self.q_proj(hidden_states), self.k_proj(kv), self.v_proj(kv), self.g_proj(hidden_states)
        q = self.q_norm(self.reshape_q(xq, L, B))
        k = self.k_norm(self.reshape_kv(xk, kv.shape[1], B))
        v = self.reshape_kv(xv, kv.shape[1], B)
        if cache is not None:
            k, v = cache.update(k, v, dim=2)
        return q, k, v, g

    def _log_n(self, q_start, L, B, device, section_log_len):
        '''log_n [B, L] or [L]: section_log_len when given, else ln(q_start + i + 1).'''
        if section_log_len is not None:
            sl = section_log_len[..., 0] if section_log_len.dim() == 3 else section_log_len
            if tuple(sl.shape) != (B, L):
                raise ValueError(f'section_log_len must be [B, q_len] or [B, q_len, 1] with B={B}, '
                                 f'q_len={L}; got {tuple(section_log_len.shape)}')
            return sl.float()
        if isinstance(q_start, torch.Tensor):
            first = q_start.reshape(-1)[:1].to(device=device, dtype=torch.float32)
            return torch.log(first + torch.arange(1, L + 1, device=device, dtype=torch.float32))
        return LogPositions.at(q_start, L, device)

    def _gated_output(self, out, g_pre):
        '''o_proj(out) * sigmoid(g_pre); decode-sized bf16 rows take one kernel with the
        gate in its epilogue.'''
        if self.o_proj.bias is None and rows_eligible(out, self.o_proj.weight) and not wants_grad(out, self.o_proj):
            return linear_rows(out, self.o_proj.weight, 'gate', aux=g_pre)
        o = self.o_proj(out)
        if o.shape == g_pre.shape and usable(o, g_pre) and not wants_grad(o, g_pre):
            return mul_sigmoid(o, g_pre)
        return o * torch.sigmoid(g_pre)

    def _merge_heads(self, out):
        B, H, L, D = out.shape
        return out.transpose(1, 2).reshape(B, L, H * D)

    @staticmethod
    def _heads_out(q):
        '''An attention destination [B, H, L, D] laid out as [B, L, H, D], so that
        _merge_heads of it is a view rather than a copy.'''
        B, H, L, D = q.shape
        return torch.empty((B, L, H, D), dtype=q.dtype, device=q.device).transpose(1, 2)

    # ------------------------------------------------------------------ forward
    def forward(
        self,
        hidden_states: torch.Tensor,
        kv_states: Optional[torch.Tensor] = None,
        attention_mask: Optional[torch.Tensor] = None,
        output_attentions: bool = False,
        embedding_start: Union[int, torch.Tensor] = 0,
        past_key_value: Optional[KVLayerCache] = None,
        section_log_len: Optional[torch.Tensor] = None,
    ) -> AttentionOutput:
        res = self._attend(hidden_states, kv_states, attention_mask, output_attentions, embedding_start,
                           past_key_value, section_log_len)
        if isinstance(res, AttentionOutput):
            return res
        merged, g, cache = res
        return AttentionOutput(output=self._gated_output(merged, g), past_key_value=cache)

    def prefill_parts(self, hidden_states: torch.Tensor, past_key_value: Optional[KVLayerCache] = None,
                      embedding_start: Union[int, torch.Tensor] = 0):
        '''A self-attention call on the prefill kernels, stopped before the output side:
        (merged heads [B, L, H * D], the output gate's pre-activation g [B, L, H * D],
        cache), so that the caller applies o_proj and the gate itself (the decoder folds
        the gate into its residual pass).  None, before anything runs, for every call
        that forward serves another way (decode at the cache cursor, the materialised
        path).'''
        return self._attend(hidden_states, None, None, False, embedding_start, past_key_value, None,
                            parts_only=True)

    def _attend(self, hidden_states, kv_states, attention_mask, output_attentions, embedding_start,
                past_key_value, section_log_len, parts_only=False):
        '''forward up to the output side: (merged heads, gate pre-activation, cache) on
        the prefill kernels, or the finished AttentionOutput of the cursor / materialised
        routes (None for those with `parts_only`).'''
        cache = past_key_value if isinstance(past_key_value, KVLayerCache) else None
        self_attn = kv_states is None or kv_states is hidden_states
        B, L, _ = hidden_states.shape
        q_start = embedding_start
        # an int position of 0 means "continue the cache" (chord_attn.py:266-268)
        if cache is not None and isinstance(q_start, int) and q_start == 0 and cache.seq_length > 0:
            q_start = cache.seq_length
        kernel = (attention_mask is None and not output_attentions and not isinstance(q_start, torch.Tensor)
                  and self._kernel_serves(hidden_states))

        if kernel and self_attn and section_log_len is None and self._on_cursor(hidden_states, cache, q_start):
            return None if parts_only else self._cursor_step(hidden_states, cache)
        if parts_only and not kernel:
            return None

        fused = kernel and self_attn and self._prep_fusable(hidden_states, cache)
        q, k, v, g = self._inputs(hidden_states, None if self_attn else kv_states, cache, fused)
        log_n = self._log_n(q_start, L, B, hidden_states.device, section_log_len)
        if kernel:
            alpha, beta, mu, ssmax = self.ggd_params()
            out = apply_chord_attention(q, k, v, alpha, beta, mu, ssmax,
                                        log_n if log_n.dim() == 2 else log_n.expand(B, L),
                                        q_start=int(q_start), softmax_scale=self.head_dim ** -0.5, eps=GGD_EPS,
                                        out=self._heads_out(q))
            return self._merge_heads(out), g, cache
        return self._materialised(q, k, v, g, q_start, log_n, attention_mask, output_attentions, cache)

    def _cursor_step(self, x, cache: StaticKVLayerCache) -> AttentionOutput:
        '''Decode at the static cache's device cursor: append, attend, advance -- all
        on the device, so the launch sequence is the same for every token.'''
        out, g_pre = self._cursor_core(self._fused_proj(x), cache)
        return AttentionOutput(output=self._gated_output(out, g_pre), past_key_value=cache)

    def decode_split(self, hidden_states, cache, embedding_start=0, attention_mask=None):
        '''A decode step in three parts, for a caller that batches the projections with
        other launches: (W_in, core, W_out) or None when the device-cursor decode does not
        serve this call (same conditions as forward()).  The caller computes
        proj = hidden_states W_in^T, calls core(proj) -- which appends to `cache`,
        attends, advances and returns (out, g_pre) -- and applies the gated o_proj,
        (out W_out^T) * sigmoid(g_pre).  Together: what forward() computes for this step.'''
        if not isinstance(cache, StaticKVLayerCache) or attention_mask is not None:
            return None
        q_start = embedding_start
        if isinstance(q_start, int) and q_start == 0 and cache.seq_length > 0:
            q_start = cache.seq_length
        if isinstance(q_start, torch.Tensor) or not self._kernel_serves(hidden_states):
            return None
        if not self._on_cursor(hidden_states, cache, q_start):
            return None
        w, b = cat_weights(self, '_proj_cat', (self.q_proj, self.k_proj, self.v_proj, self.g_proj))
        if b is not None or self.o_proj.bias is not None:
            return None
        return w, (lambda proj: self._cursor_core(proj, cache)), self.o_proj.weight

    def _cursor_core(self, proj, cache: StaticKVLayerCache):
        '''The cursor step from the projected tokens proj [B, L, q|k|v|g]: (merged
        attention output [B, L, hidden], gate pre-activation [B, L, hidden]).'''
        B, L = proj.shape[0], proj.shape[1]
        ks, vs = cache._slab
        if cache.__dict__.get('log_table') is None or cache.log_table.numel() < cache.capacity:
            cache.log_table = LogPositions.get(cache.capacity, proj.device)  # held: a graph keeps its address
        alpha, beta, mu, ssmax = self.ggd_params()
        if FUSED_STEP and chord_decode_step_serves(proj, self.num_heads, self.num_kv_heads, self.head_dim):
            # norms, append, attention, merge and cursor advance in one launch
            if cache.step_workspace is None:
                cache.step_workspace = chord_decode_step_workspace(B, self.num_heads, self.num_kv_heads, L,
                                                                   cache.capacity, proj.device)
            dt = proj.dtype
            hs, kd = self.hidden_size, self.kv_dim
            out = chord_decode_step(proj, (0, hs, hs + kd), self.q_norm.weight.to(dt).contiguous(),
                                    self.k_norm.weight.to(dt).contiguous(), self.q_norm.eps, ks, vs, cache.length_dev,
                                    alpha, beta, mu, ssmax, cache.log_table, self.num_heads, self.head_dim ** -0.5,
                                    GGD_EPS, cache.step_workspace)
        else:
            q = torch.empty(B, self.num_heads, L, self.head_dim, dtype=proj.dtype, device=proj.device)
            self._prep(proj, q, ks, vs, cache.length_dev, -1, cache.capacity)
            if cache.decode_workspace is None:
                cache.decode_workspace = chord_decode_workspace(B, self.num_heads, self.num_kv_heads, L, cache.capacity,
                                                                self.head_dim, proj.dtype, proj.device)
            out = chord_decode_cursor(q, ks, vs, cache.length_dev, alpha, beta, mu, ssmax, cache.log_table,
                                      self.head_dim ** -0.5, GGD_EPS, workspace=cache.decode_workspace)
        cache.length += L
        cache.cursor_steps = getattr(cache, 'cursor_steps', 0) + 1
        return self._merge_heads(out), proj[..., self.hidden_size + 2 * self.kv_dim:]

    def forward_varlen(self, hidden_states: torch.Tensor, cu_seqlens) -> AttentionOutput:
        '''Packed sequences (B == 1; new): each sequence attends causally within itself
        with positions (and log_n) restarting at 0.  `cu_seqlens` is an int tensor or a
        motif.ops.packed.PackedSeqs (then nothing is read back from the device).  The
        payload holds the packed keys and values.'''
        B, T, _ = hidden_states.shape
        if B != 1:
            raise ValueError('forward_varlen expects packed sequences with B == 1')
        ps = PackedSeqs.of(cu_seqlens, T, hidden_states.device)
        fused = self._prep_fusable(hidden_states, None)
        q, k, v, g = self._inputs(hidden_states, None, None, fused)
        table = LogPositions.get(max(ps.max_len, 1), hidden_states.device)
        log_n = table[ps.positions()][None]
        alpha, beta, mu, ssmax = self.ggd_params()
        out = apply_chord_attention_varlen(q, k, v, alpha, beta, mu, ssmax, log_n, ps,
                                           softmax_scale=self.head_dim ** -0.5, eps=GGD_EPS, out=self._heads_out(q))
        return AttentionOutput(output=self._gated_output(self._merge_heads(out), g), payload={'k': k, 'v': v})

    def _materialised(self, q, k, v, g, q_start, log_n, attention_mask, output_attentions, cache):
        '''Attention with the bias matrix built explicitly: for masks, attention weights,
        tensor positions and shapes without a kernel.  Rounding follows the reference's
        eager computation (chord_attn.py:316-361): q.k^T and its scaling in the input
        dtype, then fp32 logits (+ bias, x ssmax * log_n, floor at finfo.min / 4), the
        causal and user masks, softmax, weights cast back before the product with v.'''
        B, H, L, D = q.shape
        S = k.shape[2]
        kf, vf = expand_kv_heads(k, H), expand_kv_heads(v, H)
        scores = torch.matmul(q, kf.transpose(-2, -1)) * (D ** -0.5)
        fdt = torch.float32 if scores.dtype in (torch.float16, torch.bfloat16) else scores.dtype
        alpha, beta, mu, ssmax = self.ggd_params()
        dev = scores.device
        q_pos = torch.arange(L, device=dev) + (q_start.to(dev).reshape(-1)[:1] if isinstance(q_start, torch.Tensor)
                                               else q_start)
        k_pos = torch.arange(S, device=dev)
        bias = ggd_bias(alpha, beta, mu, k_pos[None, :] - q_pos[:, None]).to(fdt)         # [H, L, S]
        ln = log_n.view(1, 1, L, 1) if log_n.dim() == 1 else log_n.view(B, 1, L, 1)
        logits = (scores.to(fdt) + bias[None]) * (ssmax.view(1, H, 1, 1).to(fdt) * ln.to(fdt))
        logits = logits.clamp_min(torch.finfo(fdt).min / 4)
        logits = logits.masked_fill(k_pos[None, :] > q_pos[:, None], float('-inf'))
        if attention_mask is not None:
            if attention_mask.dtype == torch.bool:
                keep = attention_mask
                while keep.dim() < 4:
                    keep = keep.unsqueeze(1)
                logits = logits.masked_fill(~keep, float('-inf'))
            else:
                logits = logits + attention_mask
        weights = torch.softmax(logits, dim=-1)
        out = self._merge_heads(torch.matmul(weights.to(vf.dtype), vf))
        out = self.o_proj(out) * torch.sigmoid(g)
        payload = None
        if output_attentions:
            first = int(q_start.reshape(-1)[0]) if isinstance(q_start, torch.Tensor) else q_start
            reach = max(L - 1, S - 1 - first, 1) + 1
            payload = {'prior': self.relative_prior(reach, device=dev)}
        return AttentionOutput(output=out, attention_weights=weights if output_attentions else None,
                               past_key_value=cache, payload=payload)


__all__ = ['ChordAttention', 'LogPositions', 'ggd_bias', 'StaticKVLayerCache']
