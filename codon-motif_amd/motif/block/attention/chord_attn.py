'''ChordAttention with the reference interface (motif/block/attention/chord_attn.py:59-379).

Same constructor, parameters (theta_alpha / theta_beta / theta_mu frozen /
ssmax_s), GGD helpers, cache handling, log_n table and forward contract.  The
attention itself runs on the HIP Chord kernels (`apply_chord_attention`) for
the inference path; as in the reference, a request for an additive / boolean
attention mask or for the attention weights takes the explicit eager path,
since neither is a kernel feature.  Kernel errors propagate (no silent
fallback).
'''
from typing import Optional, Union

import torch
import torch.nn as nn

from motif.block.attention.base import AttentionOutput, BasicAttention
from motif.model.cache import KVLayerCache, StaticKVLayerCache
from motif.ops import RMSNorm, apply_chord_attention, apply_chord_attention_varlen
from motif.ops import _lib
from motif.ops.epilogue import mul_sigmoid, usable
from motif.ops.linear_rows import cat_weights, linear_rows, project, rows_eligible

_HALF_DTYPES = (torch.float16, torch.bfloat16)
_GGD_EPS = 1e-5
_LOG_TABLE = {}


def _log_n_table(n: int, device, dtype=torch.float32) -> torch.Tensor:
    '''log(1 .. size), size a power of two >= max(n, 8192), cached per (device, dtype).'''
    key = (str(device), str(dtype))
    table = _LOG_TABLE.get(key)
    if table is None or table.numel() < n:
        size = max(n, 8192)
        size = 1 << (size - 1).bit_length()
        table = torch.log(torch.arange(1, size + 1, device=device, dtype=dtype))
        _LOG_TABLE[key] = table
    return table


def _promote(t: torch.Tensor) -> torch.Tensor:
    return t.float() if t.dtype in _HALF_DTYPES else t


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

    @classmethod
    def cache_type(cls) -> type:
        return KVLayerCache

    def _ggd_parameters(self):
        '''(alpha, beta, mu) = (exp(theta_alpha), theta_beta, exp(theta_mu) - exp(-theta_mu)) in fp32.'''
        ta, tb, tm = _promote(self.theta_alpha), _promote(self.theta_beta), _promote(self.theta_mu)
        return torch.exp(ta), tb, torch.exp(tm) - torch.exp(-tm)

    def _compute_ggd_bias(self, q_len: int, kv_len: int, q_start: Union[int, torch.Tensor],
                          device: torch.device, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        '''[num_heads, q_len, kv_len] bias -alpha * (|d - mu| + eps) ** beta, d = key - query position.'''
        alpha, beta, mu = self._ggd_parameters()
        cd = alpha.dtype
        if isinstance(q_start, torch.Tensor):
            start = q_start.to(device=device, dtype=cd).reshape(-1)[0]
        else:
            start = float(q_start)
        q_pos = torch.arange(q_len, device=device, dtype=cd) + start
        k_pos = torch.arange(kv_len, device=device, dtype=cd)
        d = k_pos[None, :] - q_pos[:, None]
        b = torch.abs(d[None] - mu[:, None, None]) + _GGD_EPS
        return (-alpha[:, None, None] * b ** beta[:, None, None]).to(dtype)

    @torch.no_grad()
    def relative_prior(self, max_distance: int, device=None, dtype=torch.float32) -> torch.Tensor:
        alpha, beta, mu = self._ggd_parameters()
        device = device if device is not None else self.theta_alpha.device
        d = torch.arange(-max_distance, max_distance + 1, device=device, dtype=alpha.dtype)
        b = torch.abs(d[None, :] - mu[:, None]) + _GGD_EPS
        return (-alpha[:, None] * b ** beta[:, None]).to(dtype)

    def _log_n(self, q_start, q_len, batch_size, device, section_log_len):
        if section_log_len is not None:
            sl = section_log_len.squeeze(-1) if section_log_len.dim() == 3 else section_log_len
            if sl.shape != (batch_size, q_len):
                raise ValueError(f'section_log_len expects [B, q_len] or [B, q_len, 1], '
                                 f'got {tuple(section_log_len.shape)}')
            return sl.float()
        if isinstance(q_start, torch.Tensor):
            start = q_start.reshape(-1)[0].to(device=device, dtype=torch.float32)
            return torch.log(start + torch.arange(1, q_len + 1, dtype=torch.float32, device=device))
        return _log_n_table(q_start + q_len, device)[q_start:q_start + q_len]

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
        if kv_states is None:
            kv_states = hidden_states
        batch_size, q_len, _ = hidden_states.shape
        kv_len_input = kv_states.shape[1]
        use_cache = isinstance(past_key_value, KVLayerCache)
        q_start = embedding_start
        if use_cache:
            cached = past_key_value.seq_length
            if isinstance(q_start, int) and q_start == 0 and cached > 0:
                q_start = cached
        if kv_states is hidden_states and self._prep_fusable(hidden_states):
            q, k, v, xg = self._fused_inputs(hidden_states, past_key_value if use_cache else None)
        else:
            xq, xk, xv, xg = self._project(hidden_states, kv_states)
            q = self.q_norm(self.reshape_q(xq, q_len, batch_size))
            k = self.k_norm(self.reshape_kv(xk, kv_len_input, batch_size))
            v = self.reshape_kv(xv, kv_len_input, batch_size)
            if use_cache:
                k, v = past_key_value.update(k, v, dim=2)
        current_key_value = past_key_value if use_cache else None
        kv_len = k.shape[2]
        log_n = self._log_n(q_start, q_len, batch_size, hidden_states.device, section_log_len)

        if attention_mask is None and not output_attentions:
            alpha, beta, mu, ssmax = self._ggd_cached()
            start = int(q_start.reshape(-1)[0]) if isinstance(q_start, torch.Tensor) else int(q_start)
            out = apply_chord_attention(
                q, k, v, alpha, beta, mu, ssmax,
                log_n if log_n.dim() == 2 else log_n.expand(batch_size, q_len),
                q_start=start, softmax_scale=self.head_dim ** -0.5, eps=_GGD_EPS)
            out = out.transpose(1, 2).reshape(batch_size, q_len, self.hidden_size)
            return AttentionOutput(output=self._gated_output(out, xg), past_key_value=current_key_value)

        return self._eager(q, k, v, torch.sigmoid(xg), q_start, q_len, kv_len, batch_size, log_n,
                           attention_mask, output_attentions, current_key_value)

    def _ggd_cached(self):
        '''(alpha, beta, mu, ssmax) as contiguous fp32, cached until a parameter changes.'''
        params = (self.theta_alpha, self.theta_beta, self.theta_mu, self.ssmax_s)
        if torch.is_grad_enabled() and any(p.requires_grad for p in params):
            alpha, beta, mu = self._ggd_parameters()
            return tuple(t.contiguous() for t in (alpha, beta, mu, _promote(self.ssmax_s)))
        key = tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in params)
        cached = self.__dict__.get('_ggd_cat')
        if cached is None or cached[0] != key:
            with torch.no_grad():
                alpha, beta, mu = self._ggd_parameters()
                vals = tuple(t.contiguous() for t in (alpha, beta, mu, _promote(self.ssmax_s)))
            cached = (key, vals)
            self.__dict__['_ggd_cat'] = cached
        return cached[1]

    def _prep_fusable(self, x):
        '''Self-attention inputs the fused input kernel (motif_chord_qkv_prep) serves.'''
        if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float32):
            return False
        if (self.head_dim * x.element_size()) % 16 or self.head_dim * x.element_size() > 512:
            return False
        if self.q_norm.weight is None or self.k_norm.weight is None or self.q_norm.eps != self.k_norm.eps:
            return False
        return not (torch.is_grad_enabled() and any(p.requires_grad for p in self.parameters()))

    def _fused_inputs(self, hidden_states, cache):
        '''(q, k, v, g) from one projection GEMM and one kernel for the q / k RMSNorms and
        the placement of k / v: straight into a preallocated cache (StaticKVLayerCache with
        room), else into new tensors that the cache (if any) appends.  k, v are the cache
        views the attention reads; g is the gate pre-activation (G = sigmoid(g)).'''
        B, L, _ = hidden_states.shape
        H, Hkv, D, hs, kd = self.num_heads, self.num_kv_heads, self.head_dim, self.hidden_size, self.kv_dim
        dev, dt = hidden_states.device, hidden_states.dtype
        w, b = cat_weights(self, '_proj_cat', (self.q_proj, self.k_proj, self.v_proj, self.g_proj))
        proj = project(hidden_states, w, b)
        if proj.stride(-1) != 1:
            proj = proj.contiguous()
        static = (isinstance(cache, StaticKVLayerCache) and cache.k is not None and cache.k.dtype == dt
                  and cache.length + L <= cache.capacity)
        if static:
            pos = cache.reserve(L)
            kd_t, vd_t, len_dev = cache.k, cache.v, cache.length_dev
        else:
            pos = 0
            kd_t = torch.empty(B, Hkv, L, D, dtype=dt, device=dev)
            vd_t = torch.empty(B, Hkv, L, D, dtype=dt, device=dev)
            len_dev = None
        q = torch.empty(B, H, L, D, dtype=dt, device=dev)
        qw = self.q_norm.weight.to(dt).contiguous()
        kw = self.k_norm.weight.to(dt).contiguous()
        rc = _lib.lib().motif_chord_qkv_prep(
            proj.data_ptr(), proj.stride(0), proj.stride(1), 0, hs, hs + kd,
            qw.data_ptr(), kw.data_ptr(), float(self.q_norm.eps),
            q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
            kd_t.data_ptr(), kd_t.stride(0), kd_t.stride(1), kd_t.stride(2),
            vd_t.data_ptr(), vd_t.stride(0), vd_t.stride(1), vd_t.stride(2),
            _lib.ptr(len_dev), pos, B, L, H, Hkv, D, _lib.dtype_code(dt), _lib.stream_ptr(dev))
        _lib.check(rc, 'motif_chord_qkv_prep')
        if static:
            k, v = cache.k[:, :, :cache.length], cache.v[:, :, :cache.length]
        elif cache is not None:
            k, v = cache.update(kd_t, vd_t, dim=2)
        else:
            k, v = kd_t, vd_t
        return q, k, v, proj[..., hs + 2 * kd:]

    def _project(self, hidden_states, kv_states):
        '''q, k, v and the gate pre-activation g (G = sigmoid(g)).  Self-attention runs the
        four projections as one GEMM against their concatenated weights (the results are
        column views of it); cross-attention projects k, v from kv_states.'''
        if kv_states is hidden_states:
            w, b = cat_weights(self, '_proj_cat', (self.q_proj, self.k_proj, self.v_proj, self.g_proj))
            proj = project(hidden_states, w, b)
            hs, kd = self.hidden_size, self.kv_dim
            return (proj[..., :hs], proj[..., hs:hs + kd], proj[..., hs + kd:hs + 2 * kd],
                    proj[..., hs + 2 * kd:])
        return (self.q_proj(hidden_states), self.k_proj(kv_states), self.v_proj(kv_states),
                self.g_proj(hidden_states))

    def _gated_output(self, out, g_pre):
        '''o_proj(out) * sigmoid(g_pre); one decode kernel (gate in the epilogue) for
        decode-sized bf16 inputs.'''
        if self.o_proj.bias is None and rows_eligible(out, self.o_proj.weight):
            return linear_rows(out, self.o_proj.weight, 'gate', aux=g_pre)
        o = self.o_proj(out)
        if o.shape == g_pre.shape and usable(o, g_pre):
            return mul_sigmoid(o, g_pre)
        return o * torch.sigmoid(g_pre)

    def forward_varlen(self, hidden_states: torch.Tensor, cu_seqlens: torch.Tensor) -> AttentionOutput:
        '''Packed sequences (B == 1): each sequence attends causally within itself
        with positions (and log_n) restarting at 0.  Returns the output and the
        packed keys / values in the payload.'''
        batch_size, T, _ = hidden_states.shape
        if batch_size != 1:
            raise ValueError('forward_varlen expects packed sequences with B == 1')
        if self._prep_fusable(hidden_states):
            q, k, v, xg = self._fused_inputs(hidden_states, None)
        else:
            xq, xk, xv, xg = self._project(hidden_states, hidden_states)
            q = self.q_norm(self.reshape_q(xq, T, 1))
            k = self.k_norm(self.reshape_kv(xk, T, 1))
            v = self.reshape_kv(xv, T, 1)
        cu = cu_seqlens.detach().to('cpu', torch.int64)
        pos = torch.arange(T) - torch.repeat_interleave(cu[:-1], cu[1:] - cu[:-1])
        log_n = torch.log(pos.to(torch.float32) + 1).to(hidden_states.device)[None]
        alpha, beta, mu = self._ggd_parameters()
        out = apply_chord_attention_varlen(
            q, k, v, alpha.contiguous(), beta.contiguous(), mu.contiguous(),
            _promote(self.ssmax_s).contiguous(), log_n, cu_seqlens,
            softmax_scale=self.head_dim ** -0.5, eps=_GGD_EPS)
        out = out.transpose(1, 2).reshape(1, T, self.hidden_size)
        return AttentionOutput(output=self._gated_output(out, xg), payload={'k': k, 'v': v})

    def _eager(self, q, k, v, G, q_start, q_len, kv_len, batch_size, log_n,
               attention_mask, output_attentions, current_key_value):
        '''Materialised-bias path for masks / attention weights (chord_attn.py:316-379).'''
        if self.num_kv_queries > 1 and k.shape[1] != self.num_heads:
            k = k.repeat_interleave(self.num_kv_queries, dim=1)
            v = v.repeat_interleave(self.num_kv_queries, dim=1)
        scores = (q @ k.transpose(-2, -1)) * (self.head_dim ** -0.5)
        logit_dtype = torch.float32 if scores.dtype in _HALF_DTYPES else scores.dtype
        bias = self._compute_ggd_bias(q_len, kv_len, q_start, scores.device, logit_dtype)
        logits = scores.to(logit_dtype) + bias.unsqueeze(0)
        ln = log_n.view(1, 1, q_len, 1) if log_n.dim() == 1 else log_n.view(batch_size, 1, q_len, 1)
        logits = logits * (_promote(self.ssmax_s).view(1, -1, 1, 1) * ln.to(logit_dtype))
        logits = logits.clamp_min(torch.finfo(logit_dtype).min / 4)
        q_pos = torch.arange(q_len, device=logits.device) + q_start
        k_pos = torch.arange(kv_len, device=logits.device)
        logits = logits.masked_fill(k_pos[None, :] > q_pos[:, None], float('-inf'))
        if attention_mask is not None:
            if attention_mask.dtype == torch.bool:
                keep = attention_mask
                if keep.dim() == 2:
                    keep = keep[:, None, None, :]
                elif keep.dim() == 3:
                    keep = keep[:, None]
                logits = logits.masked_fill(~keep, float('-inf'))
            else:
                logits = logits + attention_mask
        attn = torch.softmax(logits, dim=-1)
        out = (attn.to(v.dtype) @ v).transpose(1, 2).reshape(batch_size, q_len, self.hidden_size)
        out = self.o_proj(out) * G
        payload = None
        if output_attentions:
            start = q_start if isinstance(q_start, int) else int(q_start.reshape(-1)[0])
            payload = {'prior': self.relative_prior(max(q_len - 1, kv_len - 1 - start, 1) + 1,
                                                    device=logits.device)}
        return AttentionOutput(output=out, attention_weights=attn if output_attentions else None,
                               past_key_value=current_key_value, payload=payload)


__all__ = ['ChordAttention', 'StaticKVLayerCache']
