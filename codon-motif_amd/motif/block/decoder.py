'''Decoder / DecoderBlock with the reference interface (motif/block/decoder.py:44-222):
pre-norm attention in parallel with a pre-norm SwiGLU MLP, and the intra-block
attention-residual read in front of every decoder.'''
import contextlib
from dataclasses import dataclass
from typing import List, Literal, Optional, Union

import torch
import torch.nn as nn

from motif.block.attention import AttentionOutput, ChordAttention, GatedDeltaAttention
from motif.block.mlp import SwiGLU
from motif.model.cache import DecoderBlockCache, GatedDeltaAttentionLayerCache, KVLayerCache
from motif.model.config import MotifChordConfig
from motif.ops import RMSNorm
from motif.ops.attn_res import apply_block_attn_res, attn_res_read_norms
from motif.ops.autograd_path import wants_grad
from motif.ops.epilogue import residual_fold, swiglu, usable
from motif.ops.linear_rows import linear_rows_dual, linear_rows_pair, rows_eligible, sum_weights


@dataclass
class DecoderBlockOutput:
    hidden_states: torch.Tensor
    cache: DecoderBlockCache

    @property
    def blocks(self) -> List[torch.Tensor]:
        return self.cache.attn_res.blocks


class Decoder(nn.Module):
    def __init__(self, attn_type: Literal['gdn', 'chord'], config: MotifChordConfig):
        super().__init__()
        self.attn_type = attn_type.lower()
        self.attn_norm = RMSNorm(config.model_dim)
        if self.attn_type == 'chord':
            self.attn = ChordAttention(hidden_size=config.model_dim, num_heads=config.num_heads,
                                       num_kv_heads=config.num_kv_heads)
        else:
            self.attn = GatedDeltaAttention(hidden_size=config.model_dim, num_heads=config.num_heads,
                                            head_k_dim=config.head_k_dim, expand_v=2.0, chunk_size=64,
                                            bias=False)
        self.mlp_norm = RMSNorm(config.model_dim)
        self.mlp = SwiGLU(in_features=config.model_dim)

    @property
    def cache_type(self):
        return KVLayerCache if self.attn_type == 'chord' else GatedDeltaAttentionLayerCache


def _split_step(decoder, x, m, layer_cache, mask, position, prev):
    '''One decoder's decode step as three launches around the attention core: the
    attention input projection with the MLP gate/up projection (one launch), the core,
    and o_proj with the MLP down projection and the residual fold (one launch).  The
    result equals the layer-then-MLP sequence bit for bit.  Returns (f_h, partial), or
    None (before anything ran) when the step does not qualify.'''
    mlp = decoder.mlp
    if not (mlp._fused(m) and rows_eligible(x, mlp.gate_up_proj.weight)):
        return None
    if isinstance(decoder.attn, ChordAttention):
        split = decoder.attn.decode_split(x, layer_cache, embedding_start=position, attention_mask=mask)
    elif isinstance(decoder.attn, GatedDeltaAttention):
        split = decoder.attn.decode_split(x, layer_cache)
    else:
        split = None
    if split is None:
        return None
    w_in, core, w_out = split
    w_gu, w_down = mlp.gate_up_proj.weight, mlp.down_proj.weight
    if (not rows_eligible(x, w_in) or x.shape[-1] % 64 or w_out.shape[1] % 64 or w_down.shape[1] % 64
            or w_out.shape[0] != w_down.shape[0] or w_out.dtype != torch.bfloat16 or w_down.dtype != torch.bfloat16
            or (prev is not None and (prev.dtype != x.dtype or prev.stride(-1) != 1))):
        return None
    proj, act = linear_rows_pair(x, w_in, m, w_gu)
    o, g_pre = core(proj)
    return linear_rows_dual(o, w_out, act, w_down, gate=g_pre, aux2=prev)


def _prefill_step(decoder, x, m, layer_cache):
    '''A GatedDelta decoder's prefill with its two output projections as one library GEMM:
    the layer writes its o_proj input y and the MLP its SwiGLU output s side by side
    into one [B, L, H dv + I] buffer, and f_h = [y | s] [W_o | W_down]^T (no reference
    counterpart as one op: motif/block/decoder.py:205-210 computes o_proj(y) and
    down_proj(s) as two GEMMs, rounds each to the activation dtype and adds them; here
    the sum is accumulated in fp32 and rounded once).  Returns f_h (the caller registers
    it with the block's running-sum add put off), or None (before anything ran) when the
    step does not qualify: not a GatedDelta layer, decode-sized input, autograd, biases,
    or inputs the fused prefill kernels do not serve.'''
    attn, mlp = decoder.attn, decoder.mlp
    if (not isinstance(attn, GatedDeltaAttention) or x.dim() != 3 or x.dtype != torch.bfloat16
            or mlp.gate_up_proj.bias is not None or rows_eligible(m, mlp.gate_up_proj.weight)
            or attn.o_proj.out_features != mlp.down_proj.out_features):
        return None
    w = sum_weights(decoder, '_out_sum', (attn.o_proj, mlp.down_proj))
    m2 = _rows(m)
    if w is None or m2 is None:
        return None
    B, L, _ = x.shape
    hv, inner = attn.o_proj.in_features, mlp.down_proj.in_features
    # everything the side branch writes is allocated before the fork (see _Fork)
    buf = torch.empty(B, L, hv + inner, dtype=x.dtype, device=x.device)
    h1 = torch.empty(B * L, 2 * inner, dtype=x.dtype, device=x.device)
    if not usable(buf[..., hv:]):
        return None
    fork = _Fork(x.device)
    if not attn.prefill_core(x, layer_cache, buf[..., :hv]):
        fork.join()  # (a capture may not end with the side stream forked)
        return None
    with fork.side():
        torch.mm(m2, mlp.gate_up_proj.weight.t(), out=h1)
        swiglu(h1.view(B, L, 2 * inner), out=buf[..., hv:])
    fork.join()
    return torch.nn.functional.linear(buf, w)


def _chord_prefill_step(decoder, x, m, layer_cache, mask, position, attn_res):
    '''A Chord decoder's prefill with its output side in one elementwise pass: the layer
    stops before its output gate (o = o_proj(attention), g its pre-activation), the MLP
    runs, and motif.ops.epilogue.residual_fold forms f_h = o * sigmoid(g) + mlp and the
    block's running sum with every add put off since it was last stored -- the
    reference's ops in its order, one rounding each (motif/block/attention/
    chord_attn.py:254, motif/block/decoder.py:205-213).  Returns (f_h, partial, layer
    cache), or None when the call takes another route (having run at most the sum of the
    put-off adds, which partial_block then holds).'''
    attn, mlp = decoder.attn, decoder.mlp
    if (not isinstance(attn, ChordAttention) or x.dim() != 3 or x.dtype != torch.bfloat16 or not x.is_cuda
            or mask is not None
            or attn.o_proj.bias is not None or mlp._fused(m) or wants_grad(x, m, attn, mlp)):
        return None
    chain = attn_res.pending_sum()
    if not chain:
        p = attn_res.partial_block
        chain = [] if p is None else [p]
    if chain and tuple(chain[0].shape) != (*x.shape[:-1], attn.o_proj.out_features):
        return None
    m2 = _rows(m)
    if m2 is None or mlp.gate_up_proj.bias is not None or mlp.down_proj.bias is not None:
        return None
    B, L, _ = x.shape
    inner = mlp.down_proj.in_features
    # everything the side branch writes is allocated before the fork (see _Fork)
    h1 = torch.empty(B * L, 2 * inner, dtype=x.dtype, device=x.device)
    s = torch.empty(B, L, inner, dtype=x.dtype, device=x.device)
    d = torch.empty(B, L, mlp.down_proj.out_features, dtype=x.dtype, device=x.device)
    fork = _Fork(x.device)
    parts = attn.prefill_parts(x, past_key_value=layer_cache, embedding_start=position)
    if parts is None:
        fork.join()
        return None
    merged, g_pre, layer_cache = parts
    with fork.side():
        torch.mm(m2, mlp.gate_up_proj.weight.t(), out=h1)
        swiglu(h1.view(B, L, 2 * inner), out=s)
        torch.mm(s.view(B * L, inner), mlp.down_proj.weight.t(), out=d.view(B * L, -1))
    o = torch.nn.functional.linear(merged, attn.o_proj.weight)
    fork.join()
    f_h, partial = residual_fold(o, d, gate=g_pre, chain=chain)
    return f_h, partial, layer_cache


_SIDE_STREAMS = {}


class _Fork:
    '''The MLP branch of a prefill on a second stream of the device while the attention
    layer runs on the current one (the branches only meet at the output side).

    The fork point is recorded when the _Fork is made, before the layer's kernels are
    enqueued; the MLP's launches are enqueued after them (so the layer's whole-CU
    workgroups are dispatched first and the MLP fills the CUs they leave, e.g. during
    the GatedDelta state scan), and join() makes the current stream wait for them.
    The side branch allocates nothing and touches only tensors that existed before the
    fork (the MLP input, the weights, and outputs allocated before it): a block that
    the current stream frees after the fork could still be in use by its own pending
    kernels, so it must never reach the side branch.  Both streams keep the default
    priority.

    Only while a graph is being captured: launched one by one from the host, the
    forked prefill measured 6.3 ms against 4.3 in sequence (config 3, B = 1, T = 4096);
    replayed from a graph, 3.0 ms against 3.2.  Both forms give the same bits.'''

    def __init__(self, device):
        self.on = torch.device(device).type == 'cuda' and torch.cuda.is_current_stream_capturing()
        if not self.on:
            return
        self.main = torch.cuda.current_stream(device)
        stream = _SIDE_STREAMS.get(device)
        if stream is None:
            stream = _SIDE_STREAMS[device] = torch.cuda.Stream(device=device)
        self.stream = stream
        stream.wait_stream(self.main)

    def side(self):
        return torch.cuda.stream(self.stream) if self.on else contextlib.nullcontext()

    def join(self):
        if self.on:
            self.main.wait_stream(self.stream)


def _rows(t):
    '''[M, K] view of t's rows, or None when there is none.'''
    if t.stride(-1) != 1:
        return None
    try:
        return t.view(-1, t.shape[-1])
    except RuntimeError:
        return None


def _prev(attn_res, like):
    p = attn_res.partial_block
    return p if p is not None and p.shape == like.shape else None


class DecoderBlock(nn.Module):
    def __init__(self, config: MotifChordConfig):
        super().__init__()
        self.features = nn.ModuleList([Decoder(attn_type=t, config=config) for t in config.block])
        self.pseudo_queries = nn.ParameterList([nn.Parameter(torch.zeros(config.model_dim)) for _ in self.features])
        self.attn_res_norms = nn.ModuleList([RMSNorm(config.model_dim) for _ in self.features])

    def _read(self, attn_res, i, decoder):
        '''(attn_norm(h), mlp_norm(h)) for h, the attention-residual read of decoder i.
        ROCm tensors: one kernel (read and both norms, h never stored); the wrapper
        computes the torch formula itself for reads that need gradients or hold more
        sources than the kernel takes.'''
        sources = attn_res.aligned_values()
        an, mn = decoder.attn_norm, decoder.mlp_norm
        x0 = sources[0]
        if (x0.is_cuda and an.weight is not None and mn.weight is not None
                and x0.shape[-1] * x0.element_size() <= 4096 and (x0.shape[-1] * x0.element_size()) % 16 == 0
                and an.eps == mn.eps and x0.dtype in (torch.bfloat16, torch.float32)):
            return attn_res_read_norms(sources, self.pseudo_queries[i], self.attn_res_norms[i], an, mn)
        h = apply_block_attn_res(attn_res, self.pseudo_queries[i], self.attn_res_norms[i])
        return an(h), mn(h)

    def forward(self, hidden_states: torch.Tensor, cache: Optional[DecoderBlockCache] = None,
                mask: Optional[torch.Tensor] = None, position: Union[int, torch.Tensor] = 0,
                cu_seqlens: Optional[torch.Tensor] = None) -> DecoderBlockOutput:
        '''Run every decoder, threading the attention-residual state.

        `cu_seqlens` (packed sequences, B == 1; no reference counterpart) runs
        every layer in its varlen form and uses no layer caches.'''
        if cache is None:
            cache = DecoderBlockCache()
        attn_res = cache.attn_res
        attn_res.init_embedding(hidden_states)
        if cu_seqlens is None:
            if len(cache.attn) == 0:
                if not self.training:
                    cache.ensure_attn([d.cache_type for d in self.features])
            elif len(cache.attn) != len(self.features):
                raise ValueError(f'cache.attn has {len(cache.attn)} entries but the block has '
                                 f'{len(self.features)} layers')
        use_attn_cache = cu_seqlens is None and len(cache.attn) == len(self.features)

        # At prefill (the steps below) each decoder's MLP branch runs on a second stream
        # while its attention layer runs on this one when a graph is being captured
        # (_Fork); other calls run the branches in sequence.  The GatedDelta decoders put the block's running-sum add
        # off; the next Chord decoder (or the first read of partial_block) folds every
        # put-off add into one pass.
        for i, decoder in enumerate(self.features):
            x, m = self._read(attn_res, i, decoder)
            if cu_seqlens is None:
                layer_cache = cache.attn[i] if use_attn_cache else None
                done = None
                if use_attn_cache and decoder.mlp._fused(m):
                    done = _split_step(decoder, x, m, layer_cache, mask, position, _prev(attn_res, m))
                if done is None:
                    f_h = _prefill_step(decoder, x, m, layer_cache)
                    if f_h is not None:
                        attn_res.update_increment(f_h, defer=True)
                        continue
                    tail = _chord_prefill_step(decoder, x, m, layer_cache, mask, position, attn_res)
                    if tail is not None:
                        if use_attn_cache:
                            cache.attn[i] = tail[2]
                        done = tail[:2]
                if done is not None:
                    attn_res.update_increment(*done)
                    continue
            if cu_seqlens is not None:
                attn_out = decoder.attn.forward_varlen(x, cu_seqlens)
            elif isinstance(decoder.attn, ChordAttention):
                attn_out = decoder.attn(hidden_states=x, past_key_value=cache.attn[i] if use_attn_cache else None,
                                        attention_mask=mask, embedding_start=position)
            else:
                attn_out = decoder.attn(hidden_states=x, past_key_value=cache.attn[i] if use_attn_cache else None)
            prev = attn_res.partial_block
            prev = prev if prev is not None and prev.shape == attn_out.output.shape else None
            f_h, partial = decoder.mlp.forward_residual(m, attn_out.output, prev)
            if use_attn_cache:
                cache.attn[i] = attn_out.past_key_value
            attn_res.update_increment(f_h, partial)

        block_repr = attn_res.partial_block
        if block_repr is None:
            block_repr = hidden_states
        return DecoderBlockOutput(hidden_states=block_repr, cache=cache)
