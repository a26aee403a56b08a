'''CPU restatement of the decoder block and MotifChordModel forward.  Test infrastructure only.

Follows motif/block/decoder.py:139-222 (attention-residual read in front of
each decoder, pre-norm attention in parallel with the pre-norm SwiGLU MLP,
block output = sum of the decoder increments), motif/ops/attn_res.py:588-593
(eager read), motif/block/mlp.py:42-63 with motif/ops/swiglu.py:252-253 and
motif/model/motif.py:545-630 (embed -> blocks -> norm -> tied lm_head).
Parameters are a flat dict named like the reference state_dict.
'''
import torch
import torch.nn.functional as F

from oracle.chord import chord_layer
from oracle.gdn import gdn_layer, rms_norm


def attn_res_read(sources, query, norm_weight, eps=1e-6):
    '''softmax over sources of <query, RMSNorm(source)>, weighted sum of the raw sources.'''
    if len(sources) == 1:
        return sources[0]
    V = torch.stack(sources, 0)
    K = rms_norm(V, norm_weight, eps)
    alpha = torch.einsum('d,nbtd->nbt', query.to(K.dtype), K).softmax(0)
    return torch.einsum('nbt,nbtd->btd', alpha, V)


def swiglu_mlp(x, p, prefix):
    y = x @ p[prefix + 'gate_up_proj.weight'].t()
    a, gate = y.chunk(2, dim=-1)
    return (a * F.silu(gate)) @ p[prefix + 'down_proj.weight'].t()


class OracleModel:
    '''Stateful oracle of MotifChordModel (one instance per sequence batch).'''

    def __init__(self, params, cfg, dtype=torch.float64):
        self.p = {k: v.to(dtype) for k, v in params.items()}
        self.cfg = cfg
        self.dtype = dtype
        self.D = cfg['model_dim']
        self.H = cfg['num_heads']
        self.Hkv = cfg['num_kv_heads'] or self.H
        self.dk = cfg['head_k_dim'] or self.D // self.H
        self.dv = 2 * self.dk
        self.reset()

    def reset(self):
        n = len(self.cfg['block']) * self.cfg['block_n']
        self.state = [None] * n
        self.conv = [None] * n
        self.kc = [None] * n
        self.vc = [None] * n
        self.pos = 0

    def _layer_params(self, prefix):
        return {k[len(prefix):]: v for k, v in self.p.items() if k.startswith(prefix)}

    def forward(self, ids, cu_seqlens=None):
        '''Logits [B, T, vocab]; continues from the state of previous calls.'''
        p = self.p
        x = p['embed.weight'][ids]
        li_global = 0
        for bi in range(self.cfg['block_n']):
            hist = [x]
            partial = None
            for li, kind in enumerate(self.cfg['block']):
                pre = f'blocks.{bi}.features.{li}.'
                h = attn_res_read(hist, p[f'blocks.{bi}.pseudo_queries.{li}'],
                                  p[f'blocks.{bi}.attn_res_norms.{li}.weight'])
                xin = rms_norm(h, p[pre + 'attn_norm.weight'])
                lp = self._layer_params(pre + 'attn.')
                if kind == 'chord':
                    out, k_all, v_all = chord_layer(xin, lp, self.H, self.Hkv, self.kc[li_global],
                                                    self.vc[li_global], 0, cu_seqlens=cu_seqlens)
                    self.kc[li_global], self.vc[li_global] = k_all, v_all
                else:
                    out, S, conv = gdn_layer(xin, lp, self.H, self.dk, self.dv, self.state[li_global],
                                             self.conv[li_global], cu_seqlens=cu_seqlens)
                    self.state[li_global], self.conv[li_global] = S, conv
                f_h = out + swiglu_mlp(rms_norm(h, p[pre + 'mlp_norm.weight']), p, pre + 'mlp.')
                hist.append(f_h)
                partial = f_h if partial is None else partial + f_h
                li_global += 1
            x = partial
        x = rms_norm(x, p['norm.weight'])
        self.pos += ids.shape[1]
        return x @ p['lm_head.weight'].t()
