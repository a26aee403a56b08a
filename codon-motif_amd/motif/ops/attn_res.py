'''Intra-block attention-residual read (adjacent to the hot path; PyTorch-ROCm).

Softmax over the block's sources of <query, RMSNorm(source)>, then the
weighted sum of the raw sources; same math as the reference's eager read
(motif/ops/attn_res.py:588-593) and `apply_block_attn_res` (:596-622).
'''
import torch


def attn_res_read(sources, query, norm):
    V = torch.stack(list(sources), dim=0)
    K = norm(V)
    logits = torch.einsum('d,nbtd->nbt', query.to(K.dtype), K)
    alpha = logits.softmax(dim=0)
    return torch.einsum('nbt,nbtd->btd', alpha, V)


def apply_block_attn_res(cache, query, norm):
    sources = cache.aligned_values()
    if len(sources) == 1:
        return sources[0]
    return attn_res_read(sources, query, norm)
