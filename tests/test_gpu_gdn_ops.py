'''GPU parity of the GDN ops (HIP kernels through the C ABI) against the CPU oracle.

Tolerances (from the measurement contract): fp32 inputs within 1e-4; bf16
inputs within max-abs 2e-2 / mean-rel 5e-3 of the fp64 oracle; final
recurrent state within relative error 1e-2 (bf16) or 1e-4 (fp32).
'''
import pytest
import torch

from oracle import gdn as ogdn
from support import assert_bf16_close, assert_fp32_close, assert_state_close, gdn_inputs

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _ops():
    import motif.ops as ops
    assert ops.HAS_TRITON, 'HIP library not loaded on a GPU box'
    return ops


def _oracle_rec(q, k, v, b, g, S=None):
    return ogdn.recurrent(*(t.double() for t in (q, k, v, b, g)), None if S is None else S.double())


def _oracle_chunk(q, k, v, b, g, S=None, C=64):
    return ogdn.chunked(*(t.double() for t in (q, k, v, b, g)), None if S is None else S.double(), C)


@pytest.mark.parametrize('dk,dv', [(64, 128), (64, 64), (32, 64), (128, 128)])
def test_recurrent_fp32(dk, dv):
    ops = _ops()
    q, k, v, b, g = gdn_inputs(2, 3, 9, dk, dv, seed=1)
    S0 = torch.randn(2, 3, dk, dv, generator=torch.Generator().manual_seed(5)) * 0.1
    o, S = ops.recurrent_gated_delta_rule(*(t.to(DEV) for t in (q, k, v, b, g)), S0.to(DEV))
    ro, rS = _oracle_rec(q, k, v, b, g, S0)
    assert_fp32_close(o, ro, 1e-4, 'o')
    assert_fp32_close(S, rS, 1e-4, 'S')


def test_recurrent_bf16_decode_shape():
    '''Config-4 GDN decode shape: one token, B=64, H=12, dk=64, dv=128, fp32 state.'''
    ops = _ops()
    q, k, v, b, g = gdn_inputs(64, 12, 1, 64, 128, seed=2, dtype=torch.bfloat16)
    S0 = torch.randn(64, 12, 64, 128, generator=torch.Generator().manual_seed(3)) * 0.05
    o, S = ops.recurrent_gated_delta_rule(*(t.to(DEV) for t in (q, k, v, b, g)), S0.to(DEV))
    ro, rS = _oracle_rec(q, k, v, b, g, S0)
    assert o.dtype == torch.bfloat16
    assert_bf16_close(o, ro, what='o')
    assert_state_close(S, rS, 1e-4, 'S')


def test_recurrent_noncontiguous_layer_layout():
    '''q/k/v as the layer produces them: [B, L, H, D] memory viewed as [B, H, L, D].'''
    ops = _ops()
    B, L, H, dk, dv = 2, 5, 4, 64, 128
    gg = torch.Generator().manual_seed(7)
    q = torch.nn.functional.normalize(torch.randn(B, L, H, dk, generator=gg), dim=-1).transpose(1, 2)
    k = torch.nn.functional.normalize(torch.randn(B, L, H, dk, generator=gg), dim=-1).transpose(1, 2)
    v = torch.randn(B, L, H, dv, generator=gg).transpose(1, 2)
    b = torch.sigmoid(torch.randn(B, L, H, generator=gg)).transpose(1, 2)
    g = torch.nn.functional.logsigmoid(torch.randn(B, L, H, generator=gg)).transpose(1, 2)
    o, S = ops.recurrent_gated_delta_rule(*(t.to(DEV) for t in (q, k, v, b, g)))
    ro, rS = _oracle_rec(q, k, v, b, g)
    assert_fp32_close(o, ro, 1e-4, 'o')
    assert_fp32_close(S, rS, 1e-4, 'S')


@pytest.mark.parametrize('T', [256, 100, 1, 64, 130])
def test_chunk_fp32_config1(T):
    '''Config 1: B=1, H=4, dk=dv=64, chunk 64, fp32 (plus ragged lengths).'''
    ops = _ops()
    q, k, v, b, g = gdn_inputs(1, 4, T, 64, 64, seed=0)
    o, S = ops.chunk_gated_delta_rule(*(t.to(DEV) for t in (q, k, v, b, g)), None, 64)
    ro, rS = _oracle_chunk(q, k, v, b, g, None, 64)
    assert_fp32_close(o, ro, 1e-4, 'o')
    assert_fp32_close(S, rS, 1e-4, 'S')


@pytest.mark.parametrize('C', [16, 32, 64])
@pytest.mark.parametrize('dk,dv', [(64, 128), (128, 256), (32, 64)])
def test_chunk_fp32_chunks_and_dims(C, dk, dv):
    ops = _ops()
    q, k, v, b, g = gdn_inputs(2, 2, 150, dk, dv, seed=C + dk)
    S0 = torch.randn(2, 2, dk, dv, generator=torch.Generator().manual_seed(9)) * 0.1
    o, S = ops.chunk_gated_delta_rule(*(t.to(DEV) for t in (q, k, v, b, g)), S0.to(DEV), C)
    ro, rS = _oracle_rec(q, k, v, b, g, S0)
    assert_fp32_close(o, ro, 1e-4, 'o')
    assert_fp32_close(S, rS, 1e-4, 'S')


def test_chunk_bf16_layer_shape():
    '''bf16 inputs at the model's GDN shape (H=12, dk=64, dv=128), T=512.'''
    ops = _ops()
    q, k, v, b, g = gdn_inputs(1, 12, 512, 64, 128, seed=4, dtype=torch.bfloat16)
    o, S = ops.chunk_gated_delta_rule(*(t.to(DEV) for t in (q, k, v, b, g)))
    ro, rS = _oracle_chunk(q, k, v, b, g)
    assert o.dtype == torch.bfloat16
    assert_bf16_close(o, ro, what='o')
    assert_state_close(S, rS, 1e-2, 'S')


@pytest.mark.parametrize('B,H,T,init', [(2, 3, 1100, False), (1, 2, 1024, True), (1, 2, 4096, True)])
def test_chunk_bf16_long_sequences(B, H, T, init):
    '''Long sequences on the bf16 MFMA path (18 chunks with a partial last one, 16, and
    the model's 64), from zero or a given state, against the fp64 oracle.'''
    ops = _ops()
    q, k, v, b, g = gdn_inputs(B, H, T, 64, 128, seed=31 + T, dtype=torch.bfloat16)
    S0 = torch.randn(B, H, 64, 128, generator=torch.Generator().manual_seed(5)) * 0.1 if init else None
    o, S = ops.chunk_gated_delta_rule(*(t.to(DEV) for t in (q, k, v, b, g)), None if S0 is None else S0.to(DEV))
    ro, rS = _oracle_chunk(q, k, v, b, g, S0)
    assert_bf16_close(o, ro, what='o')
    assert_state_close(S, rS, 1e-2, 'S')


def test_chunk_bf16_batch_equals_packed():
    '''A fixed-length batch row and the same sequence packed (cu_seqlens) give the same
    result on the bf16 MFMA path (the scan groups differ: batch rows vs sequences).'''
    ops = _ops()
    T = 2100
    q, k, v, b, g = (t.to(DEV) for t in gdn_inputs(1, 4, T, 64, 128, seed=41, dtype=torch.bfloat16))
    o2, S2 = ops.chunk_gated_delta_rule(q, k, v, b, g)
    cu = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    o1, S1 = ops.chunk_gated_delta_rule_varlen(q, k, v, b, g, cu)
    assert torch.equal(o2, o1)
    assert torch.equal(S2, S1)


def _gated_inputs(B, H, T, dk, dv, seed):
    q, k, v, b, g = gdn_inputs(B, H, T, dk, dv, seed=seed, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(seed + 100)
    gate = torch.randn(B, T, H * dv, generator=gen).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(dv, generator=gen)).to(torch.bfloat16)
    return q, k, v, b, g, gate, w


@pytest.mark.parametrize('T', [512, 130, 1])
def test_chunk_gated_norm_fused(T):
    '''The chunk rule with the output GatedRMSNorm fused into its output pass equals
    the two separate launches (chunk, then gated_rms_norm_heads) to one bf16 rounding,
    and the fp64 oracle (chunk, o rounded to bf16, eager GatedRMSNorm) within the bf16 bar.'''
    ops = _ops()
    from motif.ops.epilogue import gated_rms_norm_heads
    from oracle.gdn import gated_rms_norm
    B, H, dk, dv = 2, 12, 64, 128
    q, k, v, b, g, gate, w = _gated_inputs(B, H, T, dk, dv, seed=21)
    dq, dk_, dv_, db, dg, dgate, dw = (t.to(DEV) for t in (q, k, v, b, g, gate, w))
    y, S = ops.chunk_gated_delta_rule_gated_norm(dq, dk_, dv_, db, dg, dgate, dw, 1e-6)
    o2, S2 = ops.chunk_gated_delta_rule(dq, dk_, dv_, db, dg)
    y2 = gated_rms_norm_heads(o2, dgate, dw, 1e-6)
    assert y.shape == (B, T, H * dv) and y.dtype == torch.bfloat16
    assert torch.equal(S, S2)
    d = (y.float() - y2.float()).abs()
    assert d.max().item() <= 2 ** -7 * y2.float().abs().max().item(), d.max().item()
    assert (d > 0).float().mean().item() < 0.01
    ro, _ = _oracle_chunk(q, k, v, b, g)
    ob = ro.to(torch.bfloat16).transpose(1, 2)                          # [B, T, H, dv]
    ref = gated_rms_norm(torch.cat([ob, gate.view(B, T, H, dv)], -1), w, dv, 1e-6).reshape(B, T, H * dv)
    # y reaches |y| ~ 10 (unit-RMS rows times silu(gate)): the bf16 bar is applied to
    # y / max(1, max|ref| / 2), where one bf16 step of the largest values is < 1e-2
    scale = max(1.0, ref.abs().max().item() / 2)
    assert_bf16_close(y.double().cpu() / scale, ref.double() / scale, what='y')


def test_chunk_gated_norm_fused_varlen():
    ops = _ops()
    from motif.ops.epilogue import gated_rms_norm_heads
    lens = [70, 1, 200, 64, 33]
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    T = int(cu[-1])
    q, k, v, b, g, gate, w = _gated_inputs(1, 4, T, 64, 128, seed=23)
    args = [t.to(DEV) for t in (q, k, v, b, g)]
    y, S = ops.chunk_gated_delta_rule_gated_norm(*args, gate.to(DEV), w.to(DEV), 1e-6, cu_seqlens=cu.to(DEV))
    o2, S2 = ops.chunk_gated_delta_rule_varlen(*args, cu.to(DEV))
    y2 = gated_rms_norm_heads(o2, gate.to(DEV), w.to(DEV), 1e-6)
    assert torch.equal(S, S2)
    d = (y.float() - y2.float()).abs()
    assert d.max().item() <= 2 ** -7 * y2.float().abs().max().item(), d.max().item()


def test_chunk_gated_norm_declines_fp32():
    '''fp32 inputs are not served by the fused kernel: the op returns None.'''
    ops = _ops()
    q, k, v, b, g = (t.to(DEV) for t in gdn_inputs(1, 2, 80, 64, 128, seed=3))
    gate = torch.randn(1, 80, 256, device=DEV)
    assert ops.chunk_gated_delta_rule_gated_norm(q, k, v, b, g, gate, torch.ones(128, device=DEV), 1e-6) is None


def test_chunk_triton_name_rejects_small_chunk():
    ops = _ops()
    q, k, v, b, g = (t.to(DEV) for t in gdn_inputs(1, 1, 8, 64, 64))
    with pytest.raises(NotImplementedError):
        ops.chunk_gated_delta_rule_triton(q, k, v, b, g, None, 8)


def test_chunk_continuation_equals_full():
    '''Running [0, t) then [t, T) from the carried state equals one run over [0, T).'''
    ops = _ops()
    q, k, v, b, g = (t.to(DEV) for t in gdn_inputs(1, 3, 300, 64, 128, seed=11))
    o_full, S_full = ops.chunk_gated_delta_rule(q, k, v, b, g)
    t = 173
    o1, S1 = ops.chunk_gated_delta_rule(q[:, :, :t], k[:, :, :t], v[:, :, :t], b[:, :, :t], g[:, :, :t])
    o2, S2 = ops.chunk_gated_delta_rule(q[:, :, t:], k[:, :, t:], v[:, :, t:], b[:, :, t:], g[:, :, t:], S1)
    assert_fp32_close(torch.cat([o1, o2], 2), o_full, 1e-4, 'o')
    assert_fp32_close(S2, S_full, 1e-4, 'S')


def test_chunk_varlen_equals_independent_runs():
    ops = _ops()
    lens = [70, 1, 0, 200, 64, 33]
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    T = int(cu[-1])
    q, k, v, b, g = gdn_inputs(1, 4, T, 64, 128, seed=13)
    o, S = ops.chunk_gated_delta_rule_varlen(*(t.to(DEV) for t in (q, k, v, b, g)), cu.to(DEV))
    ro, rS = ogdn.chunked_varlen(*(t.double() for t in (q, k, v, b, g)), cu)
    assert_fp32_close(o, ro, 1e-4, 'o')
    assert_fp32_close(S, rS, 1e-4, 'S')


@pytest.mark.parametrize('cache', [False, True])
@pytest.mark.parametrize('L', [1, 7, 200])
def test_short_conv_silu(cache, L):
    ops = _ops()
    gg = torch.Generator().manual_seed(L)
    B, D, K = 3, 96, 4
    x = torch.randn(B, L, D, generator=gg)
    w = torch.randn(D, 1, K, generator=gg) * 0.5
    tail = torch.randn(B, D, K - 1, generator=gg) if cache else None
    y, nt = ops.short_conv_silu(x.to(DEV), w.to(DEV), None if tail is None else tail.to(DEV))
    ry, rt = ogdn.short_conv_silu(x.double(), w.double(), None if tail is None else tail.double())
    assert_fp32_close(y, ry, 1e-5, 'y')
    assert_fp32_close(nt, rt, 0.0, 'tail')


def test_short_conv_silu_inplace_tail_bf16():
    ops = _ops()
    gg = torch.Generator().manual_seed(3)
    B, D, K = 4, 1536, 4
    x = torch.randn(B, 1, D, generator=gg).to(torch.bfloat16)
    w = (torch.randn(D, 1, K, generator=gg) * 0.5).to(torch.bfloat16)
    tail = torch.randn(B, D, K - 1, generator=gg).to(torch.bfloat16)
    ry, rt = ogdn.short_conv_silu(x.double(), w.double(), tail.double())
    tdev = tail.to(DEV)
    y, nt = ops.short_conv_silu(x.to(DEV), w.to(DEV), tdev, new_cache=tdev)
    assert nt.data_ptr() == tdev.data_ptr()
    assert_bf16_close(y, ry, what='y')
    assert torch.equal(nt.cpu().double(), rt)


def test_short_conv_silu_varlen():
    ops = _ops()
    lens = [5, 0, 130, 2]
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    gg = torch.Generator().manual_seed(21)
    D, K = 64, 4
    x = torch.randn(1, int(cu[-1]), D, generator=gg)
    w = torch.randn(D, 1, K, generator=gg)
    y, tails = ops.short_conv_silu_varlen(x.to(DEV), w.to(DEV), cu.to(DEV))
    ry, rt = ogdn.short_conv_silu_varlen(x.double(), w.double(), cu)
    assert_fp32_close(y, ry, 1e-5, 'y')
    assert_fp32_close(tails, rt, 0.0, 'tails')


@pytest.mark.parametrize('hd,D', [(64, 768), (32, 96), (16, 48)])
@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_short_conv_silu_l2norm(hd, D, dtype):
    '''conv + SiLU, then every hd channels L2-normalised (F.normalize) and scaled.'''
    ops = _ops()
    gg = torch.Generator().manual_seed(D + hd)
    B, L, K, scale = 2, 37, 4, hd ** -0.5
    x = torch.randn(B, L, D, generator=gg).to(dtype)
    w = (torch.randn(D, 1, K, generator=gg) * 0.5).to(dtype)
    tail = torch.randn(B, D, K - 1, generator=gg).to(dtype)
    y, nt = ops.short_conv_silu(x.to(DEV), w.to(DEV), tail.to(DEV), head_dim=hd, scale=scale)
    ry, rt = ogdn.short_conv_silu(x.double(), w.double(), tail.double())
    ry = torch.nn.functional.normalize(ry.view(B, L, D // hd, hd), dim=-1).view(B, L, D) * scale
    if dtype == torch.float32:
        assert_fp32_close(y, ry, 1e-5, 'y')
    else:
        assert_bf16_close(y, ry, what='y')
    assert torch.equal(nt.cpu().double(), rt)


def test_short_conv_silu_l2norm_varlen():
    ops = _ops()
    lens = [5, 0, 130, 2]
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    gg = torch.Generator().manual_seed(22)
    D, K = 128, 4
    x = torch.randn(1, int(cu[-1]), D, generator=gg)
    w = torch.randn(D, 1, K, generator=gg)
    y, tails = ops.short_conv_silu_varlen(x.to(DEV), w.to(DEV), cu.to(DEV), head_dim=64, scale=0.125)
    ry, rt = ogdn.short_conv_silu_varlen(x.double(), w.double(), cu)
    ry = torch.nn.functional.normalize(ry.view(1, -1, 2, 64), dim=-1).view(1, -1, D) * 0.125
    assert_fp32_close(y, ry, 1e-5, 'y')
    assert_fp32_close(tails, rt, 0.0, 'tails')


@pytest.mark.parametrize('cache', [False, True])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_short_conv_silu_multi_equals_separate(cache, dtype):
    '''The GDN q / k / v front ends in one launch give the same bits as three calls.'''
    ops = _ops()
    gen = torch.Generator().manual_seed(31)
    B, L, K = 2, 77, 4
    Ds, hds, scales = (768, 768, 1536), (64, 64, None), (64 ** -0.5, 1.0, 1.0)
    proj = torch.randn(B, L, sum(Ds) + 40, generator=gen).to(dtype).to(DEV)   # q | k | v | rest
    offs = (0, 768, 1536)
    xs = [proj[..., o:o + D] for o, D in zip(offs, Ds)]
    ws = [(torch.randn(D, 1, K, generator=gen) * 0.3).to(dtype).to(DEV) for D in Ds]
    cs = [(torch.randn(B, D, K - 1, generator=gen) * 0.5).to(dtype).to(DEV) if cache else None for D in Ds]
    outs = ops.short_conv_silu_multi(xs, ws, cs, hds, scales)
    assert outs is not None
    for i in range(3):
        y, t = ops.short_conv_silu(xs[i], ws[i], cs[i], head_dim=hds[i], scale=scales[i])
        assert torch.equal(outs[i][0], y), i
        assert torch.equal(outs[i][1], t), i


def test_short_conv_silu_multi_varlen():
    ops = _ops()
    gen = torch.Generator().manual_seed(33)
    lens = [70, 1, 200, 3]
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    T, K = int(cu[-1]), 4
    Ds, hds, scales = (128, 128, 256), (64, 64, None), (0.125, 1.0, 1.0)
    xs = [torch.randn(1, T, D, generator=gen).to(torch.bfloat16).to(DEV) for D in Ds]
    ws = [(torch.randn(D, 1, K, generator=gen) * 0.3).to(torch.bfloat16).to(DEV) for D in Ds]
    outs = ops.short_conv_silu_multi(xs, ws, [None] * 3, hds, scales, cu.to(DEV))
    assert outs is not None
    for i in range(3):
        y, t = ops.short_conv_silu_varlen(xs[i], ws[i], cu.to(DEV), head_dim=hds[i], scale=scales[i])
        assert torch.equal(outs[i][0], y), i
        assert torch.equal(outs[i][1], t), i

