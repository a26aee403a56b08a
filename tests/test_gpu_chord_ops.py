'''GPU parity of apply_chord_attention (HIP kernels) against the fp64 CPU oracle.

bf16 inputs; outputs within max-abs 2e-2 / mean-rel 5e-3 of the oracle.
'''
import pytest
import torch

from oracle import chord as ochord
from support import assert_bf16_close, chord_inputs

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _ops():
    import motif.ops as ops
    assert ops.HAS_TRITON, 'HIP library not loaded on a GPU box'
    return ops


def _run(ops, q, k, v, alpha, beta, mu, ssmax, log_n, q_start=None, scale=None):
    dev = [t.to(DEV) for t in (q, k, v, alpha, beta, mu, ssmax, log_n)]
    return ops.apply_chord_attention(*dev, q_start=q_start, softmax_scale=scale)


def _log_n(B, L, q_start):
    return ochord.log_n_table(q_start, L).float()[None].expand(B, L).contiguous()


def _check_heads(out, q, k, v, alpha, beta, mu, ssmax, log_n, q_start, heads=None, what=''):
    '''Compare selected heads (all by default) with the fp64 oracle.'''
    H = q.shape[1]
    Hkv = k.shape[1]
    heads = range(H) if heads is None else heads
    for h in heads:
        kh = h // (H // Hkv)
        ref = ochord.chord_attention(
            q[:, h:h + 1], k[:, kh:kh + 1], v[:, kh:kh + 1], alpha[h:h + 1], beta[h:h + 1],
            mu[h:h + 1], ssmax[h:h + 1], log_n, q_start)
        assert_bf16_close(out[:, h:h + 1], ref, what=f'{what} head {h}')


@pytest.mark.parametrize('Hkv', [12, 3])
def test_prefill_config2_shape(Hkv):
    '''Config 2 (B=2, H=12, T=2048, D=64, causal), every head checked against fp64.'''
    ops = _ops()
    B, H, L = 2, 12, 2048
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(B, H, Hkv, L, L, seed=0)
    log_n = _log_n(B, L, 0)
    out = _run(ops, q, k, v, alpha, beta, mu, ssmax, log_n, q_start=0)
    assert out.dtype == torch.bfloat16 and out.shape == (B, H, L, 64)
    _check_heads(out.cpu(), q, k, v, alpha, beta, mu, ssmax, log_n, 0, heads=range(H), what='cfg2')


@pytest.mark.parametrize('L', [1, 31, 77, 200])
@pytest.mark.parametrize('Hkv', [4, 2, 1])
def test_prefill_small_ragged(L, Hkv):
    ops = _ops()
    B, H = 2, 4
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(B, H, Hkv, L, L, seed=L + Hkv)
    log_n = _log_n(B, L, 0)
    out = _run(ops, q, k, v, alpha, beta, mu, ssmax, log_n, q_start=0)
    _check_heads(out.cpu(), q, k, v, alpha, beta, mu, ssmax, log_n, 0, what=f'L={L}')


def test_prefill_continuation_with_cache():
    '''Chunked prefill: 100 new queries over a 300-key cache (q_start = 200 default).'''
    ops = _ops()
    B, H, Hkv, L, S = 1, 8, 2, 100, 300
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(B, H, Hkv, L, S, seed=3)
    mu = torch.linspace(-2.0, 3.0, H)
    ssmax = torch.linspace(0.5, 1.5, H)
    log_n = _log_n(B, L, S - L)
    out = _run(ops, q, k, v, alpha, beta, mu, ssmax, log_n)
    _check_heads(out.cpu(), q, k, v, alpha, beta, mu, ssmax, log_n, S - L, what='cont')


@pytest.mark.parametrize('B,S', [(4, 4097), (64, 1000), (2, 9)])
def test_decode_split(B, S):
    '''Decode: one query per sequence over an S-key cache, GQA 12:3 (split-K path).'''
    ops = _ops()
    H, Hkv = 12, 3
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(B, H, Hkv, 1, S, seed=S)
    log_n = _log_n(B, 1, S - 1)
    out = _run(ops, q, k, v, alpha, beta, mu, ssmax, log_n)
    _check_heads(out.cpu(), q, k, v, alpha, beta, mu, ssmax, log_n, S - 1, what=f'decode B={B}')


def test_decode_row_equals_last_prefill_row():
    ops = _ops()
    B, H, Hkv, S = 2, 12, 3, 700
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(B, H, Hkv, S, S, seed=8)
    log_n = _log_n(B, S, 0)
    full = _run(ops, q, k, v, alpha, beta, mu, ssmax, log_n, q_start=0)
    last = _run(ops, q[:, :, -1:], k, v, alpha, beta, mu, ssmax, log_n[:, -1:].contiguous(), q_start=S - 1)
    d = (full[:, :, -1:].float() - last.float()).abs().max().item()
    assert d <= 2e-2, d


def test_varlen_equals_independent_runs():
    ops = _ops()
    lens = [130, 1, 64, 257, 0, 40]
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    T = int(cu[-1])
    H, Hkv = 12, 3
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(1, H, Hkv, T, T, seed=17)
    log_n = torch.cat([ochord.log_n_table(0, n) for n in lens]).float()[None]
    out = ops.apply_chord_attention_varlen(*(t.to(DEV) for t in (q, k, v, alpha, beta, mu, ssmax, log_n)), cu.to(DEV))
    ref = ochord.chord_attention_varlen(q, k, v, alpha, beta, mu, ssmax, cu, softmax_scale=64 ** -0.5)
    assert_bf16_close(out, ref, what='varlen')


def test_validation_errors_match_reference_types():
    ops = _ops()
    q, k, v, alpha, beta, mu, ssmax = (t.to(DEV) for t in chord_inputs(1, 4, 2, 8, 8))
    log_n = _log_n(1, 8, 0).to(DEV)
    with pytest.raises(ValueError):
        ops.apply_chord_attention(q, k, v, alpha, beta, mu, ssmax, log_n, q_start=-1)
    with pytest.raises(ValueError):
        ops.apply_chord_attention(q, k, v, alpha[:3], beta, mu, ssmax, log_n)
    with pytest.raises(ValueError):
        ops.apply_chord_attention(q, k[:, :1].expand(1, 3, 8, 64), v[:, :1].expand(1, 3, 8, 64),
                                  alpha, beta, mu, ssmax, log_n)


@pytest.mark.parametrize('B,H,Hkv,L,S', [(2, 4, 2, 77, 77), (1, 12, 3, 300, 300), (2, 12, 3, 5, 900), (3, 4, 4, 1, 2000)])
def test_fp32_mode(B, H, Hkv, L, S):
    """fp32 inputs run the fp32 vector kernel: within 1e-4 of the fp64 oracle."""
    ops = _ops()
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(B, H, Hkv, L, S, seed=L + S)
    q, k, v = q.float(), k.float(), v.float()
    mu = torch.linspace(-1.0, 1.0, H)
    log_n = _log_n(B, L, S - L)
    out = _run(ops, q, k, v, alpha, beta, mu, ssmax, log_n)
    assert out.dtype == torch.float32
    ref = ochord.chord_attention(q, k, v, alpha, beta, mu, ssmax, log_n, S - L)
    err = (out.double().cpu() - ref).abs().max().item()
    assert err <= 1e-4, err


@pytest.mark.parametrize('L,S', [(200, 200), (77, 300)])
def test_prefill_signed_ssmax_and_mu(L, S):
    '''Negative, zero-crossing and positive ssmax with a nonzero mu (bf16 prefill).'''
    ops = _ops()
    B, H, Hkv = 2, 8, 2
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(B, H, Hkv, L, S, seed=L * 7 + S)
    ssmax = torch.linspace(-1.5, 1.5, H)
    mu = torch.linspace(-3.0, 2.0, H)
    log_n = _log_n(B, L, S - L)
    out = _run(ops, q, k, v, alpha, beta, mu, ssmax, log_n)
    _check_heads(out.cpu(), q, k, v, alpha, beta, mu, ssmax, log_n, S - L, what=f'signed ssmax L={L}')


def test_varlen_long_sequences_split_keys():
    '''Packed sequences longer than one key-range split (1024 keys) of the prefill.'''
    ops = _ops()
    lens = [1200, 5, 1500]
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    T = int(cu[-1])
    H, Hkv = 4, 1
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(1, H, Hkv, T, T, seed=29)
    log_n = torch.cat([ochord.log_n_table(0, n) for n in lens]).float()[None]
    out = ops.apply_chord_attention_varlen(*(t.to(DEV) for t in (q, k, v, alpha, beta, mu, ssmax, log_n)), cu.to(DEV))
    ref = ochord.chord_attention_varlen(q, k, v, alpha, beta, mu, ssmax, cu, softmax_scale=64 ** -0.5)
    assert_bf16_close(out, ref, what='varlen long')


# ---------------------------------------------------------------- fp16 and other head dims
# The reference's apply_chord_attention takes fp16 / bf16 / fp32 and any head dim >= 16
# (motif/ops/chord_attention.py:960-1034).  Here fp16, and D in {16, 32, 128} in every
# dtype, run on the vector kernel (bf16 at D = 64 keeps the MFMA kernels).

@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize('D', [16, 32, 64, 128])
@pytest.mark.parametrize('B,H,Hkv,L,S', [(2, 4, 2, 70, 70), (3, 6, 3, 1, 1500), (1, 4, 1, 9, 300)])
def test_dtypes_and_head_dims(dtype, D, B, H, Hkv, L, S):
    '''Prefill (L = S), decode (L = 1, split keys) and a short block over a longer cache,
    against the fp64 oracle: fp32 within 1e-4; fp16 / bf16 within the bf16 bar.'''
    ops = _ops()
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(B, H, Hkv, L, S, seed=D + L + S, D=D)
    q, k, v = q.float().to(dtype), k.float().to(dtype), v.float().to(dtype)
    mu = torch.linspace(-0.5, 0.5, H)
    log_n = _log_n(B, L, S - L)
    out = _run(ops, q, k, v, alpha, beta, mu, ssmax, log_n)
    assert out.dtype == dtype and out.shape == (B, H, L, D)
    ref = ochord.chord_attention(q.double(), k.double(), v.double(), alpha, beta, mu, ssmax, log_n, S - L)
    if dtype == torch.float32:
        err = (out.double().cpu() - ref).abs().max().item()
        assert err <= 1e-4, err
    else:
        assert_bf16_close(out, ref, what=f'{dtype} D={D}')


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize('D', [20, 48, 80, 112])
@pytest.mark.parametrize('B,H,Hkv,L,S', [(2, 4, 2, 70, 70), (3, 6, 3, 1, 700)])
def test_head_dims_between_kernel_sizes(dtype, D, B, H, Hkv, L, S):
    '''Any head dim from 16 to 128 (the reference takes any D >= 16): sizes between the
    kernels' own run zero-padded to the next one, with the caller's softmax scale.'''
    ops = _ops()
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(B, H, Hkv, L, S, seed=D + L, D=D)
    q, k, v = q.float().to(dtype), k.float().to(dtype), v.float().to(dtype)
    log_n = _log_n(B, L, S - L)
    out = _run(ops, q, k, v, alpha, beta, mu, ssmax, log_n)
    assert out.dtype == dtype and out.shape == (B, H, L, D)
    ref = ochord.chord_attention(q.double(), k.double(), v.double(), alpha, beta, mu, ssmax, log_n, S - L)
    if dtype == torch.float32:
        err = (out.double().cpu() - ref).abs().max().item()
        assert err <= 1e-4, err
    else:
        assert_bf16_close(out, ref, what=f'{dtype} D={D}')


def test_head_dim_above_128_raises_not_implemented():
    ops = _ops()
    q, k, v, alpha, beta, mu, ssmax = (t.to(DEV) for t in chord_inputs(1, 2, 1, 8, 8, D=160))
    with pytest.raises(NotImplementedError):
        ops.apply_chord_attention(q, k, v, alpha, beta, mu, ssmax, _log_n(1, 8, 0).to(DEV))


@pytest.mark.parametrize('dtype,D', [(torch.float32, 64), (torch.float16, 64), (torch.bfloat16, 32),
                                     (torch.float32, 48)])
def test_varlen_other_dtypes_and_head_dims(dtype, D):
    '''Packed sequences outside the packed kernel's bf16 / D = 64 (each sequence on the
    kernels by itself): equal to the separate runs, and within the bar of the oracle.'''
    ops = _ops()
    lens = [40, 1, 0, 97]
    T = sum(lens)
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(1, 4, 2, T, T, seed=D, D=D)
    q, k, v = q.float().to(dtype), k.float().to(dtype), v.float().to(dtype)
    pos = torch.cat([torch.arange(n) for n in lens])
    log_n = torch.log(pos.float() + 1)[None]
    dev = [t.to(DEV) for t in (q, k, v, alpha, beta, mu, ssmax, log_n)]
    out = ops.apply_chord_attention_varlen(*dev, cu.to(DEV))
    for a, b in zip(cu[:-1].tolist(), cu[1:].tolist()):
        if b == a:
            continue
        alone = ops.apply_chord_attention(*[t[:, :, a:b] for t in dev[:3]], *dev[3:7], dev[7][:, a:b].contiguous(),
                                          q_start=0)
        assert torch.equal(out[:, :, a:b], alone), (a, b)
        ref = ochord.chord_attention(q[:, :, a:b].double(), k[:, :, a:b].double(), v[:, :, a:b].double(),
                                     alpha, beta, mu, ssmax, log_n[:, a:b], 0)
        if dtype == torch.float32:
            assert (out[:, :, a:b].double().cpu() - ref).abs().max().item() <= 1e-4
        else:
            assert_bf16_close(out[:, :, a:b], ref, what=f'{dtype} D={D} rows {a}:{b}')


def _merged(q):
    B, H, L, D = q.shape
    return torch.empty((B, L, H, D), dtype=q.dtype, device=q.device).transpose(1, 2)


@pytest.mark.parametrize('dtype,D,L,S', [
    (torch.bfloat16, 64, 2048, 2048),   # the prefill kernel
    (torch.bfloat16, 64, 1, 900),       # a decode-shaped call (split-K kernel)
    (torch.float32, 64, 100, 300),
    (torch.bfloat16, 48, 77, 77),       # a padded head dim (output copied back)
])
@torch.no_grad()
def test_out_destination_equals_new_output(dtype, D, L, S):
    '''`out=` a [B, L, H, D] buffer's transposed view: the same values bit for bit as a
    new [B, H, L, D] output, written in place (the heads come out merged).'''
    ops = _ops()
    B, H, Hkv = 2, 12, 3
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(B, H, Hkv, L, S, seed=21, D=D)
    q, k, v = (t.to(DEV, dtype) for t in (q, k, v))
    params = [t.to(DEV) for t in (alpha, beta, mu, ssmax)]
    log_n = _log_n(B, L, S - L).to(DEV)
    ref = ops.apply_chord_attention(q, k, v, *params, log_n)
    dst = _merged(q)
    got = ops.apply_chord_attention(q, k, v, *params, log_n, out=dst)
    assert got is dst and dst.transpose(1, 2).is_contiguous()
    assert torch.equal(got, ref)


@torch.no_grad()
def test_varlen_out_destination_equals_new_output():
    ops = _ops()
    lens = [130, 1, 64, 0, 257]
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32).to(DEV)
    T, H, Hkv = sum(lens), 12, 3
    q, k, v, alpha, beta, mu, ssmax = chord_inputs(1, H, Hkv, T, T, seed=22)
    args = [t.to(DEV) for t in (q, k, v, alpha, beta, mu, ssmax)]
    log_n = torch.cat([ochord.log_n_table(0, n) for n in lens]).float()[None].to(DEV)
    ref = ops.apply_chord_attention_varlen(*args, log_n, cu)
    dst = _merged(args[0])
    assert ops.apply_chord_attention_varlen(*args, log_n, cu, out=dst) is dst
    assert torch.equal(dst, ref)


def test_out_destination_under_autograd():
    '''With gradients recorded the result is copied into `out`; the gradients through
    `out` equal those of the call without it.'''
    ops = _ops()
    B, H, Hkv, L = 1, 4, 2, 200
    base = chord_inputs(B, H, Hkv, L, L, seed=23)
    log_n = _log_n(B, L, 0).to(DEV)
    grads = []
    for use_out in (False, True):
        q, k, v = (t.to(DEV, torch.bfloat16).requires_grad_() for t in base[:3])
        params = [t.to(DEV) for t in base[3:]]
        dst = _merged(q.detach()) if use_out else None
        o = ops.apply_chord_attention(q, k, v, *params, log_n, q_start=0, out=dst)
        (o.float() * torch.linspace(-1, 1, 64, device=DEV)).sum().backward()
        grads.append([o.detach().clone(), q.grad, k.grad, v.grad])
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_out_destination_rejects_wrong_buffers():
    ops = _ops()
    B, H, Hkv, L = 1, 4, 2, 16
    q, k, v, alpha, beta, mu, ssmax = (t.to(DEV) for t in chord_inputs(B, H, Hkv, L, L, seed=24))
    log_n = _log_n(B, L, 0).to(DEV)
    for bad in (torch.empty((B, H, L, 32), dtype=q.dtype, device=DEV),           # shape
                torch.empty((B, H, L, 64), dtype=torch.float32, device=DEV),     # dtype
                torch.empty((B, H, 64, L), dtype=q.dtype, device=DEV).transpose(2, 3)):  # feature stride
        with torch.no_grad(), pytest.raises(ValueError):
            ops.apply_chord_attention(q, k, v, alpha, beta, mu, ssmax, log_n, q_start=0, out=bad)
