'''Pins for the Chord oracle (CPU, float64).

- pure-Python brute force on tiny inputs (scalar loops, explicit softmax);
- reduction to scaled_dot_product_attention when the GGD bias is constant
  (alpha = 0, or beta = 0 which makes it -alpha for every pair) and the logit
  scale ssmax * log_n is 1;
- log_n = 0 gives uniform weights: the prefix mean of the visible values;
- GQA equals MHA with each kv head repeated over its query group;
- the decode row equals the last prefill row;
- the bias formula at a few hand-computed points.
'''
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import chord

D64 = torch.float64


def _inp(B=2, H=4, Hkv=2, L=6, S=6, D=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, L, D, generator=g, dtype=D64)
    k = torch.randn(B, Hkv, S, D, generator=g, dtype=D64)
    v = torch.randn(B, Hkv, S, D, generator=g, dtype=D64)
    alpha = torch.rand(H, generator=g, dtype=D64)
    beta = torch.randn(H, generator=g, dtype=D64) * 0.3
    mu = torch.randn(H, generator=g, dtype=D64)
    ssmax = torch.rand(H, generator=g, dtype=D64) + 0.5
    log_n = torch.rand(B, L, generator=g, dtype=D64) * 2
    return q, k, v, alpha, beta, mu, ssmax, log_n


@pytest.mark.parametrize('q_start,L,S', [(0, 6, 6), (3, 4, 7), (5, 1, 6)])
def test_against_bruteforce(q_start, L, S):
    q, k, v, alpha, beta, mu, ssmax, log_n = _inp(L=L, S=S)
    out = chord.chord_attention(q, k, v, alpha, beta, mu, ssmax, log_n, q_start, 8 ** -0.5)
    ref = chord.chord_attention_bruteforce(q, k, v, alpha, beta, mu, ssmax, log_n, q_start, 8 ** -0.5)
    assert torch.allclose(out, ref, atol=1e-12)


@pytest.mark.parametrize('which', ['alpha0', 'beta0'])
def test_constant_bias_reduces_to_sdpa(which):
    q, k, v, alpha, beta, mu, ssmax, _ = _inp(Hkv=4, L=9, S=9)
    if which == 'alpha0':
        alpha = torch.zeros_like(alpha)
    else:
        beta = torch.zeros_like(beta)
    ones = torch.ones(2, 9, dtype=D64)
    out = chord.chord_attention(q, k, v, alpha, beta, mu, torch.ones_like(ssmax), ones, 0, 0.37)
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=0.37)
    assert torch.allclose(out, ref, atol=1e-12)


def test_log_n_zero_gives_prefix_mean():
    q, k, v, alpha, beta, mu, ssmax, _ = _inp(Hkv=4, L=7, S=7)
    out = chord.chord_attention(q, k, v, alpha, beta, mu, ssmax, torch.zeros(2, 7, dtype=D64), 0)
    prefix = v.cumsum(2) / torch.arange(1, 8, dtype=D64)[None, None, :, None]
    assert torch.allclose(out, prefix, atol=1e-12)


def test_gqa_equals_repeated_mha():
    q, k, v, alpha, beta, mu, ssmax, log_n = _inp(H=6, Hkv=2, L=5, S=5)
    out = chord.chord_attention(q, k, v, alpha, beta, mu, ssmax, log_n, 0)
    kr, vr = k.repeat_interleave(3, 1), v.repeat_interleave(3, 1)
    out2 = chord.chord_attention(q, kr, vr, alpha, beta, mu, ssmax, log_n, 0)
    assert torch.allclose(out, out2, atol=1e-14)
    # head h reads kv head h // 3: perturbing kv head 1 leaves heads 0..2 unchanged
    # (a per-key perturbation: a constant shift of every key would cancel in the softmax)
    k2 = k.clone()
    k2[:, 1] += torch.randn(k2[:, 1].shape, dtype=D64)
    out3 = chord.chord_attention(q, k2, v, alpha, beta, mu, ssmax, log_n, 0)
    assert torch.allclose(out3[:, :3], out[:, :3], atol=1e-14)
    assert not torch.allclose(out3[:, 3:], out[:, 3:])


def test_decode_row_equals_last_prefill_row():
    q, k, v, alpha, beta, mu, ssmax, log_n = _inp(L=8, S=8)
    full = chord.chord_attention(q, k, v, alpha, beta, mu, ssmax, log_n, 0)
    last = chord.chord_attention(q[:, :, -1:], k, v, alpha, beta, mu, ssmax, log_n[:, -1:], None)
    assert torch.allclose(full[:, :, -1:], last, atol=1e-13)


def test_bias_formula_points():
    alpha = torch.tensor([2.0], dtype=D64)
    beta = torch.tensor([0.5], dtype=D64)
    mu = torch.tensor([1.0], dtype=D64)
    b = chord.ggd_bias(alpha, beta, mu, 3, 4, q_start=1, eps=1e-5)
    # query 0 sits at position 1; key 3 -> d = 2, |d - mu| = 1
    assert b[0, 0, 3].item() == pytest.approx(-2.0 * math.sqrt(1.0 + 1e-5), rel=1e-14)
    # query 2 (position 3), key 0 -> d = -3, |d - mu| = 4
    assert b[0, 2, 0].item() == pytest.approx(-2.0 * math.sqrt(4.0 + 1e-5), rel=1e-14)


def test_log_n_table_matches_reference_indexing():
    t = chord.log_n_table(5, 3)
    assert torch.allclose(t, torch.log(torch.tensor([6.0, 7.0, 8.0], dtype=D64)))


def test_varlen_equals_separate_runs():
    H, Hkv, D = 4, 2, 8
    lens = [3, 0, 5]
    T = sum(lens)
    q, k, v, alpha, beta, mu, ssmax, _ = _inp(B=1, H=H, Hkv=Hkv, L=T, S=T, D=D)
    cu = torch.tensor([0, 3, 3, 8])
    out = chord.chord_attention_varlen(q, k, v, alpha, beta, mu, ssmax, cu)
    s = 0
    for n in lens:
        if n:
            ref = chord.chord_attention(q[:, :, s:s + n], k[:, :, s:s + n], v[:, :, s:s + n], alpha, beta,
                                        mu, ssmax, chord.log_n_table(0, n)[None], 0)
            assert torch.allclose(out[:, :, s:s + n], ref, atol=1e-14)
        s += n


def test_prefill_flops_config2():
    assert chord.chord_prefill_flops(2, 12, 64, 2048) == pytest.approx(1.289e10, rel=1e-3)
