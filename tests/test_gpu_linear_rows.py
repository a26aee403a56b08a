'''GPU parity of the decode projection kernel (motif_linear_rows) and its fused
epilogues against a torch fp32 reference of the same ops, rounded to bf16 at the
points where the reference's separate ops round (GEMM output, sigmoid / SiLU,
product / sum).  The kernel accumulates in fp32 in another order than the
reference GEMM, so the bar is the bf16 one (max-abs 2e-2, mean-rel 5e-3) on O(1)
outputs.'''
import pytest
import torch
import torch.nn.functional as F

from support import assert_bf16_close, gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'
bf = torch.bfloat16


def _r(t):
    return t.to(bf).float()


def _operands(M, N, K, seed):
    g = gen(seed)
    x = torch.randn(M, K, generator=g).to(bf)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(bf)
    return x, w


@pytest.mark.parametrize('M,N,K', [(1, 16, 32), (5, 50, 96), (16, 768, 768), (33, 4632, 768), (64, 768, 2048),
                                   (64, 4096, 768), (100, 200, 1536), (64, 32000, 768)])
def test_linear_rows_plain(M, N, K):
    from motif.ops.linear_rows import linear_rows
    x, w = _operands(M, N, K, M + N + K)
    y = linear_rows(x.to(DEV), w.to(DEV))
    ref = _r(x.float() @ w.float().t())
    assert y.shape == (M, N)
    assert_bf16_close(y, ref, 2e-2, 5e-3, f'plain M={M} N={N} K={K}')


@pytest.mark.parametrize('M,N,K', [(3, 80, 64), (64, 768, 768)])
def test_linear_rows_gate(M, N, K):
    from motif.ops.linear_rows import linear_rows
    x, w = _operands(M, N, K, 1)
    gpre = torch.randn(M, N, generator=gen(2)).to(bf)
    y = linear_rows(x.to(DEV), w.to(DEV), 'gate', aux=gpre.to(DEV))
    ref = _r(_r(x.float() @ w.float().t()) * _r(torch.sigmoid(gpre.float())))
    assert_bf16_close(y, ref, 2e-2, 5e-3, 'gate')


@pytest.mark.parametrize('M,N,K', [(7, 96, 128), (64, 768, 2048)])
def test_linear_rows_resid(M, N, K):
    from motif.ops.linear_rows import linear_rows
    x, w = _operands(M, N, K, 3)
    r = torch.randn(M, N, generator=gen(4)).to(bf)
    p = torch.randn(M, N, generator=gen(5)).to(bf)
    y, y2 = linear_rows(x.to(DEV), w.to(DEV), 'resid', aux=r.to(DEV), aux2=p.to(DEV))
    ref = _r(_r(x.float() @ w.float().t()) + r.float())
    assert_bf16_close(y, ref, 2e-2, 5e-3, 'resid y')
    assert_bf16_close(y2, _r(p.float() + ref), 2e-2, 5e-3, 'resid y2')
    y_only = linear_rows(x.to(DEV), w.to(DEV), 'resid', aux=r.to(DEV))
    assert torch.equal(y_only.cpu(), y.cpu())


@pytest.mark.parametrize('M,N,K', [(2, 64, 32), (64, 4096, 768), (19, 400, 256)])
def test_linear_rows_swiglu(M, N, K):
    from motif.ops.linear_rows import linear_rows
    x, w = _operands(M, N, K, 6)
    h = _r(x.float() @ w.float().t())
    o, gt = h[:, :N // 2], h[:, N // 2:]
    ref = _r(o * _r(F.silu(gt)))
    y = linear_rows(x.to(DEV), w.to(DEV), 'swiglu')
    assert y.shape == (M, N // 2)
    assert_bf16_close(y, ref, 2e-2, 5e-3, 'swiglu')


def test_linear_rows_strided_rows_and_3d():
    '''x as a column slice of a wider tensor (row stride > K) and a [B, 1, K] input.'''
    from motif.ops.linear_rows import linear_rows, rows_eligible
    g = gen(7)
    big = torch.randn(12, 1, 1024, generator=g).to(bf)
    x = big[..., 256:256 + 512]
    w = (torch.randn(300, 512, generator=g) / 512 ** 0.5).to(bf)
    xd, wd = x.to(DEV), w.to(DEV)
    assert rows_eligible(xd, wd)
    y = linear_rows(xd, wd)
    assert y.shape == (12, 1, 300)
    assert_bf16_close(y, _r(x.float() @ w.float().t()), 2e-2, 5e-3, 'strided')


def test_linear_rows_rejects_bad_shapes():
    from motif.ops.linear_rows import linear_rows
    x = torch.zeros(4, 40, dtype=bf, device=DEV)
    w = torch.zeros(8, 40, dtype=bf, device=DEV)
    with pytest.raises(NotImplementedError):
        linear_rows(x, w)  # K not a multiple of 32


def test_linear_rows_deterministic_across_calls():
    """Repeated calls give identical bits (no cross-workgroup accumulation), for
    every tile shape the launcher picks (M 8 / 20 / 64 and narrow / wide N)."""
    from motif.ops.linear_rows import linear_rows
    for M, N, K in [(8, 768, 2048), (20, 1920, 768), (64, 768, 1536), (64, 4632, 768)]:
        x, w = _operands(M, N, K, 12)
        xd, wd = x.to(DEV), w.to(DEV)
        y1 = linear_rows(xd, wd)
        y2 = linear_rows(xd, wd)
        assert torch.equal(y1.cpu(), y2.cpu())
        assert_bf16_close(y1, _r(x.float() @ w.float().t()), 2e-2, 5e-3, f'M={M} N={N} K={K}')
