'''GPU parity of the fused attention-residual read (HIP) against the fp64 oracle.

fp32: within 1e-5 relative; bf16: the bf16 bar (max-abs 2e-2, mean-rel 5e-3),
the kernel computing in fp32 from bf16 sources and rounding the output once.
'''
import pytest
import torch

from oracle.model import attn_res_read as oracle_read
from support import assert_bf16_close

pytestmark = pytest.mark.gpu

DEV = 'cuda'


class _Norm:
    def __init__(self, weight, eps=1e-6):
        self.weight, self.eps = weight, eps

    def __call__(self, x):  # the RMSNorm the reference applies to the sources
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype) * self.weight


def _case(nsrc, B, T, D, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    srcs = [torch.randn(B, T, D, generator=g) * (0.3 + 0.1 * n) for n in range(nsrc)]  # |x| < 8: bf16 half-ulp < 2e-2
    q = torch.randn(D, generator=g) * 0.1
    w = 1.0 + 0.1 * torch.randn(D, generator=g)
    srcs = [s.to(dtype) for s in srcs]
    return srcs, q.to(dtype), w.to(dtype)


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
@pytest.mark.parametrize('nsrc,B,T,D', [(2, 2, 37, 768), (3, 1, 5, 128), (5, 3, 64, 768), (8, 1, 130, 1024)])
def test_matches_oracle(dtype, nsrc, B, T, D):
    from motif.ops.attn_res import attn_res_read
    srcs, q, w = _case(nsrc, B, T, D, nsrc * 100 + T, dtype)
    out = attn_res_read([s.to(DEV) for s in srcs], q.to(DEV), _Norm(w.to(DEV)))
    ref = oracle_read([s.double() for s in srcs], q.double(), w.double(), 1e-6)
    assert out.dtype == dtype and out.shape == (B, T, D)
    if dtype == torch.float32:
        err = ((out.double().cpu() - ref).abs().max() / ref.abs().max()).item()
        assert err <= 1e-5, err
    else:
        assert_bf16_close(out, ref, what=f'attn_res n={nsrc}')


def test_strided_sources_and_limits():
    '''Sources that are time slices of longer tensors (as the cache aligns them).'''
    from motif.ops.attn_res import attn_res_read
    srcs, q, w = _case(4, 2, 50, 768, 7, torch.float32)
    long = [torch.cat([torch.randn(2, 9, 768), s], 1).to(DEV) for s in srcs]
    views = [x[:, 9:] for x in long]
    out = attn_res_read(views, q.to(DEV), _Norm(w.to(DEV)))
    ref = oracle_read([s.double() for s in srcs], q.double(), w.double(), 1e-6)
    assert ((out.double().cpu() - ref).abs().max() / ref.abs().max()).item() <= 1e-5
    # more sources than the kernel takes: the torch formula, with a warning
    import motif.ops.attn_res as ar
    ar._warned_many = False
    many = views + views + views[:1]
    with pytest.warns(RuntimeWarning, match='at most'):
        out9 = attn_res_read(many, q.to(DEV), _Norm(w.to(DEV)))
    ref9 = oracle_read([s.double() for s in srcs + srcs + srcs[:1]], q.double(), w.double(), 1e-6)
    assert ((out9.double().cpu() - ref9).abs().max() / ref9.abs().max()).item() <= 1e-5


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
@pytest.mark.parametrize('nsrc,B,T,D', [(1, 4, 3, 768), (3, 2, 17, 768), (6, 64, 1, 768), (2, 1, 9, 256)])
def test_read_with_norms_matches_oracle(dtype, nsrc, B, T, D):
    '''Read + the decoder's two RMSNorms in one kernel: norm_i(h) for the stored h.
    bf16: against the oracle's norms of the kernel's own h (the same bf16 h the
    reference would normalise), so the bar covers the norms only; fp32: 1e-5.'''
    from motif.ops.attn_res import attn_res_read, attn_res_read_norms
    from oracle.gdn import rms_norm
    srcs, q, w = _case(nsrc, B, T, D, nsrc * 10 + B, dtype)
    g = torch.Generator().manual_seed(5)
    wa = (1.0 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    wb = (1.0 + 0.1 * torch.randn(D, generator=g)).to(dtype)
    ds = [s.to(DEV) for s in srcs]
    ya, yb = attn_res_read_norms(ds, q.to(DEV), _Norm(w.to(DEV)), _Norm(wa.to(DEV)), _Norm(wb.to(DEV)))
    h = attn_res_read(ds, q.to(DEV), _Norm(w.to(DEV))) if nsrc > 1 else ds[0]
    if dtype == torch.float32:
        href = oracle_read([s.double() for s in srcs], q.double(), w.double(), 1e-6)
        for y, wt in ((ya, wa), (yb, wb)):
            ref = rms_norm(href, wt.double(), 1e-6)
            err = ((y.double().cpu() - ref).abs().max() / ref.abs().max()).item()
            assert err <= 1e-5, err
    else:
        hc = h.cpu()
        for y, wt in ((ya, wa), (yb, wb)):
            ref = rms_norm(hc, wt, 1e-6)   # bf16 eager norm of the same h
            assert_bf16_close(y, ref.float(), 2e-2, 5e-3, f'norm n={nsrc}')
