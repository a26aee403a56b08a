'''The allocation-free Chord decode entry point (motif_chord_decode_noalloc, scratch
in the library's own per-device array) against the workspace entry point
(motif_chord_decode) through the C ABI: two calls in a row, the second with a
smaller input, bf16 and fp32; each call must give the workspace entry's output
bit for bit (same kernels, same key-range splits) and advance the device cursor
the same way.  Sizes past the scratch are rejected before any launch.'''
import ctypes

import pytest
import torch

from support import gen

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _case(B, H, Hkv, cap, cached, dtype, seed):
    g = gen(seed)
    D = 64
    mk = lambda *s: (torch.randn(*s, generator=g) * 0.5).to(DEV, dtype)
    q = mk(B, H, 1, D)
    k, v = mk(B, Hkv, cap, D), mk(B, Hkv, cap, D)
    params = [(torch.randn(H, generator=g) * 0.1).abs().to(DEV), (torch.randn(H, generator=g) * 0.1).to(DEV),
              torch.zeros(H, device=DEV), torch.ones(H, device=DEV)]
    table = torch.log(torch.arange(1, cap + 1, dtype=torch.float32, device=DEV))
    return q, k, v, params, table, cached


def _run(case, library_scratch):
    from motif.ops.chord_attention import chord_decode_cursor
    q, k, v, (al, be, mu, ss), table, cached = case
    cursor = torch.tensor([cached], dtype=torch.int32, device=DEV)
    out = chord_decode_cursor(q, k, v, cursor, al, be, mu, ss, table, library_scratch=library_scratch)
    torch.cuda.synchronize()
    return out, int(cursor.item())


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@torch.no_grad()
def test_noalloc_equals_workspace_entry_twice(dtype):
    from motif.ops import _lib
    assert _lib.lib().motif_chord_decode_noalloc_scratch_bytes() == 16 << 20
    big = _case(64, 12, 3, 4104, 4096, dtype, seed=1)
    small = _case(5, 4, 2, 300, 171, dtype, seed=2)
    for case in (big, small):
        want, cur_want = _run(case, False)
        got, cur_got = _run(case, True)
        assert torch.equal(got, want), (got.float() - want.float()).abs().max().item()
        assert cur_got == cur_want == case[5] + 1


@torch.no_grad()
def test_noalloc_rejects_sizes_past_its_scratch():
    from motif.ops import _lib
    lib = _lib.lib()
    B, H, Hkv, L, cap = 8192, 12, 3, 1, 4096
    need = lib.motif_chord_decode_workspace_bytes(B, H, Hkv, L, cap, 64, _lib.MOTIF_BF16, None)
    assert need > lib.motif_chord_decode_noalloc_scratch_bytes()
    dummy = torch.zeros(64, device=DEV, dtype=torch.bfloat16)
    cursor = torch.zeros(1, dtype=torch.int32, device=DEV)
    fz = torch.zeros(16, device=DEV)
    p, f = dummy.data_ptr(), fz.data_ptr()
    rc = lib.motif_chord_decode_noalloc(p, 0, 0, 0, p, 0, 0, 0, p, 0, 0, 0, cursor.data_ptr(), cap, f, f, f, f,
                                        None, 0, 0, f, cap, p, 0, 0, 0, B, H, Hkv, L, 64, 0.125, 1e-5,
                                        _lib.MOTIF_BF16, _lib.stream_ptr(torch.device(DEV)))
    assert rc == _lib.ERR_INVALID
    assert b'scratch' in lib.motif_last_error()
