'''Packed-sequence metadata (motif.ops.packed.PackedSeqs, CPU): the host values the packed
launches take -- sequence count, longest sequence, chunk offsets of the chunked delta rule,
each token's position inside its sequence -- against direct computations, and the
boundary checks every packed op makes.'''
import pytest
import torch

from motif.model.presets import cu_seqlens_of, packed_lengths
from motif.ops.packed import PackedSeqs

PACKINGS = [packed_lengths(), [0, 1, 63, 64, 65, 0, 127, 128, 129, 1, 3, 0], [8192], [1] * 40, [5]]


@pytest.mark.parametrize('lengths', PACKINGS, ids=['config5', 'edges', 'one_long', 'all_tiny', 'one'])
def test_metadata_matches_direct_computation(lengths):
    cu = cu_seqlens_of(lengths)
    ps = PackedSeqs(cu, total=sum(lengths), device='cpu')
    assert ps.nseq == len(lengths) and ps.total == sum(lengths) and ps.max_len == max(lengths)
    assert ps.bounds() == [(sum(lengths[:i]), sum(lengths[:i + 1])) for i in range(len(lengths))]
    assert ps.cu.dtype == torch.int32 and ps.cu.tolist() == cu.tolist()
    for C in (16, 64):
        coff, total = ps.chunk_offsets(C)
        expect = [0]
        for n in lengths:
            expect.append(expect[-1] + (n + C - 1) // C)
        assert coff.dtype == torch.int32 and coff.tolist() == expect and total == expect[-1]
        assert ps.chunk_offsets(C)[0] is coff   # built once
    pos = [i for n in lengths for i in range(n)]
    assert ps.positions().tolist() == pos


def test_of_passes_an_instance_through_and_checks_its_length():
    ps = PackedSeqs(torch.tensor([0, 3, 7]), device='cpu')
    assert PackedSeqs.of(ps, 7) is ps
    with pytest.raises(ValueError, match='cu_seqlens'):
        PackedSeqs.of(ps, 8)


@pytest.mark.parametrize('cu,total', [([5, 20, 50], 50), ([0, 30, 20, 50], 50), ([0, 20, 40], 50), ([], None)])
def test_bad_boundaries_raise(cu, total):
    with pytest.raises(ValueError, match='cu_seqlens'):
        PackedSeqs(torch.tensor(cu, dtype=torch.int64), total=total, device='cpu')
