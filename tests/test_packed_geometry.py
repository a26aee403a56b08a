'''Host-side walk of the packed-sequence launch geometry (CPU; no GPU).

For config 5's sixteen lengths (presets.packed_lengths(), seed 0) and for edge-case
packings (empty, one-token, chunk-multiple and chunk-plus-one sequences), every
workgroup of the packed kernels is replayed here with the kernels' own index math:

- gdn_prep_mfma / gdn_chunk_out (csrc/gdn_chunk.hip; chunk map resolve_chunk in
  csrc/gdn_internal.h): each (chunk, head) workgroup's sequence, first token and
  length; the fused front end's conv-window rows and their range-checked byte offsets
  (csrc/gdn_chunk.hip, phase 1 of the FRONT form), its gate-row loads and the outgoing
  conv-tail writes by each sequence's last chunk; the workspace cell written and read;
- gdn_state_scan: each (column group, head, sequence) wave's first chunk and trip
  count from the chunk offsets, the cells its range-checked buffer covers, the state
  rows it reads and writes;
- chord_fwd_kernel (csrc/chord.hip) with cu_seqlens: each (head group, query block,
  sequence) workgroup's query rows, key-tile range and loop trip counts, and the byte
  ranges of its shrinking K / V buffers.

Every access must stay inside the tensor the host allocates for it, every loop trip
count must be bounded by the sequence's own length, and every range-checked buffer
size must fit the 32-bit record count.  The chunk offsets are built exactly as the
host code builds them (motif/ops/gated_deltanet.py).
'''
import math

import pytest
import torch

from motif.model.presets import cu_seqlens_of, packed_lengths

C = 64          # GDN chunk
K_CONV = 4      # conv kernel length
H, DK, DV = 12, 64, 128
D_MODEL = 768
NCOLS = 2 * H * DK + 2 * H * DV + 2 * H   # q | k | v | gate | a | b projection row
U32 = 1 << 32

PACKINGS = {
    'config5': packed_lengths(),
    'edges': [0, 1, 63, 64, 65, 0, 127, 128, 129, 1, 3, 0],
    'one_long': [8192],
    'all_tiny': [1] * 40,
}


def _offsets(lengths):
    '''cu_seqlens and chunk offsets, as motif.ops.gated_deltanet builds them.'''
    cu = cu_seqlens_of(lengths).to(torch.int64)
    lens = cu[1:] - cu[:-1]
    coff = torch.zeros(len(lengths) + 1, dtype=torch.int64)
    coff[1:] = torch.cumsum((lens + C - 1) // C, 0)
    return [int(x) for x in cu], [int(x) for x in coff]


def resolve_chunk(c, cu, coff):
    '''gdn_internal.h resolve_chunk (packed form): the largest s with coff[s] <= c.'''
    lo, hi, steps = 0, len(cu) - 2, 0
    while lo < hi:
        mid = (lo + hi + 1) >> 1
        if coff[mid] <= c:
            lo = mid
        else:
            hi = mid - 1
        steps += 1
    assert steps <= math.ceil(math.log2(max(len(cu) - 1, 1))) + 1
    t0 = cu[lo] + (c - coff[lo]) * C
    return lo, t0, min(C, cu[lo + 1] - t0)


def _u32(x):
    return x % U32


@pytest.mark.parametrize('name', sorted(PACKINGS))
def test_gdn_packed_chunk_map_and_front_end(name):
    lengths = PACKINGS[name]
    cu, coff = _offsets(lengths)
    L, nseq, total = cu[-1], len(lengths), coff[-1]
    x_st = NCOLS  # projection row stride (elements)
    # the entry's own guard: sequence-relative byte offsets stay below 2^32
    assert (L + K_CONV) * x_st * 2 < U32
    covered = [0] * L
    for c in range(total):
        seq, t0, ln = resolve_chunk(c, cu, coff)
        s_lo, s_hi = cu[seq], cu[seq + 1]
        assert 1 <= ln <= C and s_lo <= t0 and t0 + ln <= s_hi, (c, seq, t0, ln)
        for t in range(t0, t0 + ln):
            covered[t] += 1
        # workspace cell (h * total + chunk) of H * total cells
        assert 0 <= c < total
        # FRONT phase 1: waves 0 / 1 (q / k: 8 segments, 8 rows each), waves 2-3 (v: 16
        # segments, 8 rows each); a thread's conv window reads rows rel0 - 3 .. rel0 + rows - 1
        for prob, (chans, rows) in enumerate(((DK, DK // 8), (DK, DK // 8), (DV, DV // 16))):
            segs = chans // 8
            nthreads = 64 if prob < 2 else 128
            size = ((s_hi - s_lo - 1) * x_st + chans) * 2 if s_hi > s_lo else 0
            assert size < U32
            for t in range(nthreads):
                f_seg, f_r0 = t % segs, (t // segs) * rows
                assert f_r0 + rows <= C
                rel0 = t0 - s_lo + f_r0
                for i in range(K_CONV - 1 + rows):
                    row = rel0 - (K_CONV - 1) + i
                    off = _u32(row * x_st * 2 + 16 * f_seg)
                    in_seq = 0 <= row < s_hi - s_lo
                    # a row of the sequence is read in full range; any other row (before
                    # its start, or past its end) falls outside the buffer and reads 0
                    assert (off + 16 <= size) == in_seq, (c, prob, t, i, row, off, size)
        # gate inputs: row t0 + min(lane, len - 1), inside the sequence
        assert s_lo <= t0 + min(63, ln - 1) < s_hi
        # outgoing tails: written by the sequence's last chunk only, rows of the sequence
        if t0 + ln == s_hi:
            assert c == coff[seq + 1] - 1
            for r in range(K_CONV - 1):
                rel = (s_hi - s_lo) - (K_CONV - 1) + r
                if rel >= 0:
                    assert s_lo <= s_lo + rel < s_hi
            assert seq < nseq
    assert covered == [1] * L, 'every token in exactly one chunk'


@pytest.mark.parametrize('name', sorted(PACKINGS))
def test_gdn_packed_state_scan_geometry(name):
    lengths = PACKINGS[name]
    cu, coff = _offsets(lengths)
    nseq, total = len(lengths), coff[-1]
    ncg, ngroups, xcd = DV // 16, H * nseq, 8
    blocks = xcd * ((ngroups + xcd - 1) // xcd) * ncg
    seen = set()
    cell = 2 * (DK * DK + C * DK + 3 * DK * DV)  # bytes per (head, chunk) cell
    for b in range(blocks):
        slot = b // xcd
        group = (slot // ncg) * xcd + b % xcd
        if group >= ngroups:
            continue
        cg, h, sq = slot % ncg, group % H, group // H
        assert sq < nseq and 0 <= cg < ncg
        seen.add((cg, h, sq))
        first, count = coff[sq], coff[sq + 1] - coff[sq]
        assert 0 <= count == (lengths[sq] + C - 1) // C and first + count <= total
        # buffer over the group's cells: count * cell bytes from cell h * total + first
        assert count * cell < U32
        assert (h * total + first + count) * cell <= H * total * cell
        # state rows read (s_in) and written (s_out): [nseq, H, DK, DV]
        sbase = (sq * H + h) * DK * DV
        assert sbase + (DK - 1) * DV + 16 * cg + 15 < nseq * H * DK * DV
    assert len(seen) == ncg * ngroups, 'every (column group, head, sequence) exactly once'


@pytest.mark.parametrize('name', sorted(PACKINGS))
@pytest.mark.parametrize('hpw', [4, 2, 1])
def test_chord_packed_geometry(name, hpw):
    lengths = PACKINGS[name]
    cu, _ = _offsets(lengths)
    nseq, L = len(lengths), cu[-1]
    maxlen = max(lengths)
    RH = 2 if hpw >= 2 else 1
    RQ = 32 // RH
    HGW = hpw // RH
    QW = (4 // HGW) * RQ
    parts, kBN, kD = 4, 64, 64
    k_st = 64      # k rows of a [1, Hkv, L, 64] tensor
    nqbg_grid = (maxlen + QW - 1) // QW if maxlen > 0 else 0
    for sq in range(nseq):
        tok0, Lq = cu[sq], cu[sq + 1] - cu[sq]
        nqbg = (Lq + QW - 1) // QW
        assert nqbg <= nqbg_grid
        for y in range(nqbg):
            qbg = nqbg - 1 - y
            wg_q_last = min(Lq, (qbg + 1) * QW) - 1
            kv_end = min(Lq, wg_q_last + 1)
            ntiles = (kv_end + kBN - 1) // kBN
            nsteps = (ntiles + parts - 1) // parts
            kbytes = ((kv_end - 1) * k_st + kD) * 2 if kv_end > 0 else 0
            assert kbytes < U32 and kv_end <= Lq
            for part in range(parts):
                t_first = part * nsteps
                t_count = max(0, min(nsteps, ntiles - t_first))
                assert t_count <= (Lq + kBN - 1) // kBN
                for t in (t_first, t_first + t_count - 1) if t_count else ():
                    krem = kbytes - 2 * t * kBN * k_st
                    assert krem > 0, (sq, y, part, t)
                    # the tile's first key is a key of this sequence
                    assert tok0 + t * kBN < tok0 + Lq
            for w in range(4):
                q0 = qbg * QW + (w // HGW) * RQ
                for cq in range(RQ):
                    my_q = q0 + cq
                    row = tok0 + min(my_q, max(Lq - 1, 0))
                    assert tok0 <= row < max(tok0 + Lq, tok0 + 1) and row < max(L, 1)
