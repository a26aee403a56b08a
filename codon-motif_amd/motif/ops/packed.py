'''Packed-sequence boundaries with their host-side metadata (no reference counterpart: the
reference has no packed forms).

The packed kernels take the boundaries on the device, but their launches need a few
host values: the number of sequences, the longest sequence (grid size), the chunk offsets
of the chunked delta rule (grid size and per-chunk sequence map) and, for the layers, each
token's position inside its sequence.  `PackedSeqs` reads `cu_seqlens` back once, checks
it, and keeps all of these, so a packed forward that is handed one `PackedSeqs` makes no
further device-to-host reads; built before a hipGraph capture, it lets the whole packed
forward be captured.  Every packed op also takes a plain `cu_seqlens` tensor (and then
builds the metadata itself).
'''
from typing import Dict, Optional, Tuple

import torch


class PackedSeqs:
    '''Sequence i covers tokens [cu[i], cu[i + 1]) of a packed batch row.'''

    def __init__(self, cu_seqlens: torch.Tensor, total: Optional[int] = None,
                 device: Optional[torch.device] = None):
        cu_host = cu_seqlens.detach().to('cpu', torch.int64).reshape(-1)
        if cu_host.numel() < 1:
            raise ValueError('cu_seqlens needs at least one entry')
        lens = cu_host[1:] - cu_host[:-1]
        if int(cu_host[0]) != 0 or (lens < 0).any() or (total is not None and int(cu_host[-1]) != total):
            raise ValueError('cu_seqlens must start at 0, be non-decreasing and end at the packed length')
        if device is None:
            device = cu_seqlens.device
        self.device = torch.device(device)
        self.cu_host = cu_host
        self.lens = lens
        self.nseq = int(lens.numel())
        self.total = int(cu_host[-1])
        self.max_len = int(lens.max()) if self.nseq else 0
        self.cu = cu_host.to(device=self.device, dtype=torch.int32)
        self._coff: Dict[int, Tuple[torch.Tensor, int]] = {}
        self._pos: Optional[torch.Tensor] = None

    @staticmethod
    def of(cu_seqlens, total: Optional[int] = None, device=None) -> 'PackedSeqs':
        '''`cu_seqlens` itself when it is a PackedSeqs (checked against `total`), else the
        metadata built from the tensor.'''
        if isinstance(cu_seqlens, PackedSeqs):
            if total is not None and cu_seqlens.total != total:
                raise ValueError('cu_seqlens must start at 0, be non-decreasing and end at the packed length')
            return cu_seqlens
        return PackedSeqs(cu_seqlens, total, device)

    def bounds(self):
        '''[(start, end)] per sequence, on the host.'''
        cu = self.cu_host.tolist()
        return list(zip(cu[:-1], cu[1:]))

    def chunk_offsets(self, chunk: int) -> Tuple[torch.Tensor, int]:
        '''(cumulative chunk counts [nseq + 1] int32 on the device, total chunks) for
        chunks of `chunk` tokens that never cross a sequence boundary.'''
        if chunk not in self._coff:
            coff = torch.zeros(self.nseq + 1, dtype=torch.int32)
            coff[1:] = torch.cumsum((self.lens + chunk - 1) // chunk, 0).to(torch.int32)
            self._coff[chunk] = (coff.to(self.device), int(coff[-1]))
        return self._coff[chunk]

    def positions(self) -> torch.Tensor:
        '''Each token's position inside its sequence, int64 [total] on the device.'''
        if self._pos is None:
            pos = torch.arange(self.total) - torch.repeat_interleave(self.cu_host[:-1], self.lens)
            self._pos = pos.to(self.device)
        return self._pos
