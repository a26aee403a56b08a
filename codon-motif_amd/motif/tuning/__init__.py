'''Library-GEMM tuning results for the shapes the model runs on hipBLASLt / rocBLAS
(prefill projections at T = 4096, the vocabulary projection), produced on an MI355X
with PyTorch TunableOp (tuning enabled, each projection shape run once, the results
file written by torch.cuda.tunable.write_file).

`enable()` loads them read-only (no tuning at run time).  PyTorch checks the
recorded PyTorch / HIP / hipBLASLt / rocBLAS versions and the GPU architecture
against the running ones and ignores the file on a mismatch, so a stale file only
costs the default algorithm choice.
'''
import os

import torch

RESULTS = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'gemm_mi355x.csv')


def enable(path: str = RESULTS) -> bool:
    '''Use the tuned GEMM algorithms in `path` (no new tuning); returns whether the file
    was found.'''
    if not os.path.exists(path):
        return False
    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(False)
    torch.cuda.tunable.set_filename(path)
    torch.cuda.tunable.read_file(path)
    return True
