'''Re-tune the library GEMMs of the benchmark model on this GPU (PyTorch TunableOp) and
write the results next to this file (gemm_mi355x.csv).

Usage (on the GPU box, from the repository root):
    python codon-motif_amd/motif/tuning/tune_gemms.py
Runs one prefill forward (B=1, T=4096) and one decode-batch forward (B=64, T=1) of the
172M-shape model with tuning on; takes tens of seconds.
'''
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(os.path.dirname(HERE)))
sys.path[:0] = [ROOT, os.path.join(ROOT, 'codon-motif_amd')]

import torch  # noqa: E402


def main():
    import bench
    from motif.model.motif import MotifChordModel
    from motif.tuning import RESULTS
    dev = torch.device('cuda', 0)
    torch.cuda.tunable.enable(True)
    torch.cuda.tunable.tuning_enable(True)
    torch.cuda.tunable.set_max_tuning_duration(30)
    torch.cuda.tunable.set_filename(RESULTS)
    cfg = bench.bench_config()
    model = bench.init_model(MotifChordModel(cfg)).to(dev, torch.bfloat16).eval()
    g = torch.Generator().manual_seed(0)
    with torch.no_grad():
        model(torch.randint(0, cfg.vocab_size, (1, 4096), generator=g).to(dev))
        model(torch.randint(0, cfg.vocab_size, (64, 1), generator=g).to(dev))
    torch.cuda.synchronize()
    torch.cuda.tunable.tuning_enable(False)
    print(RESULTS)


if __name__ == '__main__':
    main()
