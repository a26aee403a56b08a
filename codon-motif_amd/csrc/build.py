'''Build libmotif_hip.so (the C-ABI kernel library) for gfx950 with hipcc.

Usage: python codon-motif_amd/csrc/build.py [-j N] [--verbose]

Every `*.hip` file in this directory is compiled to an object in
`codon-motif_amd/csrc/_build/`, then linked into
`codon-motif_amd/motif/libmotif_hip.so`, which `motif.ops._lib` loads.
'''
import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(os.path.dirname(HERE), 'motif')
OUT = os.path.join(PKG, 'libmotif_hip.so')
BUILD_DIR = os.path.join(HERE, '_build')

HIPCC = os.environ.get('HIPCC', 'hipcc')
ARCH = os.environ.get('MOTIF_OFFLOAD_ARCH', 'gfx950')

# -packed-fp32-ops is disabled on purpose: packed fp32 forms are kept out of
# every kernel; hipcc's host pass warns that it does not know the feature.
FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-fPIC', '-std=c++17',
    '-mcode-object-version=5',
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-I', os.path.join(os.path.dirname(os.path.dirname(HERE)), 'include'),
]
# Per-source extras.  chord.hip and gdn_chunk.hip: MFMA accumulators in ordinary VGPRs,
# so the softmax / rescale code and the scan's per-chunk chain read them without
# accumulator-register copies.  The backward kernels keep the default: their register
# budgets rely on the accumulator file (the VGPR form made the per-chunk gradient
# kernel 19% slower).
EXTRA = {'chord.hip': ['-mllvm', '-amdgpu-mfma-vgpr-form'], 'gdn_chunk.hip': ['-mllvm', '-amdgpu-mfma-vgpr-form']}


def _run(cmd, verbose):
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = '\n'.join(l for l in res.stderr.splitlines() if 'packed-fp32-ops' not in l)
    if res.returncode != 0:
        raise RuntimeError(f'command failed ({res.returncode}): {" ".join(cmd)}\n{err}')
    if verbose and err.strip():
        print(err, file=sys.stderr)


def sources():
    return sorted(os.path.join(HERE, f) for f in os.listdir(HERE) if f.endswith('.hip'))


def build(jobs=None, verbose=False):
    '''Compile every kernel source and link the shared library; returns its path.'''
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(BUILD_DIR, os.path.basename(s)[:-4] + '.o') for s in srcs]
    jobs = jobs or min(len(srcs), os.cpu_count() or 1, 8)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [HIPCC, *FLAGS, *EXTRA.get(os.path.basename(s), []), '-c', s, '-o', o], verbose)
                for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    tmp = OUT + '.tmp'
    _run([HIPCC, f'--offload-arch={ARCH}', '-shared', '-fPIC', '-o', tmp, *objs], verbose)
    os.replace(tmp, OUT)
    return OUT


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('-j', type=int, default=None)
    ap.add_argument('--verbose', action='store_true')
    args = ap.parse_args()
    print(build(args.j, args.verbose))


if __name__ == '__main__':
    main()
