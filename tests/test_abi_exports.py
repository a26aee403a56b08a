'''The C-ABI boundary without a GPU: the kernel library loads, exports every entry point
include/motif_hip.h declares, and the Python binding table (motif.ops._lib) names only
declared entry points, with the argument counts of their declarations.  No compute call
is made (the two calls below touch no device).'''
import ctypes
import os
import re

import pytest

from motif.ops import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'motif_hip.h')
DECL = re.compile(r'^\s*(?:int|size_t|const char \*|void|int64_t)\s*\*?\s*(motif_\w+)\s*\(([^;]*)\);', re.M | re.S)


def _declarations():
    src = re.sub(r'/\*.*?\*/', '', open(HEADER).read(), flags=re.S)
    out = {}
    for name, args in DECL.findall(src):
        args = ' '.join(args.split())
        out[name] = 0 if args in ('', 'void') else args.count(',') + 1
    return out


def test_header_parses():
    decl = _declarations()
    assert len(decl) >= 30
    assert 'motif_gdn_chunk_fwd' in decl and 'motif_chord_fwd' in decl


def test_library_exports_every_declared_entry_point():
    assert os.path.exists(_lib.LIB_PATH), f'kernel library not built: {_lib.LIB_PATH}'
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declarations() if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_match_declarations():
    decl = _declarations()
    for name, (args, _res) in _lib._SIGNATURES.items():
        assert name in decl, f'{name} is bound but not declared in include/motif_hip.h'
        assert len(args) == decl[name], f'{name}: {len(args)} bound arguments, {decl[name]} declared'


def test_host_only_entry_points():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    lib.motif_abi_version.restype = ctypes.c_int
    assert lib.motif_abi_version() > 0
    lib.motif_last_error.restype = ctypes.c_char_p
    assert isinstance(lib.motif_last_error(), bytes)
