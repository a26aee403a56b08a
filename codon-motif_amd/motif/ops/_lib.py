'''ctypes binding of libmotif_hip.so (declared in include/motif_hip.h).

The library is loaded after `torch` so that it binds to the HIP runtime torch
already loaded (both are `libamdhip64.so.7`): one runtime per process, so the
hipStream_t handles and device pointers torch hands out are valid for it.
'''
import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), 'libmotif_hip.so')

MOTIF_F32 = 0
MOTIF_BF16 = 1
MOTIF_F16 = 2

_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_P = ctypes.c_void_p
_F32 = ctypes.c_float
_SZ = ctypes.c_size_t

# Argument lists mirror include/motif_hip.h one for one.
_T4 = [_P, _I64, _I64, _I64]
_SIGNATURES = {
    'motif_abi_version': ([], _I32),
    'motif_last_error': ([], ctypes.c_char_p),
    'motif_gdn_recurrent_fwd': (
        _T4 * 5 + [_P, _P] + _T4 + [_I32] * 5 + [_I32, _I32, _P], _I32),
    'motif_gdn_chunk_workspace_bytes': ([_I32] * 5, _SZ),
    'motif_gdn_chunk_fwd': (
        _T4 * 5 + [_P, _P] + _T4 + [_I32] * 6 + [_P, _P, _I32, _I32, _P, _SZ, _I32, _I32, _P], _I32),
    'motif_gdn_chunk_fwd_gated': (
        _T4 * 5 + [_P, _P] + _T4 + [_I32] * 6 + [_P, _P, _I32, _I32, _P, _SZ]
        + [_P, _I64, _I64, _P, _F32, _P, _I64, _I64, _I32, _P], _I32),
    'motif_gdn_prefill_fused': (
        [_P, _I64, _I64] + [_I32] * 6 + [_P] * 3 + [_I32] + [_P] * 6 + [_P, _P, _F32, _P, _F32]
        + [_P, _P, _P, _I64, _I64] + [_I32] * 5 + [_P, _P, _I32, _I32, _P, _SZ, _P], _I32),
    'motif_short_conv_silu': (
        [_P, _I64, _I64, _P, _P, _P, _P, _I64, _I64] + [_I32] * 4 + [_P, _I32, _I32, _I32, _P], _I32),
    'motif_short_conv_silu_multi': (
        [_I32] + [_P] * 12 + [_I32] * 3 + [_P, _I32, _I32, _I32, _P], _I32),
    'motif_gdn_decode_fused': (
        [_P, _I64] + [_I32] * 6 + [_P] * 12 + [_F32, _P, _P, _P, _I64] + [_I32] * 6 + [_P], _I32),
    'motif_linear_rows': (
        [_P, _I64, _P, _I64, _P, _I64] + [_I32] * 4 + [_P, _I64, _P, _I64, _P, _I64, _P], _I32),
    'motif_linear_rows_pair': (
        [_P, _I64, _P, _I64, _P, _I64, _I32, _I32, _I32, _P, _I64, _P, _I64, _P, _I64, _I32, _I32, _I32, _P], _I32),
    'motif_linear_rows_dual': (
        [_P, _I64, _P, _I64, _I32, _P, _I64, _P, _I64, _I32, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I32, _I32, _P],
        _I32),
    'motif_chord_qkv_prep': (
        [_P, _I64, _I64, _I32, _I32, _I32, _P, _P, _F32] + [_P, _I64, _I64, _I64] * 3 + [_P] + [_I32] * 8 + [_P],
        _I32),
    'motif_gated_rms_norm': (
        [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _F32, _P, _I64, _I64] + [_I32] * 5 + [_P], _I32),
    'motif_gdn_gates': (
        [_P, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _I64] + [_I32] * 4 + [_P], _I32),
    'motif_mul_sigmoid': ([_P, _I64, _P, _I64, _P, _I64, _I32, _I32, _I32, _P], _I32),
    'motif_swiglu': ([_P, _I64, _P, _I64, _I32, _I32, _I32, _P], _I32),
    'motif_add_fold': ([_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I32, _I32, _I32, _P], _I32),
    'motif_residual_fold': ([_P, _I64] * 3 + [_P, _P, _I32, _P, _I64, _P, _I64, _I32, _I32, _I32, _P], _I32),
    'motif_attn_res_read_norms': (
        [_P, _P, _P, _I32, _P, _P, _F32, _P, _I64, _I64, _I32, _P, _P, _P, _P, _F32] + [_I32] * 4 + [_P], _I32),
    'motif_attn_res_read': (
        [_P, _P, _P, _I32, _P, _P, _F32, _P, _I64, _I64] + [_I32] * 4 + [_P], _I32),
    'motif_short_conv_silu_l2norm': (
        [_P, _I64, _I64, _P, _P, _P, _P, _I64, _I64] + [_I32] * 4 + [_P, _I32, _I32, _I32, _F32, _I32, _P], _I32),
    'motif_chord_workspace_bytes': ([_I32] * 6 + [ctypes.POINTER(_I32)], _SZ),
    'motif_chord_decode_workspace_bytes': ([_I32] * 7 + [ctypes.POINTER(_I32)], _SZ),
    'motif_chord_decode': (
        _T4 * 3 + [_P, _I32] + [_P] * 4 + [_P, _I64, _I64, _P, _I32] + _T4 + [_I32] * 5 + [_F32, _F32]
        + [_P, _SZ, _I32, _P], _I32),
    'motif_chord_decode_step_workspace_bytes': ([_I32] * 5, _SZ),
    'motif_chord_decode_step': (
        [_P, _I64, _I64, _I32, _I32, _I32, _P, _P, _F32] + [_P, _I64, _I64, _I64] * 2 + [_P, _I32] + [_P] * 4
        + [_P, _I32] + _T4 + [_I32] * 5 + [_F32, _F32] + [_P, _SZ, _P], _I32),
    'motif_chord_decode_noalloc_scratch_bytes': ([], _SZ),
    'motif_chord_decode_noalloc': (
        _T4 * 3 + [_P, _I32] + [_P] * 4 + [_P, _I64, _I64, _P, _I32] + _T4 + [_I32] * 5 + [_F32, _F32]
        + [_I32, _P], _I32),
    'motif_probe_copy': ([_P, _P, _SZ, _I32, _P], _I32),
    'motif_probe_read': ([_P, _P, _SZ, _I32, _P], _I32),
    'motif_probe_mfma_bf16': ([_P, _I32, _I32, _I32, _P], _I32),
    'motif_chord_fwd': (
        _T4 * 3 + [_P, _P, _P, _P] + [_P, _I64, _I64] + _T4 + [_P] + [_I32] * 6
        + [_I32, _F32, _F32] + [_P, _I32, _I32] + [_P, _SZ] + [_I32, _P], _I32),
    'motif_gdn_scan_fwd_f32': ([_P] * 8 + [_I32] * 5 + [_P], _I32),
    'motif_gdn_scan_bwd_f32': ([_P] * 8 + [_I32] * 5 + [_P], _I32),
    'motif_gdn_opscan_f32': ([_P] * 5 + [_I32] * 6 + [_P], _I32),
    'motif_gdn_opscan_pair_f32': ([_P] * 9 + [_I32] * 4 + [_P], _I32),
    'motif_gdn_bwd_prep_f32': ([_P] * 15 + [_I32] * 5 + [_P], _I32),
    'motif_gdn_bwd_chunk_f32': ([_P] * 18 + [_I32] * 5 + [_P], _I32),
    'motif_chord_bwd_workspace_bytes': ([_I32] * 6, _SZ),
    'motif_chord_bwd': (
        _T4 * 5 + [_P] * 5 + [_P, _I64, _I64] + _T4 * 3 + [_P] + [_I32] * 7 + [_F32, _F32]
        + [_P, _SZ, _I32, _P], _I32),
}

EXPORTED = tuple(_SIGNATURES)

_lib = None
_load_error = None


def _load():
    global _lib, _load_error
    if _lib is not None or _load_error is not None:
        return
    try:
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    except (OSError, AttributeError) as exc:
        _load_error = exc


def available() -> bool:
    '''True when the kernel library loaded and a ROCm device is visible.'''
    _load()
    return _lib is not None and torch.cuda.is_available()


def lib():
    '''The loaded library; raises RuntimeError when it cannot be loaded.'''
    _load()
    if _lib is None:
        raise RuntimeError(
            f'the motif HIP kernel library is not available ({LIB_PATH}): {_load_error}. '
            'Build it with `python codon-motif_amd/csrc/build.py`.')
    return _lib


ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP = 1, 2, 3


def check(rc: int, what: str):
    '''Turn a non-zero motif_status into an exception (INVALID -> ValueError).'''
    if rc == 0:
        return
    msg = lib().motif_last_error().decode(errors='replace')
    if rc == ERR_INVALID:
        raise ValueError(f'{what}: {msg}')
    if rc == ERR_UNSUPPORTED:
        raise NotImplementedError(f'{what}: {msg}')
    raise RuntimeError(f'{what}: {msg}')


def chord_dtype_code(dt: torch.dtype) -> int:
    '''dtype code of the Chord attention entries, which also take fp16.'''
    if dt == torch.float16:
        return MOTIF_F16
    return dtype_code(dt)


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return MOTIF_F32
    if dt == torch.bfloat16:
        return MOTIF_BF16
    raise NotImplementedError(f'unsupported dtype {dt} (float32 / bfloat16 only)')


def stream_ptr(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t):
    return None if t is None else t.data_ptr()


def t4(t):
    '''(pointer, batch stride, head stride, time stride) of a [B, H, T, ...] tensor.'''
    return [t.data_ptr(), t.stride(0), t.stride(1), t.stride(2)]
