"""ctypes binding of libmolot_amd.so (the C ABI in include/molot_amd/attn_hip.h),
and of the bench-only libmolot_probe.so (include/molot_amd/probe.h).

The library is built in-tree by ``__graft_entry__.build()`` (or
``python -m molot_amd.build``).  There is no fallback: if the library is
missing, ``load()`` raises, so every caller of the product path fails loudly.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmolot_amd.so")
# measurement probes, kept out of the drop-in library (bench.py only)
PROBE_LIB_PATH = os.path.join(_HERE, "libmolot_probe.so")

KV_F32 = 0
KV_BF16 = 1
KV_Q8 = 2

OK = 0
EINVAL = -22
ENOTSUP = -95
ENOSPC = -28
ENOWS = -16
E2BIG = -7

_lock = threading.Lock()
_lib = None
_probe = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_I64 = ctypes.c_int64

# name -> argtypes (all return int status unless listed in _VOID / _STR)
_SIGS = {
    "molot_hip_rope_apply": [_P, _I, _I, _I, _P, _P],
    "molot_hip_rope_append": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _I, _P],
    "molot_hip_attn_decode_gqa_cache": [_P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I, _P],
    "molot_hip_attn_decode_gqa": [_P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _P],
    "molot_hip_attn_decode_gqa_win": [_P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I, _P],
    "molot_hip_attn_decode_head_win": [_P, _P, _P, _P, _I, _I, _F, _I, _I, _I, _P],
    "molot_hip_attn_decode_strided": [_P, _P, _P, _P, _I, _I, _I, _I, _I64, _I64, _F, _I, _I,
                                      _I, _P],
    "molot_hip_decode_step": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _F, _I, _I, _P],
    "molot_hip_decode_step_noalloc": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _F, _I, _I,
                                      _P],
    "molot_hip_decode_step_norm": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _I, _F, _P,
                                   _F, _I, _I, _P],
    "molot_hip_attn_decode_paged": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F,
                                    _I, _I, _P],
    "molot_hip_decode_step_paged": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                                    _I, _P, _F, _I, _I, _P],
    "molot_hip_decode_step_paged_norm": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                                         _I, _I, _P, _P, _I, _F, _P, _F, _I, _I, _P],
    "molot_hip_rope_append_paged": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P,
                                    _I, _P],
    "molot_hip_vexp": [_P, _P, _I64, _P],
    "molot_hip_prob_exp": [_P, _P, _I64, _P],
    "molot_hip_attn_prefill_gqa": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _I, _P],
    "molot_hip_prefill_step": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _I, _F, _P,
                               _F, _I, _I, _P],
    "molot_hip_prefill_step_paged": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                                     _P, _P, _I, _F, _P, _F, _I, _I, _P],
    "molot_hip_decode_step_shared": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _F, _P, _F, _I, _I,
                                     _P],
    "molot_hip_decode_step_paged_shared": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                                           _I, _P, _F, _P, _F, _I, _I, _P],
    "molot_hip_prefill_q": [_P, _I, _I, _I, _I, _P, _F, _P, _P],
    "molot_hip_attn_prefill_paged": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I,
                                     _I, _P],
    "molot_hip_last_plan": [ctypes.POINTER(_I), ctypes.POINTER(_I)],
    "molot_hip_q8_row_bytes": [_I, _I],
    "molot_hip_profile_begin": [_I],
    "molot_hip_profile_end": [ctypes.POINTER(_F), ctypes.POINTER(_F), ctypes.POINTER(_I),
                              ctypes.POINTER(_I)],
}
# include/molot_amd/probe.h (libmolot_probe.so)
_PROBE_SIGS = {
    "molot_probe_read": [_P, _I64, _P, _I64, _P],
    "molot_probe_copy": [_P, _P, _I64, _P],
}
_VOID = {
    "molot_rope_inv_freq": [_F, _I, ctypes.POINTER(ctypes.c_float)],
    "molot_hip_set_split_chunk": [_I],
    "molot_hip_set_tuning": [_I],
    "molot_hip_set_merge": [_I],
    "molot_hip_set_prefill_presplit": [_I],
    "molot_hip_set_block_order": [_I],
    "molot_hip_set_bf16_path": [_I],
}
_STR = {
    "molot_hip_strerror": [_I],
    "molot_hip_version": [],
}
_I64RET = {
    "molot_hip_q8_block_bytes": [_I, _I, _I],
}

# Every function include/molot_amd/attn_hip.h declares (libmolot_amd.so), and
# every function include/molot_amd/probe.h declares (libmolot_probe.so).
EXPORTS = sorted(list(_SIGS) + list(_VOID) + list(_STR) + list(_I64RET))
PROBE_EXPORTS = sorted(_PROBE_SIGS)


def load() -> ctypes.CDLL:
    """Load libmolot_amd.so once; raise if it has not been built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"molot_amd: native library not built ({LIB_PATH}); run "
                "`python -c 'import __graft_entry__ as g; g.build()'`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        for name, args in _VOID.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = None
        for name, args in _STR.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_char_p
        for name, args in _I64RET.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int64
        _lib = lib
        return lib


def load_probe() -> ctypes.CDLL:
    """Load the bench-only probe library (streaming read / copy kernels)."""
    global _probe
    with _lock:
        if _probe is not None:
            return _probe
        if not os.path.exists(PROBE_LIB_PATH):
            raise RuntimeError(f"molot_amd: probe library not built ({PROBE_LIB_PATH})")
        lib = ctypes.CDLL(PROBE_LIB_PATH)
        for name, args in _PROBE_SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        _probe = lib
        return lib


class MolotHipError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        msg = load().molot_hip_strerror(status).decode()
        super().__init__(f"{what}: {msg} (status {status})")


def check(status: int, what: str) -> None:
    if status != 0:
        raise MolotHipError(status, what)
