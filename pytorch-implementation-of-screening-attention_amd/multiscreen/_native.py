"""ctypes binding of libmsa.so, the C ABI declared in include/msa.h.

The library is built in-tree by build_lib.py next to this file.  Loading
fails loudly (RuntimeError) when it is missing: there is no other GPU path.
"""

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmsa.so")

MSA_F32 = 0
MSA_BF16 = 1
MSA_F16 = 2

# kernel ids for msa_timer_arm (include/msa.h)
K_PREP_K, K_FWD_SCREEN, K_FWD_LIVE, K_DKDV, K_DQ, K_DECODE = 1, 2, 3, 4, 5, 7

_lock = threading.Lock()
_lib = None

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_u64 = ctypes.c_uint64
_sz = ctypes.c_size_t

_SIGS = {
    "msa_version": (_i, []),
    "msa_last_error": (ctypes.c_char_p, []),
    "msa_fwd_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "msa_tile_bits_words": (_sz, [_i, _i, _i, _i]),
    "msa_bwd_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "msa_fwd": (_i, [_p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
                     _i, _i, _i, _i, _i, _i, _p, _p, _p, _i, _f, _f, _u64,
                     _p, _p, _p, _sz, _p, _sz, _p]),
    "msa_bwd": (_i, [_p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
                     _i, _i, _i, _i, _i, _i, _p, _p, _p, _i, _f, _f, _u64,
                     _p, _p, _p, _p, _sz,
                     _p, _p, _p, _p, _p, _p, _sz, _p]),
    "msa_decode_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "msa_decode": (_i, [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
                        _i, _i, _i, _i, _i, _i, _i, _p, _p, _f, _p, _p, _sz, _p]),
    "msa_decode_at": (_i, [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
                           _i, _i, _i, _i, _p, _i, _i, _p, _p, _f, _p, _p, _sz, _p]),
    "msa_decode_noalloc": (_i, [_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
                                _i, _i, _i, _i, _i, _i, _i, _p, _p, _f, _p, _p]),
    "msa_timer_arm": (_i, [_i, _i]),
    "msa_timer_arm_every": (_i, [_i, _i, _i]),
    "msa_timer_read": (_i, [_i, ctypes.POINTER(ctypes.c_float), _i]),
    "msa_selftest_mfma": (_i, [_p, _p, _p, _p, _p, _p, _p]),
}

EXPORTED = tuple(_SIGS)


def lib():
    """Returns the loaded library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"libmsa.so not found at {LIB_PATH}; build it with "
                    "`python build_lib.py` (or __graft_entry__.build())")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


class MsaError(RuntimeError):
    """A nonzero status from libmsa; the message is msa_last_error()."""


def check(rc, what):
    if rc != 0:
        msg = lib().msa_last_error().decode(errors="replace")
        raise MsaError(f"{what} failed (status {rc}): {msg}")
