"""ctypes binding of libomx_gdn.so (the C ABI declared in include/omx_gdn.h).

Loading fails loudly when the library has not been built: there is no CPU or
PyTorch fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libomx_gdn.so")

OK = 0
EINVAL = -1
EUNSUPPORTED = -2
ELAUNCH = -3
F32 = 0
BF16 = 1

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_f = ctypes.c_float
_i = ctypes.c_int
_sz = ctypes.c_size_t

# name -> (restype, argtypes); must match include/omx_gdn.h
SIGNATURES = {
    "omx_gdn_last_error": (ctypes.c_char_p, []),
    "omx_gdn_abi_version": (_i, []),
    "omx_gdn_chunk_fwd": (_i, [_p, _p, _p, _i, _p, _p, _p, _p, _i64, _p, _p,
                               _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f, _i, _p, _sz, _p]),
    "omx_gdn_chunk_fwd_workspace_size": (_sz, [_i64] * 7 + [_i]),
    "omx_gdn_prefill": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _f, _p, _i64, _p, _p, _p, _p, _p,
                             _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _sz, _p]),
    "omx_gdn_prefill_workspace_size": (_sz, [_i64] * 7),
    "omx_gdn_prefill_noalloc": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _f, _p, _i64, _p, _p, _p, _p,
                                     _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p]),
    "omx_gdn_prefill_noalloc_max_scratch": (_sz, []),
    "omx_gdn_decode_step": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _f, _p, _p, _p,
                                 _i64, _i64, _i64, _i64, _i64, _i64, _p]),
    "omx_gdn_recurrent_step": (_i, [_p, _p, _p, _i, _p, _p, _p, _p,
                                    _i64, _i64, _i64, _i64, _i64, _f, _p]),
    "omx_gdn_chunk_bwd": (_i, [_p, _p, _p, _i, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p,
                               _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f, _i, _p, _sz,
                               _p]),
    "omx_gdn_chunk_bwd_workspace_size": (_sz, [_i64] * 7 + [_i]),
    "omx_gdn_prefill_bwd": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _f, _p, _i64, _p, _p, _p, _p, _p,
                                 _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _i64, _i64, _p, _sz, _p]),
    "omx_gdn_prefill_bwd_workspace_size": (_sz, [_i64] * 7),
    "omx_gdn_ab_proj": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p]),
    "omx_gdn_qkv_conv_proj": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i, _p]),
}


class GDNError(RuntimeError):
    """A libomx_gdn call returned an error code."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load (once) and return the library with typed entry points."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m omegalax_amd.build` "
                    "(hipcc, gfx950). There is no fallback implementation.")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def call(name: str, *args) -> int:
    """Call entry point `name`; raise GDNError on a negative return."""
    L = lib()
    rc = getattr(L, name)(*args)
    if rc != OK:
        raise GDNError(name, rc, L.omx_gdn_last_error().decode())
    return rc
