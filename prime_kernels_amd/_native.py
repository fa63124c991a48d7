"""ctypes binding of the C ABI in include/prime_decode.h (libprime_decode.so).

This is the only place Python crosses into native code.  There is no fallback: if the library
is missing the import-time call raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libprime_decode.so"

MODEL_360M = 360
MODEL_135M = 135

# status codes of include/prime_decode.h that callers act on
PK_ERR_ABORTED = 9113
PK_ERR_NOALLOC = 9115
# pk_set_option options
PK_OPT_COOPERATIVE = 1
PK_OPT_SPLIT_ROLE = 2
PK_OPT_L2_RECORDS = 3
PK_OPT_SKEW = 4
PK_OPT_SPLIT_WIDE = 5

_lib = None

vp, ci, ll, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_size_t

# symbol -> (restype, argtypes); the list every test checks against include/*.h
SIGNATURES = {
    "pk_workspace_bytes": (sz, [ci]),
    "pk_init": (ci, []),
    "pk_set_option": (ci, [ci, ci]),
    "pk_state_read": (ci, [vp, sz, ctypes.POINTER(ctypes.c_uint), ci]),
    "pk_state_status": (ci, [vp, ctypes.POINTER(ctypes.c_uint)]),
    "pk_state_take": (ci, [vp, ctypes.POINTER(ctypes.c_uint)]),
    "pk_test_exchange_units": (ci, [ci, ci, ci, ctypes.POINTER(ctypes.c_uint)]),
    "pk_test_set_epoch": (ci, [vp, ctypes.c_uint]),
    "pk_test_abort_next": (ci, [vp]),
    "pk_test_abort_next_noalloc": (ci, [vp]),
    "pk_noalloc_status": (ci, [vp, ci, ctypes.POINTER(ctypes.c_uint)]),
    "pk_decode": (ci, [vp, ci, ci, ci, vp, ci, vp, vp, vp, vp, vp, ci, vp, vp, vp,
                       ll, ll, ll, ll, ll, ci, vp, ci, vp, vp, vp, vp, vp, sz, ci]),
    "pk_decode_noalloc": (ci, [vp, ci, ci, ci, vp, ci, vp, vp, vp, vp, vp, ci, vp, vp, vp,
                               ll, ll, ll, ll, ll, ci, vp, ci, vp, vp, vp, vp, ci]),
    "pk_decode_debug": (ci, [vp, ci, ci, ci, vp, ci, vp, vp, vp, vp, vp, ci, vp, vp, vp,
                             ll, ll, ll, ll, ll, ci, vp, ci, vp, vp, vp, vp, vp, sz, ci, vp, vp, sz, ci]),
    "pk_decode_mxfp8": (ci, [vp, ci, ci, ci, vp, ci, vp, vp, vp, vp, vp, ci, vp, vp, vp,
                             ll, ll, ll, ll, ll, ci, vp, ci, vp, vp, vp, vp, vp, sz, ci]),
    "pk_mxfp8_scale_stride": (sz, [ci]),
    "pk_quantize_mxfp8": (ci, [vp, vp, vp, vp, ci, ci]),
    "pk_query": (ci, [ctypes.POINTER(ci), ctypes.POINTER(ci), ctypes.POINTER(ci), ctypes.POINTER(ci),
                      ctypes.POINTER(sz)]),
    "prime_decode_status_string": (ctypes.c_char_p, [ci]),
    "pk_set_trace": (None, [vp]),
    "decode360": (ci, [vp, ci, vp, vp, vp, vp, vp, vp, ci, vp, vp, vp, ll, ll, ll, ll, ll, ci, vp, ci,
                       vp, vp, vp, sz, vp, sz, ci, ci]),
    "decode360_workspace_bytes": (sz, []),
    "decode360_debug_bytes": (sz, []),
    "decode360_status_string": (ctypes.c_char_p, [ci]),
    "mk_decode": (ci, [vp, ci, vp, ci, vp, vp, vp, ci, vp, vp, vp, vp, vp, ll, ll, ll, ll, ll, ci, vp,
                       ci, vp, vp, sz, ci]),
    "mk_workspace_bytes": (sz, [ci, ci]),
    "mk_status_string": (ctypes.c_char_p, [ci]),
    "block360_decode": (ci, [vp, ci, vp, vp, vp, vp, ci, vp, vp, vp, ll, ll, ll, ll, ll, ci, vp, ci, vp, vp, sz,
                             vp, sz, ci]),
    "block360_workspace_bytes": (sz, []),
    "block360_debug_bytes": (sz, []),
    "block360_status_string": (ctypes.c_char_p, [ci]),
    # include/prime_lossless.h
    "lossless_scan_workspace_bytes": (sz, []),
    "lossless_encode_layer": (ci, [vp, vp, vp, vp, vp, vp, vp, vp, sz, vp, ctypes.c_uint, vp]),
    "lossless_decode_layer": (ci, [vp, vp, vp, vp, vp]),
    "lossless_write_descriptor": (ci, [vp, ci, vp, vp, vp, vp, vp, vp]),
    "decode360_lossless": (ci, [vp, ci, vp, vp, vp, vp, vp, vp, ci, vp, vp, vp, ll, ll, ll, ll, ll, ci, vp, ci,
                                vp, vp, vp, sz, vp, sz, ci, ci, vp]),
    "pk_decode_lossless": (ci, [vp, ci, ci, ci, vp, ci, vp, vp, vp, vp, vp, ci, vp, vp, vp,
                                ll, ll, ll, ll, ll, ci, vp, ci, vp, vp, vp, vp, vp, sz, ci, vp]),
}


def library() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m prime_kernels_amd.build`")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def status_string(rc: int) -> str:
    return library().prime_decode_status_string(rc).decode()
