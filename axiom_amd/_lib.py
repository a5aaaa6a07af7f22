"""ctypes binding of ``libkda_mi355x.so`` (the C ABI of ``include/kda_mi355x.h``).

The library is loaded lazily and only from this package directory.  A missing
library is an error: there is no CPU or framework fallback for any entry point.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libkda_mi355x.so"
HEADER = PKG.parent / "include" / "kda_mi355x.h"

KDA_OK = 0
KDA_ERR_INVALID_ARGUMENT = -1
KDA_ERR_UNSUPPORTED = -2
KDA_ERR_WORKSPACE = -3
KDA_ERR_HIP = -4

KDA_DTYPE_F32 = 0
KDA_DTYPE_BF16 = 1
KDA_DTYPE_F16 = 2
KDA_DTYPE_BF16_F32GATES = 3

KDA_STATUS_NONFINITE = 65536

_vp = ctypes.c_void_p
_i = ctypes.c_int
_i32 = ctypes.c_int32
_f = ctypes.c_float
_sz = ctypes.c_size_t

_SIGNATURES = {
    "kda_chunk_fwd": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp,
                           _i, _i, _i, _i, _i, _i, _f, _i, _i, _vp, _sz]),
    "kda_chunk_fwd_workspace": (_sz, [_i, _i, _i, _i, _i, _i, _i32, _i]),
    "kda_chunk_fwd_workspace_min": (_sz, [_i, _i, _i, _i, _i, _i, _i32, _i]),
    "kda_chunk_fwd_noalloc": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp,
                                   _i, _i, _i, _i, _i, _i, _f, _i, _i]),
    "kda_varlen_status": (_i, [_vp, _vp, _sz, _i, _i, _i, _i, _i, _i, _i32, _i,
                               ctypes.POINTER(_i32)]),
    "kda_chunk_fwd_status": (_i, [_vp, _vp, _sz, _i, _i, _i, _i, _i, _i, _i32, _i,
                                  ctypes.POINTER(_i32)]),
    "kda_recurrent_step": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                _i, _i, _i, _i, _f, _i, _i]),
    "kda_cc_scan": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                         _i, _i, _i, _i, _i, _i, _vp, _sz]),
    "kda_cc_scan_workspace": (_sz, [_i, _i, _i, _i, _i]),
    "kda_cc_scan_bwd": (_i, [_vp] * 15 + [_i, _i, _i, _i, _i, _i, _vp, _sz]),
    "kda_cc_scan_bwd_workspace": (_sz, [_i, _i, _i, _i, _i]),
    "kda_cc_scan_batched": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                 _i, _i, _i, _i, _i, _i, _i, _vp, _sz]),
    "kda_cc_scan_batched_workspace": (_sz, [_i, _i, _i, _i, _i, _i]),
    "kda_cc_scan_bwd_batched": (_i, [_vp] * 15 + [_i, _i, _i, _i, _i, _i, _i, _vp, _sz]),
    "kda_cc_scan_bwd_batched_workspace": (_sz, [_i, _i, _i, _i, _i, _i]),
    "kda_chunk_bwd": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                           _vp, _vp, _vp, _vp, _vp, _vp,
                           _i, _i, _i, _i, _i, _i, _f, _i, _i, _vp, _sz]),
    "kda_chunk_bwd_workspace": (_sz, [_i, _i, _i, _i, _i, _i]),
    "kda_ut_solve": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "kda_ut_solve_bwd": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "kda_prologue": (_i, [_vp] * 16 + [_i] * 7),
    "kda_epilogue": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i, _i, _i]),
    "kda_decode_layer_step": (_i, [_vp] * 15 + [_i, _i, _i, _i, _f, _f, _i, _i, _vp, _sz]),
    "kda_decode_layer_workspace": (_sz, [_i, _i, _i, _i]),
    "kda_prologue_bwd": (_i, [_vp] * 22 + [_i, _i, _i, _i, _i, _i, _vp, _sz]),
    "kda_prologue_bwd_workspace": (_sz, [_i, _i, _i, _i, _i]),
    "kda_epilogue_bwd": (_i, [_vp] * 6 + [_i, _i, _i, _i, _f, _i, _i, _i, _i]),
    "kda_layer_fwd": (_i, [_vp] * 20 + [_i, _i, _i, _i, _i, _f, _f, _i, _i, _i, _vp, _sz]),
    "kda_layer_fwd_workspace": (_sz, [_i, _i, _i, _i, _i, _i]),
    "kda_last_error": (ctypes.c_char_p, []),
    "kda_abi_version": (_i, []),
}

_lib = None


def header_symbols() -> list[str]:
    """Names of every entry point ``include/kda_mi355x.h`` declares."""
    text = HEADER.read_text()
    return re.findall(r"^KDA_API\s+[\w\s\*]+?\b(kda_\w+)\s*\(", text, flags=re.M)


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError when it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"axiom_amd: {LIB_PATH.name} is not built (run `python -m axiom_amd.build`); "
                "the KDA path has no fallback implementation")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().kda_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    """Map a kda_status_t to the reference's exception classes."""
    if rc == KDA_OK:
        return
    msg = f"{what}: {last_error()} (status {rc})"
    if rc == KDA_ERR_HIP:
        raise RuntimeError(msg)
    raise ValueError(msg)
