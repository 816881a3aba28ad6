"""ctypes binding of libmoddit.so, the gfx950 C ABI declared in include/moddit.h.

The library is loaded from this package directory only. There is no fallback: if the
library is missing or fails to load, every operation raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmoddit.so"

MODDIT_OK = 0
MODDIT_EINVAL = 1
MODDIT_EUNSUPPORTED = 2
MODDIT_EHIP = 3

BF16, FP16, FP32 = 0, 1, 2
MODE_SPARSE, MODE_BLOCK_DIAGONAL, MODE_FULL = 0, 1, 2
LAYOUT_WAN, LAYOUT_HUNYUAN, LAYOUT_COGVIDEOX, LAYOUT_OTHER = 0, 1, 2, 3

_c_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float

# name -> (restype, argtypes), mirroring include/moddit.h
_SIGNATURES = {
    "moddit_last_error": (ctypes.c_char_p, []),
    "moddit_version": (ctypes.c_char_p, []),
    "moddit_flash_fwd": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                              _c_i64p, _c_i64p, _c_i64p, _c_i64p, _f, _i, _vp]),
    "moddit_block_sparse_fwd": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                     _c_i64p, _c_i64p, _c_i64p, _c_i64p, _f, _i,
                                     _vp, _vp, _i, _i, _i, _vp]),
    "moddit_flash_fwd_map": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                                  _c_i64p, _c_i64p, _c_i64p, _c_i64p, _f, _f, _i, _i, _i, _i,
                                  _vp]),
    "moddit_quantize_qkv": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _c_i64p, _c_i64p, _c_i64p, _i,
                                 _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "moddit_quantize_workspace_floats": (_i, [_i, _i, _i]),
    "moddit_flash_fwd_q8": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                                 _c_i64p, _f, _i, _vp]),
    "moddit_block_sparse_fwd_q8": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i,
                                        _i, _i, _c_i64p, _f, _i, _vp, _vp, _i, _i, _i, _vp]),
    "moddit_sparsity_map": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _c_i64p, _c_i64p,
                                 _f, _f, _i, _i, _i, _i, _i, _vp]),
    "moddit_sparsity_map_merge": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _c_i64p, _c_i64p,
                                       _f, _f, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _vp]),
    "moddit_mts": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "moddit_mts_workspace_bytes": (ctypes.c_int64, [_i, _i]),
    "moddit_mtm_host": (_i, [_i, _i, ctypes.c_double, _vp]),
    "moddit_fit_schur_host": (_i, [_i, _i, ctypes.c_double, _vp]),
    "moddit_fit_workspace_doubles": (ctypes.c_int64, [_i, _i]),
    "moddit_fit_lines": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, ctypes.c_double, _vp]),
    "moddit_fit_lines_noalloc": (_i, [_vp, _vp, _vp, _i, _i, _i, ctypes.c_double, _vp]),
    "moddit_select_lines": (_i, [_vp, _vp, _i, _i, _i, _i, _vp, _vp]),
    "moddit_check_bd": (_i, [_vp, _i, _i, _f, _vp, _vp]),
    "moddit_mask_from_lines": (_i, [_vp, _i, _i, _vp, _i, _i, _i, _i, _i, _i, _i,
                                    _vp, _vp, _vp, _i, _i, _vp]),
    "moddit_mask_to_tiles": (_i, [_vp, _i, _i, _i, ctypes.c_int64, ctypes.c_int64, _i, _i, _i,
                                  _vp, _vp, _i, _i, _vp]),
    "moddit_refresh_merge": (_i, [_vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, _i, _i,
                                  _vp, _vp]),
}

EXPORTED = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib = None


class ModditError(RuntimeError):
    """A libmoddit.so call returned a nonzero status."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python mod-dit_amd/build.py` "
                "(or __graft_entry__.build()) first"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != MODDIT_OK:
        msg = load().moddit_last_error().decode(errors="replace")
        raise ModditError(f"{what} failed (status {rc}): {msg}")


def strides3(*vals: int):
    return (ctypes.c_int64 * 3)(*vals)
