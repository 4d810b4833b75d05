"""ctypes binding of libhga.so (the C ABI declared in include/hga.h).

The library is built in-tree by ``build()`` (hipcc, gfx950).  Loading never falls back to
anything: if the shared object is missing or a symbol is absent, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libhga.so")
CSRC = os.path.join(_HERE, "csrc")

HGA_DTYPE_F32, HGA_DTYPE_BF16 = 0, 1
HGA_ROUTE_CANONICAL = 1
HGA_ROUTE_SPLIT = 2

# every exported entry point and its argument types (include/hga.h)
_i32, _i64, _f32, _vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p


class HgaConfig(ctypes.Structure):
    _fields_ = [
        ("batch", _i32), ("heads", _i32), ("kv_heads", _i32), ("head_dim", _i32),
        ("chunk_size", _i32), ("group_size", _i32), ("topk_chunks", _i32),
        ("topk_groups", _i32), ("keep_first", _i32), ("keep_last", _i32),
        ("cutoff_pair", _i32), ("dtype", _i32), ("scale", _f32), ("group_scale", _f32),
    ]


_CFG = ctypes.POINTER(HgaConfig)
_I32P = ctypes.POINTER(ctypes.c_int32)

SIGNATURES = {
    "hga_version": ([], _i32),
    "hga_last_error": ([], ctypes.c_char_p),
    "hga_prefill_widths": ([_CFG, _i32, _I32P, _I32P, _I32P], _i32),
    "hga_rope": ([_CFG, _i32, _i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _vp,
                  _i64, _i32, _vp], ctypes.c_int),
    "hga_rope_qk": ([_CFG, _i32] + [_vp, _i64, _i64, _i64] * 4 + [_vp, _vp, _i64, _i32, _vp],
                    ctypes.c_int),
    "hga_summarize": ([_CFG, _i32, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp,
                       _vp, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp],
                      ctypes.c_int),
    "hga_route_prefill": ([_CFG, _i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64,
                           _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp], ctypes.c_int),
    "hga_attend_prefill": ([_CFG, _i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp,
                            _i64, _i64, _i64, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _vp, _vp,
                            _i64, _vp], ctypes.c_int),
    "hga_attend_prefill_workspace": ([_CFG, _i32, ctypes.POINTER(ctypes.c_int64)], _i32),
    "hga_attend_prefill_bwd": ([_CFG, _i32] + [_vp, _i64, _i64, _i64] * 5 + [_vp, _vp, _vp, _i32] +
                               [_vp, _i64, _i64, _i64] * 3 + [_vp, _i64, _vp], ctypes.c_int),
    "hga_attend_prefill_bwd_workspace": ([_CFG, _i32, ctypes.POINTER(ctypes.c_int64)], _i32),
    "hga_decode_widths": ([_CFG, _i32, _I32P, _I32P], _i32),
    "hga_route_decode": ([_CFG, _i32, _i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64,
                          _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp], ctypes.c_int),
    "hga_route_decode_workspace": ([_CFG, _i32, _i32, ctypes.POINTER(ctypes.c_int64)], _i32),
    "hga_attend_decode": ([_CFG, _i32, _i32, _i64, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64,
                           _i64, _i32, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64,
                           _i32, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _vp, _i64, _vp],
                          ctypes.c_int),
    "hga_attend_decode_phase": ([_CFG, _i32, _i32, _i64, _vp, _i64, _i64, _i64, _vp, _vp, _i64,
                                 _i64, _i64, _i32, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64,
                                 _i64, _i64, _i32, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _i32,
                                 _vp, _i64, _vp], ctypes.c_int),
    "hga_attend_decode_noalloc": ([_CFG, _i32, _i32, _i64, _vp, _i64, _i64, _i64, _vp, _vp,
                                   _i64, _i64, _i64, _i32, _vp, _vp, _i64, _i64, _i64, _vp, _vp,
                                   _i64, _i64, _i64, _i32, _vp, _vp, _i32, _vp, _i64, _i64, _i64,
                                   _vp], ctypes.c_int),
    "hga_attend_decode_dca": ([_CFG, _i32, _i32, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i32,
                               _vp, _vp, _i64, _i64, _i64, _i32, _vp, _vp, _i64, _i64, _i64,
                               _vp, _vp, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _i32, _vp, _i64,
                               _i64, _i64, _vp, _i64, _vp], ctypes.c_int),
    "hga_attend_decode_workspace": ([_CFG, _i32, _i32, _i64, _i32,
                                     ctypes.POINTER(ctypes.c_int64)], _i32),
    "hga_gather_decode_sizes": ([_CFG, _i32, _I32P, ctypes.POINTER(ctypes.c_int64),
                                 ctypes.POINTER(ctypes.c_int64)], _i32),
    "hga_gather_decode": ([_CFG, _i32, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i32, _vp,
                           _vp, _i32, _vp, _vp, _i64, _vp], ctypes.c_int),
    "hga_write_tokens": ([_CFG, _i32] + [_vp, _i64, _i64, _i64] * 6 + [_vp], ctypes.c_int),
    "hga_attend_decode_overlapped": ([_CFG, _i32, _i32, _i64, _vp, _i64, _i64, _i64, _vp, _vp,
                                      _i64, _i64, _i64, _i32, _vp, _vp, _i64, _i64, _i64, _vp,
                                      _vp, _i64, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _i32,
                                      _vp, _vp, _i32, _vp, _vp, _i64, _vp, _i64, _i64, _i64,
                                      _vp, _i64, _vp], ctypes.c_int),
}

_lib = None


class HgaError(RuntimeError):
    pass


def build(jobs: int = 8) -> str:
    """Compile libhga.so for gfx950 in-tree (always recompiles out-of-date objects)."""
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", CSRC], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HgaError(f"{LIB_PATH} is missing: build it with "
                           "hierarchicalglobalattention_amd.build() (hipcc, gfx950)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(handle, name)   # AttributeError -> missing symbol, loudly
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().hga_last_error().decode(errors="replace")
        raise HgaError(f"{what} failed ({rc}): {msg}")
