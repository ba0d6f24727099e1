"""Loading of the in-tree native libraries."""
from __future__ import annotations

import ctypes as C
from functools import lru_cache
from pathlib import Path

PKG = Path(__file__).resolve().parent.parent
BUILD = PKG / "build"


def _load(name: str) -> C.CDLL:
    p = BUILD / name
    if not p.exists():
        raise RuntimeError(f"{p} is not built; run __graft_entry__.build() (or python zonos2.cpp_amd/build.py)")
    return C.CDLL(str(p), mode=C.RTLD_GLOBAL)


@lru_cache(None)
def host_lib() -> C.CDLL:
    lib = _load("libzonos2_host.so")
    lib.z2s_stream_id.restype = C.c_uint64
    lib.z2s_stream_id.argtypes = [C.c_char_p]
    lib.z2s_generate.restype = C.c_int
    lib.z2s_generate.argtypes = [C.c_uint64, C.c_uint64, C.c_int, C.c_float, C.c_float, C.c_int,
                                 C.c_int64, C.c_int64, C.c_void_p, C.c_int]
    lib.z2s_quantize.restype = C.c_int
    lib.z2s_quantize.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int]
    lib.z2s_row_bytes.restype = C.c_int64
    lib.z2s_row_bytes.argtypes = [C.c_int, C.c_int64]
    return lib
