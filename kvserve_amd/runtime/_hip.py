"""Asynchronous copies on a given stream through the HIP runtime (the one torch and
the kernel library already share, found by its soname).  The runtime issues its
small uploads and downloads this way so that they go to the slot's stream without
making it torch's current stream."""

from __future__ import annotations

import ctypes

H2D, D2H = 1, 2

_hip = None


def memcpy_async(dst: int, src: int, nbytes: int, kind: int, stream: int) -> None:
    global _hip
    if _hip is None:
        lib = ctypes.CDLL("libamdhip64.so.7")
        lib.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                       ctypes.c_void_p]
        lib.hipMemcpyAsync.restype = ctypes.c_int
        _hip = lib
    rc = _hip.hipMemcpyAsync(dst, src, nbytes, kind, stream)
    if rc != 0:
        raise RuntimeError(f"hipMemcpyAsync failed ({rc})")
