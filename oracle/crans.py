"""ctypes wrapper of oracle/rans.c -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The C file defines this engine's rANS stream format (its header comment is the
specification); these helpers take and return numpy uint8 arrays."""

from __future__ import annotations

import ctypes

import numpy as np

from . import cbitpack

BLOCK = 65536
HEADER = 32


def _lib():
    lib = cbitpack._load()
    if not getattr(lib, "_rans_ready", False):
        u8p = ctypes.POINTER(ctypes.c_uint8)
        lib.oracle_rans_max_bytes.argtypes = [ctypes.c_uint64, ctypes.c_int]
        lib.oracle_rans_max_bytes.restype = ctypes.c_int64
        lib.oracle_rans_encode.argtypes = [u8p, ctypes.c_uint64, ctypes.c_int, u8p, ctypes.c_int64]
        lib.oracle_rans_encode.restype = ctypes.c_int64
        lib.oracle_rans_decode.argtypes = [u8p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int, u8p]
        lib.oracle_rans_decode.restype = ctypes.c_int
        lib._rans_ready = True
    return lib


def max_bytes(n: int, w: int) -> int:
    return int(_lib().oracle_rans_max_bytes(n, w))


def pack(sym: np.ndarray, w: int) -> np.ndarray:
    """LSB-first packing of w-bit symbols (the bitpack body, without its header)."""
    return cbitpack.encode(sym, w)[16:]


def unpack(body: np.ndarray, n: int, w: int) -> np.ndarray:
    hdr = cbitpack.encode(np.zeros(0, np.uint8), w)[:16].copy()
    hdr[8:16] = np.frombuffer(np.uint64(n).tobytes(), np.uint8)
    return cbitpack.decode(np.concatenate([hdr, np.ascontiguousarray(body, np.uint8)]), n, w)


def encode_packed(body: np.ndarray, n: int, w: int) -> np.ndarray:
    b = np.ascontiguousarray(body, np.uint8)
    if b.size != (n * w + 7) // 8:
        raise ValueError("packed body length does not match n and w")
    cap = max_bytes(n, w)
    out = np.zeros(max(cap, 1), np.uint8)
    p = ctypes.POINTER(ctypes.c_uint8)
    rc = _lib().oracle_rans_encode(b.ctypes.data_as(p), n, w, out.ctypes.data_as(p), cap)
    if rc < 0:
        raise ValueError(f"rans encode failed ({rc})")
    return out[:rc].copy()


def decode_packed(stream: np.ndarray, n: int, w: int) -> np.ndarray:
    s = np.ascontiguousarray(stream, np.uint8)
    out = np.zeros(max((n * w + 7) // 8, 1), np.uint8)
    p = ctypes.POINTER(ctypes.c_uint8)
    rc = _lib().oracle_rans_decode(s.ctypes.data_as(p), s.size, n, w, out.ctypes.data_as(p))
    if rc:
        raise ValueError(f"rans decode failed ({rc})")
    return out[:(n * w + 7) // 8]


def encode(sym: np.ndarray, w: int) -> np.ndarray:
    s = np.ascontiguousarray(sym, np.uint8).reshape(-1)
    return encode_packed(pack(s, w), s.size, w)


def decode(stream: np.ndarray, n: int, w: int) -> np.ndarray:
    return unpack(decode_packed(stream, n, w), n, w)
