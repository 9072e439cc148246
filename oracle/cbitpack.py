"""ctypes wrapper of oracle/bitpack.c -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py)."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle.so"
_lib = None


def build() -> Path:
    """Compile bitpack.c with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        u8p = ctypes.POINTER(ctypes.c_uint8)
        lib.oracle_bitpack_encode.argtypes = [u8p, ctypes.c_int64, ctypes.c_int, u8p]
        lib.oracle_bitpack_decode.argtypes = [u8p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, u8p]
        _lib = lib
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))


def encode(sym: np.ndarray, bits: int) -> np.ndarray:
    s = np.ascontiguousarray(sym, dtype=np.uint8).reshape(-1)
    out = np.empty(16 + (s.size * bits + 7) // 8, np.uint8)
    rc = _load().oracle_bitpack_encode(_ptr(s), s.size, bits, _ptr(out))
    if rc:
        raise ValueError("symbol exceeds bitpack_bits")
    return out


def decode(stream: np.ndarray, n: int, bits: int) -> np.ndarray:
    st = np.ascontiguousarray(stream, dtype=np.uint8)
    out = np.empty(n, np.uint8)
    rc = _load().oracle_bitpack_decode(_ptr(st), st.size, n, bits, _ptr(out))
    if rc == -1:
        raise ValueError("BitPackCodec payload length does not match shape and bit width")
    if rc == -2:
        raise ValueError("invalid bitpack header or decode configuration")
    return out
