"""ctypes binding of the gfx950 C-ABI library (include/kvserve_amd.h).

The library must exist (``python -m kvserve_amd.build``); there is no CPU fallback:
every entry point of the package raises if it is missing.  ctypes releases the GIL
for the duration of each call, like the reference's pybind11 bindings
(runtime/csrc/kvs_bind.cpp:10-23).
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkvserve_amd.so"
ABI_VERSION = 2

# Device error bits (KVMI_ERR_*) and host return codes (KVMI_*).
ERR_SYMBOL_RANGE = 1
ERR_BAD_HEADER = 2
ERR_CORRUPT = 4
ERR_SYNC = 8
ERR_BLOCK_ID = 16
ERR_SCHEDULE = 32
OK, EINVAL, ELAUNCH, ENOSPC = 0, -22, -5, -28
# Bytes of the fixed device array behind kvmi_v3_compress_noalloc (per GPU).
V3_NOALLOC_SCRATCH_BYTES = 4 * 1024 * 1024

F_NO_TRANSFORM = 1
F_NATIVE_LAYOUT = 2
F_NO_HEADER = 4
F_VALU_FWHT = 8
F_CLAMP_LEVELS = 16
F_TWO_PASS = 32
F_K_TOKEN = 64
F_K_TENSOR = 128
F_V_CHANNEL = 256
F_V_TENSOR = 512
F_ROW_FWHT = 1024

# Every symbol include/kvserve_amd.h declares.
EXPORTS = (
    "kvmi_abi_version",
    "kvmi_bitpack_encode",
    "kvmi_bitpack_decode",
    "kvmi_gather_blocks",
    "kvmi_scatter_blocks",
    "kvmi_gather_blocks_kv_adjacent",
    "kvmi_scatter_blocks_kv_adjacent",
    "kvmi_check_block_ids",
    "kvmi_hadamard",
    "kvmi_kstats_paged",
    "kvmi_encode_paged",
    "kvmi_decode_paged",
    "kvmi_compress_schedule",
    "kvmi_compress_workspace_bytes",
    "kvmi_compress_paged",
    "kvmi_rans_max_bytes",
    "kvmi_rans_scratch_bytes",
    "kvmi_rans_encode",
    "kvmi_rans_decode",
    "kvmi_rans_encode_batch",
    "kvmi_rans_decode_batch",
    "kvmi_v3_compress",
    "kvmi_v3_scratch_bytes",
    "kvmi_v3_decompress",
    "kvmi_v3_compress_noalloc",
    "kvmi_rt_encode",
    "kvmi_rt_decode",
    "kvmi_rt_hadamard",
    "kvmi_rt_scratch_bytes",
)


class Geometry(ctypes.Structure):
    _fields_ = [
        ("block_size", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("bits", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
        ("max_groups", ctypes.c_int32),
        ("reserved", ctypes.c_int32 * 2),
    ]


class RansEncJob(ctypes.Structure):
    _fields_ = [("packed", ctypes.c_void_p), ("n", ctypes.c_int64), ("out", ctypes.c_void_p),
                ("out_capacity", ctypes.c_int64), ("scratch", ctypes.c_void_p), ("scratch_bytes", ctypes.c_int64),
                ("out_len", ctypes.c_void_p)]


class RansDecJob(ctypes.Structure):
    _fields_ = [("stream", ctypes.c_void_p), ("in_bytes", ctypes.c_int64), ("n", ctypes.c_int64),
                ("packed_out", ctypes.c_void_p)]


RT_TRANSFORM = 1
RT_QUANTIZE = 2
RT_ALIGNED = 4
RT_GENERIC = 8


class RtGeometry(ctypes.Structure):
    _fields_ = [("num_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("kernel_tokens", ctypes.c_int32),
                ("flags", ctypes.c_uint32), ("axes", ctypes.c_uint32), ("reserved", ctypes.c_int32 * 3)]


class RtSection(ctypes.Structure):
    _fields_ = [("head_start", ctypes.c_int32), ("head_count", ctypes.c_int32), ("levels", ctypes.c_int32),
                ("axis", ctypes.c_int32), ("aux_min_offset", ctypes.c_int64), ("aux_scale_offset", ctypes.c_int64)]


class RtLayer(ctypes.Structure):
    _fields_ = [("cache", ctypes.c_void_p), ("block_stride", ctypes.c_int64), ("head_stride", ctypes.c_int64),
                ("token_stride", ctypes.c_int64), ("channel_offset", ctypes.c_int64), ("signs", ctypes.c_void_p),
                ("head_order", ctypes.c_void_p), ("u8_offset", ctypes.c_int64), ("sections", RtSection * 2),
                ("num_sections", ctypes.c_int32), ("reserved", ctypes.c_int32)]


# kvmi_layer_job: 8 pointers, 4 int64, 2 int32 -> 104 bytes, 8-byte aligned.  It is
# written as 13 int64 words; the last word carries num_blocks (low half) and
# write_header (high half).
JOB_FIELDS = (
    "pool", "block_ids", "stream", "kmeta", "vmeta", "signs", "profile", "kstats", "pool_blocks",
    "pool_part_stride", "symbol_offset", "chunk_symbols", "num_blocks_and_header",
)
JOB_INT64S = 13
JOB_BYTES = JOB_INT64S * 8

_lock = threading.Lock()
_lib = None

_vp, _i64, _i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
_SIGNATURES = {
    "kvmi_abi_version": ([], ctypes.c_int),
    "kvmi_bitpack_encode": ([_vp, _i64, _i32, _vp, _vp, _vp], ctypes.c_int),
    "kvmi_bitpack_decode": ([_vp, _i64, _i64, _i32, _vp, _vp, _vp], ctypes.c_int),
    "kvmi_gather_blocks": ([_vp, _i64, _vp, _i32, _i64, _vp, _vp], ctypes.c_int),
    "kvmi_scatter_blocks": ([_vp, _i64, _vp, _i32, _i64, _vp, _vp], ctypes.c_int),
    "kvmi_gather_blocks_kv_adjacent": ([_vp, _vp, _i32, _i64, _vp, _vp], ctypes.c_int),
    "kvmi_check_block_ids": ([_vp, _i32, _vp, _vp], ctypes.c_int),
    "kvmi_scatter_blocks_kv_adjacent": ([_vp, _vp, _i32, _i64, _vp, _vp], ctypes.c_int),
    "kvmi_hadamard": ([_vp, _vp, _i64, _i32, _i32, _vp, _i32, _vp], ctypes.c_int),
    "kvmi_kstats_paged": ([ctypes.POINTER(Geometry), _vp, _i32, _i32, _vp, _vp], ctypes.c_int),
    "kvmi_encode_paged": ([ctypes.POINTER(Geometry), _vp, _i32, _i32, _vp, _vp], ctypes.c_int),
    "kvmi_decode_paged": ([ctypes.POINTER(Geometry), _vp, _i32, _i32, _vp, _vp], ctypes.c_int),
    "kvmi_compress_schedule": ([ctypes.POINTER(Geometry), _vp, _i32, _vp, _i64], _i64),
    "kvmi_compress_workspace_bytes": ([_vp], _i64),
    "kvmi_compress_paged": ([ctypes.POINTER(Geometry), _vp, _i32, _i32, _vp, _vp, _vp, _vp], ctypes.c_int),
    "kvmi_rans_max_bytes": ([_i64, _i32], _i64),
    "kvmi_rans_scratch_bytes": ([_i64, _i32], _i64),
    "kvmi_rans_encode": ([_vp, _i64, _i32, _vp, _i64, _vp, _i64, _vp, _vp], ctypes.c_int),
    "kvmi_rans_decode": ([_vp, _i64, _i64, _i32, _vp, _vp, _vp], ctypes.c_int),
    "kvmi_rans_encode_batch": ([ctypes.POINTER(RansEncJob), _i32, _i32, _vp], ctypes.c_int),
    "kvmi_rans_decode_batch": ([ctypes.POINTER(RansDecJob), _i32, _i32, _vp, _vp], ctypes.c_int),
    "kvmi_v3_compress": ([_vp, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], ctypes.c_int),
    "kvmi_v3_scratch_bytes": ([_i64, _i32, _i32], _i64),
    "kvmi_v3_decompress": ([_vp, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp], ctypes.c_int),
    "kvmi_v3_compress_noalloc": ([_vp, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp], ctypes.c_int),
    "kvmi_rt_encode": ([ctypes.POINTER(RtGeometry), _vp, _i32, _vp, _i64, _vp, _vp, _vp, _i64, _vp], ctypes.c_int),
    "kvmi_rt_decode": ([ctypes.POINTER(RtGeometry), _vp, _i32, _vp, _i64, _vp, _vp, _vp], ctypes.c_int),
    "kvmi_rt_hadamard": ([_vp, _vp, _i64, _i32, _vp], ctypes.c_int),
    "kvmi_rt_scratch_bytes": ([_i32, _i64, _i32, _i32], _i64),
}


class KvmiError(RuntimeError):
    """A host-visible failure of a C-ABI call."""


def load(path: Path = LIB_PATH):
    """Load (once) and return the ctypes library; raises if it was not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not path.exists():
            raise KvmiError(
                f"{path} is missing: build the HIP library with `python -m kvserve_amd.build` "
                "(no CPU fallback exists)")
        lib = ctypes.CDLL(str(path))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        ver = lib.kvmi_abi_version()
        if ver != ABI_VERSION:
            raise KvmiError(f"{path} has ABI version {ver}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc == OK:
        return
    if rc == EINVAL:
        raise ValueError(f"{what}: invalid arguments (KVMI_EINVAL)")
    if rc == ENOSPC:
        raise ValueError(f"{what}: the call needs more scratch than the fixed device array holds (KVMI_ENOSPC)")
    raise KvmiError(f"{what}: failed with code {rc}")
