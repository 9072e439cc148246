"""Torch-level wrappers of the unit C-ABI entry points (bitpack, gather / scatter,
Hadamard, rANS).  Each enqueues on the current stream of the tensors' device.

Device data errors (a symbol wider than the bit width, a header that does not match)
are reported through a device error word.  By default the wrappers synchronize and
raise, which is the loud failure of the reference's device asserts
(bitpack_codec.py:32, :38, :60); set ``KVSERVE_AMD_CHECK_ERRORS=0`` (or pass
``check=False``) to keep calls asynchronous, and no check is made while a stream is
being captured into a graph.
"""

from __future__ import annotations

import ctypes
import math
import os
from typing import Optional, Sequence

import torch

from . import _lib
from .engine import SIGNS, raise_device_error

HEADER_BYTES = 16


def _check_default() -> bool:
    return os.environ.get("KVSERVE_AMD_CHECK_ERRORS", "1") != "0"


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _maybe_check(err: torch.Tensor, check: Optional[bool]) -> None:
    if check is None:
        check = _check_default()
    if check and not torch.cuda.is_current_stream_capturing():
        raise_device_error(int(err.item()))


def _bits(bits) -> int:
    if type(bits) is not int or not 1 <= bits <= 8:
        raise ValueError("bitpack_bits must be an integer in [1, 8]")
    return bits


def bitpack_encode(sym: torch.Tensor, bits: int, check: Optional[bool] = None) -> torch.Tensor:
    """BitPackCodec.encode (bitpack_codec.py:100-110): 1-D uint8 stream of
    16 + ceil(n*bits/8) bytes for the contiguous flattening of `sym`."""
    bits = _bits(bits)
    if not isinstance(sym, torch.Tensor) or sym.dtype != torch.uint8:
        raise TypeError("BitPackCodec requires a torch.uint8 tensor")
    if not sym.is_cuda:
        raise ValueError("BitPackCodec requires a CUDA tensor")
    src = sym.contiguous()
    n = src.numel()
    out = torch.empty(HEADER_BYTES + (n * bits + 7) // 8, dtype=torch.uint8, device=src.device)
    err = torch.zeros(1, dtype=torch.int32, device=src.device)
    with torch.cuda.device(src.device):
        _lib.check(_lib.load().kvmi_bitpack_encode(src.data_ptr() if n else None, n, bits, out.data_ptr(),
                                                   err.data_ptr(), _stream()), "kvmi_bitpack_encode")
    _maybe_check(err, check)
    return out


def bitpack_decode(stream: torch.Tensor, shape: Sequence[int], bits: int, check: Optional[bool] = None) -> torch.Tensor:
    """BitPackCodec.decode (bitpack_codec.py:112-135): uint8 tensor of `shape`."""
    bits = _bits(bits)
    if not isinstance(stream, torch.Tensor) or stream.dtype != torch.uint8:
        raise TypeError("BitPackCodec requires a torch.uint8 tensor")
    if not stream.is_cuda:
        raise ValueError("BitPackCodec requires a CUDA tensor")
    if any(type(d) is not int or d < 0 for d in shape):
        raise ValueError("original_shape must contain nonnegative integers")
    n = math.prod(shape)
    if stream.numel() != HEADER_BYTES + (n * bits + 7) // 8:
        raise ValueError("BitPackCodec payload length does not match shape and bit width")
    src = stream.contiguous()
    out = torch.empty(list(shape), dtype=torch.uint8, device=src.device)
    err = torch.zeros(1, dtype=torch.int32, device=src.device)
    with torch.cuda.device(src.device):
        _lib.check(_lib.load().kvmi_bitpack_decode(src.data_ptr(), src.numel(), n, bits,
                                                   out.data_ptr() if n else None, err.data_ptr(), _stream()),
                   "kvmi_bitpack_decode")
    _maybe_check(err, check)
    return out


def _pool_layout(pool: torch.Tensor) -> str:
    """"flash" for [2, num_blocks, ...], "kv_adjacent" for [num_blocks, 2, ...] (the
    reference tests the first before the second, kv_utils.py:74-80)."""
    if pool.dim() >= 3 and pool.shape[0] == 2:
        layout = "flash"
    elif pool.dim() >= 3 and pool.shape[1] == 2:
        layout = "kv_adjacent"
    else:
        raise RuntimeError(f"Unsupported KV layout shape: {tuple(pool.shape)}")
    if pool.element_size() != 2 or not pool.is_contiguous() or not pool.is_cuda:
        raise ValueError("paged gather/scatter needs a contiguous 16-bit CUDA KV cache")
    return layout


def _ids(block_ids, num_blocks: int, device) -> torch.Tensor:
    if isinstance(block_ids, torch.Tensor):
        ids = block_ids.to(device=device, dtype=torch.int32).contiguous()
        if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= num_blocks):
            raise IndexError("block id outside the KV cache")
        return ids
    ids_list = [int(b) for b in block_ids]
    if ids_list and (min(ids_list) < 0 or max(ids_list) >= num_blocks):
        raise IndexError("block id outside the KV cache")
    return torch.tensor(ids_list, dtype=torch.int32, device=device)


def gather_blocks(pool: torch.Tensor, block_ids, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """extract_kv_from_layer_by_blocks (kv_utils.py:59-80): pool[:, block_ids] of a
    FlashAttention cache [2, num_blocks, ...], or pool[block_ids] of a [num_blocks, 2,
    ...] cache (MLA / FlashInfer branch), as a new contiguous tensor, or written into
    `out` (contiguous, same shape and dtype; e.g. one layer's slice of a stacked
    tensor) and returned."""
    layout = _pool_layout(pool)
    flash = layout == "flash"
    P = pool.shape[1] if flash else pool.shape[0]
    ids = _ids(block_ids, P, pool.device)
    shape = ((2, ids.numel()) if flash else (ids.numel(), 2)) + tuple(pool.shape[2:])
    if out is None:
        out = torch.empty(shape, dtype=pool.dtype, device=pool.device)
    elif tuple(out.shape) != shape or out.dtype != pool.dtype or out.device != pool.device \
            or not out.is_contiguous():
        raise ValueError(f"gather output must be a contiguous {pool.dtype} tensor of shape {shape} on {pool.device}")
    blk = math.prod(pool.shape[2:])
    lib = _lib.load()
    with torch.cuda.device(pool.device):
        if flash:
            _lib.check(lib.kvmi_gather_blocks(pool.data_ptr(), P * blk, ids.data_ptr(), ids.numel(), blk,
                                              out.data_ptr(), _stream()), "kvmi_gather_blocks")
        else:
            _lib.check(lib.kvmi_gather_blocks_kv_adjacent(pool.data_ptr(), ids.data_ptr(), ids.numel(), blk,
                                                          out.data_ptr(), _stream()), "kvmi_gather_blocks_kv_adjacent")
    return out


def scatter_blocks(pool: torch.Tensor, payload: torch.Tensor, block_ids) -> None:
    """inject_kv_into_layer_by_blocks (kv_utils.py:83-119): pool[:, ids[:nb]] =
    payload for a FlashAttention cache, pool[ids[:nb]] = payload for a [num_blocks, 2,
    ...] cache; nb = the payload's block count."""
    layout = _pool_layout(pool)
    flash = layout == "flash"
    n_ids = block_ids.numel() if isinstance(block_ids, torch.Tensor) else len(block_ids)
    if n_ids == 0:
        return
    P = pool.shape[1] if flash else pool.shape[0]
    ids = _ids(block_ids, P, pool.device)
    src = payload.to(device=pool.device, dtype=pool.dtype).contiguous()
    nb = src.shape[1] if flash else src.shape[0]
    ids = ids[:nb].contiguous()
    if ids.numel() < nb or tuple(src.shape[2:]) != tuple(pool.shape[2:]) or (not flash and src.shape[1] != 2) \
            or (flash and src.shape[0] != 2):
        raise ValueError("payload does not match the KV cache blocks")
    blk = math.prod(pool.shape[2:])
    lib = _lib.load()
    with torch.cuda.device(pool.device):
        if flash:
            _lib.check(lib.kvmi_scatter_blocks(pool.data_ptr(), P * blk, ids.data_ptr(), nb, blk, src.data_ptr(),
                                               _stream()), "kvmi_scatter_blocks")
        else:
            _lib.check(lib.kvmi_scatter_blocks_kv_adjacent(pool.data_ptr(), ids.data_ptr(), nb, blk, src.data_ptr(),
                                                           _stream()), "kvmi_scatter_blocks_kv_adjacent")


def hadamard(x: torch.Tensor, layer_id: int, seed: int, inverse: bool = False,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """HadamardTransform.transform / .inverse (hadamard_func.py:161-231) of a bf16
    tensor [..., H, D] with the signs of (seed, layer_id)."""
    if x.dtype != torch.bfloat16 or not x.is_cuda:
        raise TypeError("the Hadamard transform takes a bf16 CUDA tensor")
    H, D = x.shape[-2], x.shape[-1]
    src = x.contiguous()
    dst = torch.empty_like(src) if out is None else out
    if dst.shape != src.shape or not dst.is_contiguous() or dst.dtype != torch.bfloat16:
        raise ValueError("out must be a contiguous bf16 tensor of the input's shape")
    signs = SIGNS.table(int(seed), [int(layer_id)], H, D, src.device)
    rows = src.numel() // D
    with torch.cuda.device(src.device):
        _lib.check(_lib.load().kvmi_hadamard(src.data_ptr(), dst.data_ptr(), rows, H, D, signs.data_ptr(),
                                             1 if inverse else 0, _stream()), "kvmi_hadamard")
    return dst


def _aligned8(t: torch.Tensor) -> torch.Tensor:
    return t if t.data_ptr() % 8 == 0 else t.clone()


def rans_encode_batch(items: Sequence[tuple], bits: int) -> list:
    """Entropy-code several packed symbol buffers [(packed, n), ...] of one width in one
    launch per kernel -- the codec stage's nvCOMP ANS encode (nvcomp_func.py:54-95)
    for every stream of a request.  Synchronizes once to learn the stream lengths;
    returns views of the streams' bytes."""
    bits = _bits(bits)
    lib = _lib.load()
    jobs = (_lib.RansEncJob * max(1, len(items)))()
    keep = []
    for i, (packed, n) in enumerate(items):
        if packed.dtype != torch.uint8 or packed.dim() != 1 or not packed.is_cuda:
            raise TypeError("rans_encode takes 1-D uint8 CUDA tensors")
        n = int(n)
        if packed.numel() < (n * bits + 7) // 8:
            raise ValueError("packed buffer is shorter than n symbols of this width")
        cap, scr = int(lib.kvmi_rans_max_bytes(n, bits)), int(lib.kvmi_rans_scratch_bytes(n, bits))
        if cap < 0 or scr < 0:
            raise ValueError("invalid rANS size or width")
        dev = packed.device
        src = _aligned8(packed.contiguous())
        out = torch.empty((cap + 7) // 8 * 8, dtype=torch.uint8, device=dev)
        scratch = torch.empty(max(scr, 8), dtype=torch.uint8, device=dev)
        length = torch.empty(1, dtype=torch.int64, device=dev)
        jobs[i] = _lib.RansEncJob(src.data_ptr() if n else None, n, out.data_ptr(), out.numel(), scratch.data_ptr(),
                                  scratch.numel(), length.data_ptr())
        keep.append((src, out, scratch, length))
    if not items:
        return []
    devs = {k[1].device for k in keep}
    if len(devs) != 1:
        raise ValueError("one rANS batch runs on one device")
    with torch.cuda.device(keep[0][1].device):
        _lib.check(lib.kvmi_rans_encode_batch(jobs, len(items), bits, _stream()), "kvmi_rans_encode_batch")
    lengths = torch.cat([k[3] for k in keep]).tolist()
    return [k[1][:int(n)] for k, n in zip(keep, lengths)]


def rans_encode(packed: torch.Tensor, n: int, bits: int) -> torch.Tensor:
    """One stream of rans_encode_batch."""
    return rans_encode_batch([(packed, n)], bits)[0]


def rans_decode_batch(items: Sequence[tuple], bits: int, check: Optional[bool] = None) -> list:
    """Inverse of rans_encode_batch for [(stream, n[, out]), ...] in one launch: the
    ceil(n*bits/8) packed bytes of each stream (into `out`, an 8-byte aligned uint8
    tensor of at least that size, when given) -- the codec stage's nvCOMP ANS decode
    (nvcomp_func.py:97-143)."""
    bits = _bits(bits)
    jobs = (_lib.RansDecJob * max(1, len(items)))()
    outs, keep = [], []
    for i, item in enumerate(items):
        stream, n = item[0], int(item[1])
        out = item[2] if len(item) > 2 else None
        if stream.dtype != torch.uint8 or stream.dim() != 1 or not stream.is_cuda:
            raise TypeError("rans_decode takes 1-D uint8 CUDA tensors")
        if stream.numel() < 32:
            raise ValueError("rANS stream is shorter than its header")
        nbytes = (n * bits + 7) // 8
        if out is None:
            out = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=stream.device)[:nbytes]
        elif out.dtype != torch.uint8 or not out.is_contiguous() or out.numel() < nbytes or out.data_ptr() % 8:
            raise ValueError("out must be a contiguous, 8-byte aligned uint8 tensor of ceil(n*bits/8) bytes")
        src = _aligned8(stream.contiguous())
        jobs[i] = _lib.RansDecJob(src.data_ptr(), src.numel(), n, out.data_ptr())
        keep.append(src)
        outs.append(out)
    if not items:
        return []
    dev = keep[0].device
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.load().kvmi_rans_decode_batch(jobs, len(items), bits, err.data_ptr(), _stream()),
                   "kvmi_rans_decode_batch")
    _maybe_check(err, check)
    return outs


def rans_decode(stream: torch.Tensor, n: int, bits: int, out: Optional[torch.Tensor] = None,
                check: Optional[bool] = None) -> torch.Tensor:
    """One stream of rans_decode_batch."""
    return rans_decode_batch([(stream, n) if out is None else (stream, n, out)], bits, check)[0]
