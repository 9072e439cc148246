"""Entropy codec operator: this engine's rANS in the place of nvCOMP ANS.

Contract of kvserve_v1/compression/codec/nvcomp_func.py:54-143: `encode` takes a
device tensor of any dtype and returns compressed uint8 bytes; `decode` takes them
with the original dtype, shape and device and restores the tensor.  nvCOMP is a
closed NVIDIA library (its stream format is unpublished), so the stream is this
engine's own (kvmi_rans_* in include/kvserve_amd.h) and only this engine reads it.

`symbol_bits` (1..8) is the width of the values being coded.  Quantized symbols of
a profile whose largest level count is L take bit_length(L) bits: they are packed
to that width (the bitpack body) and rANS codes the w-bit symbols; the fused
pipeline codes its packed output the same way, so both produce the same stream.
Anything else is coded as bytes (w = 8).
"""

from __future__ import annotations

from typing import Any, Optional

import numpy as np
import torch

from ... import ops
from ..components import Codec


def bitpack_header(bits: int, n: int) -> np.ndarray:
    """The 16-byte bitpack header (bitpack_codec.py:20-47) for n symbols of `bits`."""
    h = np.zeros(16, np.uint8)
    h[0:4] = np.frombuffer(np.uint32(0x0150424B).tobytes(), np.uint8)
    h[4] = bits
    h[8:16] = np.frombuffer(np.uint64(n).tobytes(), np.uint8)
    return h


def unpack_target(n: int, bits: int, device) -> torch.Tensor:
    """A bitpack stream buffer (header written, body to be filled) for n symbols,
    its body 8-byte aligned for the rANS decoder."""
    body = (n * bits + 7) // 8
    buf = torch.empty(16 + max(body, 8), dtype=torch.uint8, device=device)[:16 + body]
    buf[:16].copy_(torch.from_numpy(bitpack_header(bits, n)))
    return buf


class RANSCodec(Codec):
    def __init__(self, **kwargs: Any) -> None:
        self.symbol_bits: Optional[int] = None
        self.update_params(**kwargs)

    def update_params(self, **kwargs: Any) -> None:
        if kwargs.get("symbol_bits") is not None:
            self.symbol_bits = self._width(kwargs["symbol_bits"])

    @staticmethod
    def _width(bits) -> int:
        if type(bits) is not int or not 1 <= bits <= 8:
            raise ValueError("symbol_bits must be an integer in [1, 8]")
        return bits

    def _bits_for(self, dtype: torch.dtype, kwargs) -> int:
        bits = kwargs.get("symbol_bits", self.symbol_bits)
        if bits is None or dtype != torch.uint8:
            return 8
        return self._width(bits)

    def encode(self, tensor: torch.Tensor, **kwargs: Any) -> torch.Tensor:
        if not isinstance(tensor, torch.Tensor) or not tensor.is_cuda:
            raise ValueError("RANSCodec.encode requires a CUDA tensor")
        bits = self._bits_for(tensor.dtype, kwargs)
        flat = tensor.reshape(-1).contiguous().view(torch.uint8)
        if flat.numel() == 0:
            return ops.rans_encode(flat, 0, bits)
        if bits == 8:
            return ops.rans_encode(flat, flat.numel(), 8)
        packed = ops.bitpack_encode(flat, bits)
        return ops.rans_encode(packed[16:], flat.numel(), bits)

    def decode(self, compressed_data: torch.Tensor, original_dtype: str, original_shape: list, device: str,
               **kwargs: Any) -> torch.Tensor:
        if not isinstance(compressed_data, torch.Tensor) or compressed_data.dtype != torch.uint8:
            raise TypeError("RANSCodec decodes a torch.uint8 tensor")
        target = torch.device(device) if device is not None else compressed_data.device
        dev = target if target.type == "cuda" else compressed_data.device
        if dev.type != "cuda":
            raise ValueError("RANSCodec decodes on a CUDA device")
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        dtype = getattr(torch, str(original_dtype).removeprefix("torch."))
        shape = [int(s) for s in original_shape]
        nbytes = int(np.prod(shape, dtype=np.int64)) * torch.empty((), dtype=dtype).element_size()
        src = compressed_data.to(dev)
        bits = self._bits_for(dtype, kwargs)
        if bits == 8:
            out = ops.rans_decode(src, nbytes, 8)
            return out.view(dtype).reshape(shape).to(target)
        buf = unpack_target(nbytes, bits, dev)
        ops.rans_decode(src, nbytes, bits, out=buf[16:])
        return ops.bitpack_decode(buf, shape, bits).to(target)
