"""Fixed-width bit packing of bounded uint8 symbols on the GPU.

Same contract as kvserve_v1/compression/codec/bitpack_codec.py:72-135: 16-byte
header (magic 0x0150424B, bits, symbol count), LSB-first payload, bits in [1, 8]
(default 8), uint8 device tensors only.  The packing runs in the gfx950 kernels
of kvmi_bitpack_encode / kvmi_bitpack_decode.  Data errors (a symbol wider than
the bit width, a header that does not match) raise RuntimeError with the
reference's assert messages once the stream is synchronized (see kvserve_amd.ops).
"""

from __future__ import annotations

from typing import Any

import torch

from ... import ops
from ..components import Codec


class BitPackCodec(Codec):
    def __init__(self, **kwargs: Any) -> None:
        self.bitpack_bits = 8
        self.update_params(**kwargs)

    def update_params(self, **kwargs: Any) -> None:
        self.bitpack_bits = self._width(kwargs)

    def _width(self, kwargs) -> int:
        bits = kwargs.get("bitpack_bits", self.bitpack_bits)
        if type(bits) is not int or not 1 <= bits <= 8:
            raise ValueError("bitpack_bits must be an integer in [1, 8]")
        return bits

    def encode(self, tensor: torch.Tensor, **kwargs: Any) -> torch.Tensor:
        return ops.bitpack_encode(tensor, self._width(kwargs))

    def decode(self, compressed_data: torch.Tensor, original_dtype: str, original_shape: list, device: str,
               **kwargs: Any) -> torch.Tensor:
        bits = self._width(kwargs)
        if not isinstance(compressed_data, torch.Tensor) or compressed_data.dtype != torch.uint8:
            raise TypeError("BitPackCodec requires a torch.uint8 tensor")
        if not compressed_data.is_cuda:
            raise ValueError("BitPackCodec requires a CUDA tensor")
        if str(original_dtype).removeprefix("torch.") != "uint8":
            raise TypeError("BitPackCodec restores uint8 symbols only")
        target = torch.device(device)
        if target.type != "cuda" or (target.index is not None and target.index != compressed_data.device.index):
            raise ValueError("BitPackCodec decodes on the payload's CUDA device")
        return ops.bitpack_decode(compressed_data, list(original_shape), bits)
