"""KVServeCodec: the `codec_type` switch (kvserve_v1/compression/codec/kvserve_codec.py:158-341).

Only "bitpack" exists on this engine.  "nvcomp" wraps NVIDIA's closed nvCOMP
library and "lc" an external CUDA build; both are entropy codecs outside the
bitpack hot path, so they are rejected with a clear message.
"""

from __future__ import annotations

import torch

from ..components import Codec
from .bitpack_codec import BitPackCodec

_CODECS = ("nvcomp", "lc", "bitpack")


class KVServeCodec(Codec):
    def __init__(self, **kwargs) -> None:
        self.codec_type = kwargs.get("codec_type", "nvcomp")
        self._kwargs = dict(kwargs)
        self.codec = None
        self.validate()
        self.codec = BitPackCodec(**kwargs)

    def validate(self) -> None:
        if self.codec_type not in _CODECS:
            raise ValueError(f"Invalid codec type: {self.codec_type}, expected one of: {list(_CODECS)}")
        if self.codec_type != "bitpack":
            raise ValueError(f"codec_type '{self.codec_type}' is not available on the ROCm engine; use 'bitpack'")

    def update_params(self, **kwargs) -> None:
        self._kwargs.update(kwargs)
        self.codec_type = self._kwargs.get("codec_type", self.codec_type)
        self.validate()
        self.codec.update_params(**kwargs)

    def encode(self, layer_id: int, tensor: torch.Tensor, **kwargs) -> torch.Tensor:
        return self.codec.encode(tensor, **kwargs)

    def decode(self, layer_id: int, compressed_data, original_dtype: str, original_shape: list, device: str,
               **kwargs) -> torch.Tensor:
        return self.codec.decode(compressed_data, original_dtype, original_shape, device, **kwargs)
