"""KVServeCodec: the `codec_type` switch (kvserve_v1/compression/codec/kvserve_codec.py:23-198).

  "bitpack"                 BitPackCodec (the reference's format, byte for byte)
  "rans"                    RANSCodec, this engine's GPU rANS entropy codec
  "nvcomp" (algorithm ANS)  RANSCodec: the same role as nvCOMP ANS -- a lossless
                            entropy stage over the symbol bytes -- in this engine's
                            own stream format (nvCOMP is closed NVIDIA code)
  "lc"                      RANSCodec, likewise in the place of the external LC build
The other nvCOMP algorithms (LZ4, Zstd, Deflate, GDeflate, Bitcomp, Cascaded) are
rejected with a clear error.  Entropy-coded streams are read only by this engine.
"""

from __future__ import annotations

import torch

from ..components import Codec
from .bitpack_codec import BitPackCodec
from .rans_codec import RANSCodec

_CODECS = ("nvcomp", "lc", "bitpack", "rans")
_NVCOMP_ALGORITHMS = ("ANS", "Bitcomp", "Cascaded", "Deflate", "GDeflate", "LZ4", "Zstd")
ENTROPY_CODECS = ("nvcomp", "lc", "rans")


def is_entropy_codec(codec_config) -> bool:
    return (codec_config or {}).get("codec_type", "nvcomp") in ENTROPY_CODECS


class KVServeCodec(Codec):
    def __init__(self, **kwargs) -> None:
        self.codec_type = kwargs.get("codec_type", "nvcomp")
        self.nvcomp_algorithm = kwargs.get("nvcomp_algorithm", "ANS")
        self._kwargs = dict(kwargs)
        self.codec = None
        self.validate()
        self.codec = self._build()

    def validate(self) -> None:
        if self.codec_type not in _CODECS:
            raise ValueError(f"Invalid codec type: {self.codec_type}, expected one of: {list(_CODECS)}")
        if self.codec_type == "nvcomp":
            if self.nvcomp_algorithm not in _NVCOMP_ALGORITHMS:
                raise ValueError(f"Invalid nvcomp's algorithm: {self.nvcomp_algorithm}")
            if self.nvcomp_algorithm != "ANS":
                raise ValueError(f"nvCOMP {self.nvcomp_algorithm} is not available on the ROCm engine; "
                                 "use nvcomp_algorithm 'ANS' (served by the GPU rANS codec) or codec_type 'bitpack'")

    def _build(self):
        if self.codec_type == "bitpack":
            return BitPackCodec(**self._kwargs)
        return RANSCodec(**self._kwargs)

    def update_params(self, **kwargs) -> None:
        prev = (self.codec_type, self.nvcomp_algorithm)
        self._kwargs.update(kwargs)
        self.codec_type = self._kwargs.get("codec_type", self.codec_type)
        self.nvcomp_algorithm = self._kwargs.get("nvcomp_algorithm", self.nvcomp_algorithm)
        self.validate()
        kind = lambda t: "bitpack" if t == "bitpack" else "entropy"  # noqa: E731
        if self.codec is None or kind(prev[0]) != kind(self.codec_type):
            self.codec = self._build()
        else:
            self.codec.update_params(**kwargs)

    def encode(self, layer_id: int, tensor: torch.Tensor, **kwargs) -> torch.Tensor:
        return self.codec.encode(tensor, **kwargs)

    def decode(self, layer_id: int, compressed_data, original_dtype: str, original_shape: list, device: str,
               **kwargs) -> torch.Tensor:
        return self.codec.decode(compressed_data, original_dtype, original_shape, device, **kwargs)
