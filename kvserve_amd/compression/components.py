"""Operator interfaces of the compression pipeline (kvserve_v1/compression/components.py:11-106).

The concrete calling convention -- the one CompressionManager uses -- passes the
layer index first (compression_manager.py:277-330, :600-634):
  transform(layer_id, x[2,B,S,H,D], **cfg) -> same shape and dtype
  inverse(layer_id, y, **cfg) -> x
  quantize(layer_id, x, **cfg) -> (uint8 symbols, metadata dict)
  dequantize(layer_id, q, meta, **cfg) -> bf16
  encode(layer_id, uint8 tensor, **cfg) -> 1-D uint8 device tensor
  decode(layer_id, payload, dtype_str, shape_list, device_str, **cfg) -> tensor
"""

from abc import ABC, abstractmethod


class Transformer(ABC):
    @abstractmethod
    def transform(self, layer_id, tensor, **kwargs):
        ...

    @abstractmethod
    def inverse(self, layer_id, tensor, **kwargs):
        ...


class Quantizer(ABC):
    @abstractmethod
    def quantize(self, layer_id, tensor, **kwargs):
        ...

    @abstractmethod
    def dequantize(self, layer_id, tensor, meta_data, **kwargs):
        ...


class Codec(ABC):
    @abstractmethod
    def encode(self, layer_id, tensor, **kwargs):
        ...

    @abstractmethod
    def decode(self, layer_id, compressed_data, original_dtype, original_shape, device, **kwargs):
        ...
