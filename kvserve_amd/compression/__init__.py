"""Drop-in mirror of kvserve_v1.compression for the MI355X engine.

  KVCompressionAdapter            connector-facing adapter and operator registry
  CompressionManager              operator-by-operator pipeline
  FusedCompressionManager         the fused gfx950 pipeline (default when a quantizer runs)
  KVServeTransformer / KVServeQuantizer / KVServeCodec / BitPackCodec   operators
  CompressedWire, build_wire, restore_from_wire                         transport bundle
"""

from .codec import BitPackCodec, KVServeCodec
from .components import Codec, Quantizer, Transformer
from .compression_manager import (DEFAULT_COMPRESSION_CONFIG, CompressedKVData, CompressionConfig,
                                  CompressionManager, FusedCompressionManager, get_default_compression_config)
from .manager import KVCompressionAdapter
from .quantizer import KVServeQuantizer
from .transformer import HadamardTransform, KVServeTransformer
from .wire import CompressedWire, build_wire, restore_from_wire

__all__ = [
    "BitPackCodec", "KVServeCodec", "Codec", "Quantizer", "Transformer", "DEFAULT_COMPRESSION_CONFIG",
    "CompressedKVData", "CompressionConfig", "CompressionManager", "FusedCompressionManager",
    "get_default_compression_config", "KVCompressionAdapter", "KVServeQuantizer", "HadamardTransform",
    "KVServeTransformer", "CompressedWire", "build_wire", "restore_from_wire",
]
