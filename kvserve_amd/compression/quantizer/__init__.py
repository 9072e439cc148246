"""Quantizers: KVServe's hybrid min-max quantizer and the fused Hadamard quantizer
(impl "tilelang_fused") on gfx950."""
from .fused_quantizer import FusedHadamardQuantizer, TileLangFusedQuantizer
from .kvserve_quantizer import KVServeQuantizer

__all__ = ["FusedHadamardQuantizer", "KVServeQuantizer", "TileLangFusedQuantizer"]
