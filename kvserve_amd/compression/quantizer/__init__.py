"""Quantizers: KVServe's hybrid min-max quantizer on gfx950."""
from .kvserve_quantizer import KVServeQuantizer

__all__ = ["KVServeQuantizer"]
