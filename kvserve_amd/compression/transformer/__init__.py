"""Transforms: the random-sign Hadamard transform on gfx950 (transform_type="hadamard")."""
from .hadamard_func import HadamardTransform
from .kvserve_transformer import KVServeTransformer

__all__ = ["HadamardTransform", "KVServeTransformer"]
