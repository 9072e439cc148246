"""KVServeTransformer (kvserve_v1/compression/transformer/kvserve_transformer.py:7-51).

Only transform_type="hadamard" runs on this engine (the DCT / Haar rotations of
orthogonal.py are outside the hot-path profile).  K and V of a layer
[2, B, S, H, D] share the layer's signs.
"""

from __future__ import annotations

import torch

from ... import ops
from ..components import Transformer
from .hadamard_func import HadamardTransform

DEFAULT_SEED = 0x3333  # kvserve_transformer.py:22


class KVServeTransformer(Transformer):
    def __init__(self, **kwargs):
        self.transform_type = None
        self.seed = None
        self.transformer = None
        self.update_params(**kwargs)

    def validate(self):
        if self.transform_type != "hadamard":
            raise ValueError(f"Invalid transform type: {self.transform_type}")
        if type(self.seed) is not int:
            raise ValueError("seed must be an integer")

    def update_params(self, **kwargs):
        kind = kwargs.get("transform_type", self.transform_type or "hadamard")
        seed = kwargs.get("seed", self.seed if self.seed is not None else DEFAULT_SEED)
        if kind in ("dct", "haar"):
            raise ValueError(f"transform_type '{kind}' is not available on the ROCm engine; use 'hadamard'")
        if kind != "hadamard" or type(seed) is not int:
            raise ValueError("Expected hadamard/dct/haar and an integer seed")
        if (kind, seed) == (self.transform_type, self.seed):
            return
        self.transform_type, self.seed, self.transformer = kind, seed, HadamardTransform(seed)

    def transform(self, layer_id: int, tensor: torch.Tensor, **kwargs) -> torch.Tensor:
        return ops.hadamard(tensor, layer_id, self.seed, inverse=False)

    def inverse(self, layer_id: int, tensor: torch.Tensor, **kwargs) -> torch.Tensor:
        return ops.hadamard(tensor, layer_id, self.seed, inverse=True)
