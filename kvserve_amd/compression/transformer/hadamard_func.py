"""Random-sign normalized FWHT (kvserve_v1/compression/transformer/hadamard_func.py:11-231).

transform: y = bf16(FWHT_fp32(x * s) / sqrt(c));  inverse: x = bf16(FWHT_fp32(y) / sqrt(c)) * s,
per power-of-two chunk c of head_dim (descending, :50-103; c = D for a power of two), with
Rademacher signs s from a CPU torch.Generator seeded base_seed ^ (layer << 16) ^ head
(:33-48, :137-152).  The transform itself runs in the kvmi_hadamard kernel; head_dim is
even, up to 256 (chunks below 16 channels included: 100 = 64 + 32 + 4).
"""

from __future__ import annotations

import torch

from ... import ops
from ...profiles import rademacher_sign_bits


class HadamardTransform:
    def __init__(self, base_seed: int = 0xC0FEBABE):
        self.base_seed = base_seed
        self.signs_cache = {}

    def _get_seed(self, layer_idx: int, head_idx: int) -> int:
        return self.base_seed ^ (layer_idx << 16) ^ head_idx

    def get_rademacher_signs(self, layer_idx: int, num_heads: int, head_dim: int, device, dtype) -> torch.Tensor:
        """[1, 1, H, D] tensor of +-1 (the reference's broadcast shape)."""
        key = (layer_idx, num_heads, head_dim, str(device), dtype)
        if key not in self.signs_cache:
            b = rademacher_sign_bits(self.base_seed, layer_idx, num_heads, head_dim)
            neg = ((b[:, :, None] >> torch.arange(32).numpy()) & 1).reshape(num_heads, -1)[:, :head_dim]
            s = torch.from_numpy(1.0 - 2.0 * neg).to(device=device, dtype=dtype)
            self.signs_cache[key] = s.view(1, 1, num_heads, head_dim)
        return self.signs_cache[key]

    def transform(self, layer_id: int, tensor: torch.Tensor, **kwargs) -> torch.Tensor:
        assert tensor.dim() == 4, f"Expected 4D tensor [num_blocks, block_size, num_heads, head_dim], got {tensor.shape}"
        return ops.hadamard(tensor, layer_id, self.base_seed, inverse=False)

    def inverse(self, layer_id: int, tensor: torch.Tensor, **kwargs) -> torch.Tensor:
        assert tensor.dim() == 4, f"Expected 4D tensor [num_blocks, block_size, num_heads, head_dim], got {tensor.shape}"
        return ops.hadamard(tensor, layer_id, self.base_seed, inverse=True)
