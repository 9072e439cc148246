"""KVServeQuantizer on gfx950 (kvserve_v1/compression/quantizer/kvserve_quantizer.py:17-294).

Same configuration keys, validation, head / layer masks and metadata dicts as the
reference; the arithmetic (bf16 per-op min-max on each part's axis -- channel, token
or tensor, quantizer_func.py:41-49 -- heads reordered [low, high]) runs in the fused
kernels with the transform switched off and 8-bit raw symbols in native order, i.e.
the operator-level entry of the same code the fused pipeline uses.
"""

from __future__ import annotations

from typing import Any, Dict, Tuple

import torch

from ...engine import FusedKVCodec, Packet, check_packet
from ...profiles import (head_low_mask, layer_low_mask, scores_from_csv, section_profile, tp_head_slice,
                         whole_layer_profile)
from ..components import Quantizer
from .._meta import layer_dict, tables_from_dicts


class KVServeQuantizer(Quantizer):
    supports_out_buffer = False

    def __init__(self, **kwargs) -> None:
        self.model_name = kwargs.get("model_name", "Llama-3.1-8B-Instruct")
        self.hybrid_ratio = kwargs.get("hybrid_ratio", 0.3)
        self.high_key_max_value = kwargs.get("high_key_max_value", 16)
        self.high_value_max_value = kwargs.get("high_value_max_value", 16)
        self.low_key_max_value = kwargs.get("low_key_max_value", 12)
        self.low_value_max_value = kwargs.get("low_value_max_value", 12)
        self.axis_key = kwargs.get("axis_key", "channel")
        self.axis_value = kwargs.get("axis_value", "token")
        self.split_type = kwargs.get("split_type", "head")
        self.tensor_parallel_size = kwargs.get("tensor_parallel_size", 1)
        self.tp_rank = kwargs.get("tp_rank", 0)
        self.validate()
        self.head_scores = scores_from_csv(self.model_name)
        self.head_scores_mask = head_low_mask(self.head_scores, self.hybrid_ratio)
        self.layer_scores_mask = layer_low_mask(self.head_scores.shape[0])
        self._codecs: Dict[tuple, FusedKVCodec] = {}

    def validate(self) -> None:
        """kvserve_quantizer.py:105-141 (same assertions)."""
        assert 0 <= self.hybrid_ratio <= 1, f"hybrid_ratio must be between 0 and 1, got {self.hybrid_ratio}"
        for name in ("low_key_max_value", "low_value_max_value", "high_key_max_value", "high_value_max_value"):
            v = getattr(self, name)
            assert 0 < v < 255, f"{name} must be greater than 0 and less than 255, got {v}"
        assert self.low_key_max_value <= self.high_key_max_value, "low_key_max_value must be less than high_key_max_value"
        assert self.low_value_max_value <= self.high_value_max_value, \
            "low_value_max_value must be less than high_value_max_value"
        assert self.axis_key in ("channel", "token", "tensor"), f"axis_key must be 'channel', 'token' or 'tensor'"
        assert self.axis_value in ("channel", "token", "tensor"), f"axis_value must be 'channel', 'token' or 'tensor'"
        assert self.split_type in ("head", "layer"), f"split_type must be 'head' or 'layer', got {self.split_type}"

    def update_params(self, **kwargs) -> None:
        ratio_changed = "hybrid_ratio" in kwargs and kwargs["hybrid_ratio"] != self.hybrid_ratio
        for key, value in kwargs.items():
            if hasattr(self, key) and not key.startswith("_"):
                setattr(self, key, value)
        if ratio_changed:
            self.head_scores_mask = head_low_mask(self.head_scores, self.hybrid_ratio)
        self.validate()

    # ---------------------------------------------------------------- profiles
    def layer_profile(self, layer_id: int, num_heads: int):
        """Profile of `layer_id` for this worker's `num_heads` KV heads."""
        if self.split_type == "head":
            mask = tp_head_slice(self.head_scores_mask, num_heads, self.tensor_parallel_size, self.tp_rank)
            return section_profile(mask[layer_id], self.high_key_max_value, self.high_value_max_value,
                                   self.low_key_max_value, self.low_value_max_value)
        low = bool(self.layer_scores_mask[layer_id])
        return whole_layer_profile(num_heads, self.low_key_max_value if low else self.high_key_max_value,
                                   self.low_value_max_value if low else self.high_value_max_value, low)

    def _codec(self, H: int, D: int, S: int) -> FusedKVCodec:
        key = (H, D, S, self.axis_key, self.axis_value)
        if key not in self._codecs:
            self._codecs[key] = FusedKVCodec(H, D, S, bits=8, transform=False, layout="native", header=False,
                                             axes=(self.axis_key, self.axis_value))
        return self._codecs[key]

    # ---------------------------------------------------------------- operator API
    def quantize(self, layer_id: int, tensor: torch.Tensor, **kwargs) -> Tuple[torch.Tensor, Dict]:
        """[2, B, S, H, D] bf16 -> (uint8 [2, B, S, H, D] with heads in [low, high]
        order, metadata dict)."""
        if tensor.dim() != 5 or tensor.shape[0] != 2:
            raise ValueError(f"expected [2, num_blocks, block_size, num_heads, head_size], got {tuple(tensor.shape)}")
        x = tensor.contiguous()
        _, B, S, H, D = x.shape
        prof = self.layer_profile(layer_id, H)
        codec = self._codec(H, D, S)
        ids = torch.arange(B, dtype=torch.int32, device=x.device)
        packet = codec.compress([x], ids, [prof], layer_ids=[layer_id], chunk_layers=0)
        check_packet(packet)
        sym = packet.streams[0].view(2, B, S, H, D)
        return sym, layer_dict(packet.kmeta[0], packet.vmeta[0], prof, B, S, packet.axes)

    def dequantize(self, layer_id: int, tensor: torch.Tensor, meta_data: Any, **kwargs) -> torch.Tensor:
        if tensor.dim() != 5 or tensor.shape[0] != 2 or tensor.dtype != torch.uint8:
            raise ValueError("expected uint8 symbols [2, num_blocks, block_size, num_heads, head_size]")
        _, B, S, H, D = tensor.shape
        prof = self.layer_profile(layer_id, H)
        axes = (self.axis_key, self.axis_value)
        kmeta, vmeta = tables_from_dicts([meta_data], H, D, B, S, tensor.device, axes)
        codec = self._codec(H, D, S)
        packet = Packet([tensor.contiguous().view(-1)], [(0, 1)], kmeta, vmeta, [prof], B, S, H, D, 8, codec.seed,
                        False, "native", [layer_id], axes)
        out = torch.empty((2, B, S, H, D), dtype=torch.bfloat16, device=tensor.device)
        codec.decompress(packet, [out], torch.arange(B, dtype=torch.int32, device=tensor.device))
        check_packet(packet)
        return out
