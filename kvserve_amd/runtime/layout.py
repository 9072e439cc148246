"""Arena layout of the fixed-profile runtime (kvserve_v1/compression/runtime/layout.py:16-285).

The offsets are the reference's: per KV part, every layer's packed rows at a
``u8_offset`` sized for the full chunk capacity; per quantization section, a min and a
scale array at 256-byte aligned ``aux`` offsets (channel axis: [heads, head_size];
token axis: one per token; tensor axis: one), the aux arena holding these in its first
half and the maxima / inverses at the same offsets in its second half.  Callers and
peers address the arenas through these numbers, so they are kept identical.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from math import prod
from typing import Dict, FrozenSet, Literal, Optional, Tuple

import torch

from .config import CompressionConfig, QuantAxis
from .spec import CacheSpec, round_up

KVPart = Literal[0, 1]
ALIGNMENT = 256


@dataclass(frozen=True)
class QuantSection:
    head_start: int
    head_count: int
    num_levels: int
    axis: QuantAxis
    aux_min_offset: int
    aux_scale_offset: int


@dataclass(frozen=True)
class LayerPartLayout:
    layer_name: str
    layer_index: int
    kv_part: KVPart
    group_index: int
    block_size: int
    num_heads: int
    head_size: int
    dtype: torch.dtype
    raw_offset: int
    raw_bytes: int
    u8_offset: int
    sections: Tuple[QuantSection, ...]


@dataclass(frozen=True)
class CompressionLayout:
    layer_parts: Tuple[LayerPartLayout, ...]
    raw_bytes_by_part: Tuple[int, int]
    u8_bytes_by_part: Tuple[int, int]
    packed_bytes_by_part: Tuple[int, int]
    aux_bytes_by_part: Tuple[int, int]
    arena_bytes: int
    scratch_stride: int
    u8_base: int
    aux_arena_bytes: int
    fa_group_indices: FrozenSet[int]
    index_rows_by_group: Dict[int, int] = field(default_factory=dict)
    aggregate: bool = False

    def parts(self, kv_part: int) -> Tuple[LayerPartLayout, ...]:
        return tuple(p for p in self.layer_parts if p.kv_part == kv_part)

    @property
    def raw_tail_capacity(self) -> int:
        """bf16 bytes of at most block_size - 1 tokens per layer of the larger part."""
        if self.aggregate:
            return 0
        return round_up(max(sum((p.block_size - 1) * p.num_heads * p.head_size * 2 for p in self.parts(k))
                            for k in (0, 1)), ALIGNMENT)

    def raw_tail_bytes(self, kv_part: KVPart, tokens: Dict[int, int]) -> int:
        return sum((tokens[p.group_index] % p.block_size) * p.num_heads * p.head_size * 2
                   for p in self.parts(kv_part))

    def has_body(self, tokens: Dict[int, int]) -> bool:
        return any(tokens[p.group_index] >= p.block_size for p in self.parts(0))


def _reduction_shape(axis: str, shape: Tuple[int, int, int, int]) -> Tuple[int, ...]:
    blocks, tokens, heads, head_size = shape
    if axis == "channel":
        return (1, 1, heads, head_size)
    if axis == "token":
        return (blocks, tokens, 1, 1)
    return (1, 1, 1, 1)


def _split_counts(config: CompressionConfig, layer_index: int, num_heads: int, low_head_counts: Dict[int, int],
                  num_model_layers: int) -> Tuple[int, int]:
    """(low heads, high heads): head split from the selection; layer split makes the
    last round(0.33 L) layers low (layout.py:110-124)."""
    if config.split_type == "head":
        low = low_head_counts[layer_index]
        return low, num_heads - low
    n_low = round(num_model_layers * 0.33)
    is_low = n_low > 0 and layer_index >= num_model_layers - n_low
    return (num_heads, 0) if is_low else (0, num_heads)


def build_compression_layout(specs: Dict[str, CacheSpec], config: CompressionConfig,
                             low_head_counts: Dict[int, int], num_model_layers: int,
                             group_indices: Optional[Dict[str, int]] = None) -> CompressionLayout:
    group_indices = group_indices or {}
    items = sorted(specs.items(), key=lambda kv: kv[1].layer_index)
    if not items:
        raise ValueError("Mooncake compression requires FullAttention KV caches")
    if len({s.block_size for _, s in items}) != 1:
        raise ValueError("Mooncake compression requires a common logical block size across FullAttention "
                         "cache groups.")
    for name, spec in items:
        if config.uses_transformer and any(sz < 1 or sz & (sz - 1) for sz in (spec.head_size, spec.head_size_v)):
            raise ValueError("Hadamard compression requires power-of-two head sizes")
        if spec.dtype is not torch.bfloat16:
            raise ValueError(f"Mooncake compression currently supports only BF16 KV caches; layer {name} uses "
                             f"{spec.dtype}.")
    cb = config.logical_blocks_per_chunk
    scratch_stride = round_up(max(cb * s.block_size * s.num_kv_heads * hs * 2 for _, s in items
                                  for hs in (s.head_size, s.head_size_v)), ALIGNMENT)
    u8_base = round_up(2 * scratch_stride, ALIGNMENT)
    raw_off, u8_off, aux_off = [0, 0], [0, 0], [0, 0]
    parts, groups = [], set()
    for name, spec in items:
        li = spec.layer_index
        gi = group_indices.get(name, 0)
        groups.add(gi)
        low, high = _split_counts(config, li, spec.num_kv_heads, low_head_counts, num_model_layers)
        for kv, hs, axis, lo_lv, hi_lv in ((0, spec.head_size, config.axis_key, config.low_key_num_levels,
                                             config.high_key_num_levels),
                                            (1, spec.head_size_v, config.axis_value, config.low_value_num_levels,
                                             config.high_value_num_levels)):
            numel = cb * spec.block_size * spec.num_kv_heads * hs
            sections, start = [], 0
            for count, levels in ((low, lo_lv), (high, hi_lv)):
                if count == 0:
                    continue
                nbytes = prod(_reduction_shape(axis, (cb, spec.block_size, count, hs))) * 2
                mo = round_up(aux_off[kv], ALIGNMENT)
                so = round_up(mo + nbytes, ALIGNMENT)
                aux_off[kv] = so + nbytes
                sections.append(QuantSection(start, count, levels, axis, mo, so))
                start += count
            parts.append(LayerPartLayout(name, li, kv, gi, spec.block_size, spec.num_kv_heads, hs, spec.dtype, 0,
                                         numel * 2, u8_off[kv], tuple(sections)))
            raw_off[kv] += numel * 2
            u8_off[kv] += numel
    raw_by = (raw_off[0], raw_off[1])
    u8_by = (u8_off[0], u8_off[1])
    aux_by = (round_up(aux_off[0], ALIGNMENT), round_up(aux_off[1], ALIGNMENT))
    aggregate = "aggregate" in config.pipeline
    quant = "quantizer" in config.pipeline and not aggregate
    packed_by = u8_by if quant else raw_by
    arena = (round_up(max(*raw_by), ALIGNMENT) if aggregate
             else round_up(max(2 * scratch_stride, u8_base + max(*packed_by)), ALIGNMENT))
    return CompressionLayout(layer_parts=tuple(parts), raw_bytes_by_part=raw_by, u8_bytes_by_part=u8_by,
                             packed_bytes_by_part=packed_by, aux_bytes_by_part=aux_by, arena_bytes=arena,
                             scratch_stride=scratch_stride, u8_base=u8_base,
                             aux_arena_bytes=0 if (aggregate or not quant) else 2 * max(aux_by),
                             fa_group_indices=frozenset(groups),
                             index_rows_by_group={g: r for r, g in enumerate(sorted(groups))}, aggregate=aggregate)
