"""Arena layout of the fixed-profile runtime (kvserve_v1/compression/runtime/layout.py:16-285).

Peers address a slot's arenas by these offsets, so the numbers are the reference's;
the builder below derives them from the layout rules, stated here:

* Chunk capacity: ``C = logical_blocks_per_chunk`` blocks of ``block_size`` tokens.  A
  (layer, part) of ``h`` heads of size ``d`` holds ``n = C * block_size * h * d``
  elements (``2n`` raw bf16 bytes).
* Arena A holds two raw scratch regions of ``scratch_stride`` bytes each (the largest
  ``2n`` over layers and both head sizes, 256-aligned) that successive layers reuse.
* Arena B: the packed u8 stream starts at ``u8_base = 2 * scratch_stride``; within it
  each part (K = 0, V = 1) lays its layers out back to back in layer order, ``n`` bytes
  each (``u8_offset``), so the K and V streams are two independent sequences.
* Aux arena, per part: layers in order, and within a layer its quantization sections
  (low heads, then high heads; an empty group has no section).  A section stores a min
  table and then a scale table, each starting on a 256-byte boundary and holding one
  bf16 per statistic: ``h_s * d`` on the channel axis, ``C * block_size`` on the token
  axis, one on the tensor axis.  The maxima / inverse scales of the same sections sit at
  the same offsets in the second half of the aux arena (``aux_arena_bytes`` is twice the
  larger part).
* Layer split: the last ``round(0.33 * num_model_layers)`` layers are all-low, the
  others all-high; head split: the selection's low count per layer.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, FrozenSet, List, Literal, Optional, Tuple

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

    @property
    def token_bytes(self) -> int:
        """Raw bf16 bytes of one token of this (layer, part)."""
        return self.num_heads * self.head_size * 2


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
        """Bytes for the partial last block (at most block_size - 1 tokens) of every
        layer of the larger part; the aggregate transport sends whole blocks only."""
        if self.aggregate:
            return 0
        per_part = [sum((p.block_size - 1) * p.token_bytes for p in self.parts(k)) for k in (0, 1)]
        return round_up(max(per_part), ALIGNMENT)

    def raw_tail_bytes(self, kv_part: KVPart, tokens: Dict[int, int]) -> int:
        return sum((tokens[p.group_index] % p.block_size) * p.token_bytes for p in self.parts(kv_part))

    def has_body(self, tokens: Dict[int, int]) -> bool:
        return any(tokens[p.group_index] >= p.block_size for p in self.parts(0))


def _stat_count(axis: str, tokens: int, heads: int, head_size: int) -> int:
    """Statistics (bf16 each) one section stores per table."""
    return {"channel": heads * head_size, "token": tokens}.get(axis, 1)


class _Cursor:
    """Bump allocator over one part's aux half: 256-aligned tables."""

    def __init__(self):
        self.end = 0

    def table(self, nbytes: int) -> int:
        start = round_up(self.end, ALIGNMENT)
        self.end = start + nbytes
        return start


def _check_specs(ordered: List[Tuple[str, CacheSpec]], config: CompressionConfig) -> None:
    if not ordered:
        raise ValueError("KVServe compression requires FullAttention KV caches")
    if len({s.block_size for _, s in ordered}) > 1:
        raise ValueError("KVServe compression requires a common logical block size across FullAttention "
                         "cache groups.")
    for name, s in ordered:
        sizes = (s.head_size, s.head_size_v)
        if config.uses_transformer and not all(d >= 1 and d & (d - 1) == 0 for d in sizes):
            raise ValueError("Hadamard compression requires power-of-two head sizes")
        if s.dtype is not torch.bfloat16:
            raise ValueError(f"KVServe compression currently supports only BF16 KV caches; layer {name} uses "
                             f"{s.dtype}.")


def _low_heads(config: CompressionConfig, layer: int, heads: int, low_head_counts: Dict[int, int],
               num_model_layers: int) -> int:
    if config.split_type == "head":
        return low_head_counts[layer]
    n_low_layers = round(num_model_layers * 0.33)
    return heads if n_low_layers and layer >= num_model_layers - n_low_layers else 0


def build_compression_layout(specs: Dict[str, CacheSpec], config: CompressionConfig,
                             low_head_counts: Dict[int, int], num_model_layers: int,
                             group_indices: Optional[Dict[str, int]] = None) -> CompressionLayout:
    ordered = sorted(specs.items(), key=lambda item: item[1].layer_index)
    _check_specs(ordered, config)
    groups = {name: (group_indices or {}).get(name, 0) for name, _ in ordered}
    chunk_tokens = config.logical_blocks_per_chunk * ordered[0][1].block_size
    # per part: (head size, quantization axis, (low levels, high levels))
    part_rules = ((lambda s: s.head_size, config.axis_key, (config.low_key_num_levels, config.high_key_num_levels)),
                  (lambda s: s.head_size_v, config.axis_value,
                   (config.low_value_num_levels, config.high_value_num_levels)))

    per_part: List[List[LayerPartLayout]] = [[], []]
    raw_total, u8_total, aux_end = [0, 0], [0, 0], [0, 0]
    for kv, (head_size_of, axis, levels) in enumerate(part_rules):
        cursor, u8_at = _Cursor(), 0
        for name, s in ordered:
            d = head_size_of(s)
            elems = chunk_tokens * s.num_kv_heads * d
            low = _low_heads(config, s.layer_index, s.num_kv_heads, low_head_counts, num_model_layers)
            sections, first = [], 0
            for count, lv in zip((low, s.num_kv_heads - low), levels):
                if count:
                    nbytes = 2 * _stat_count(axis, chunk_tokens, count, d)
                    mn = cursor.table(nbytes)
                    sections.append(QuantSection(first, count, lv, axis, mn, cursor.table(nbytes)))
                    first += count
            per_part[kv].append(LayerPartLayout(name, s.layer_index, kv, groups[name], s.block_size, s.num_kv_heads,
                                                d, s.dtype, 0, 2 * elems, u8_at, tuple(sections)))
            u8_at += elems
        raw_total[kv], u8_total[kv], aux_end[kv] = 2 * u8_at, u8_at, round_up(cursor.end, ALIGNMENT)

    scratch_stride = round_up(max(chunk_tokens * s.num_kv_heads * d * 2 for _, s in ordered
                                  for d in (s.head_size, s.head_size_v)), ALIGNMENT)
    u8_base = 2 * scratch_stride
    aggregate = config.uses_aggregate
    quantized = config.uses_quantizer
    packed = u8_total if quantized else raw_total
    if aggregate:
        arena = round_up(max(raw_total), ALIGNMENT)
    else:
        arena = round_up(max(2 * scratch_stride, u8_base + max(packed)), ALIGNMENT)
    group_ids = sorted(set(groups.values()))
    return CompressionLayout(
        layer_parts=tuple(p for pair in zip(*per_part) for p in pair),  # layer order, K before V
        raw_bytes_by_part=tuple(raw_total), u8_bytes_by_part=tuple(u8_total), packed_bytes_by_part=tuple(packed),
        aux_bytes_by_part=tuple(aux_end), arena_bytes=arena, scratch_stride=scratch_stride, u8_base=u8_base,
        aux_arena_bytes=2 * max(aux_end) if quantized else 0, fa_group_indices=frozenset(group_ids),
        index_rows_by_group={g: row for row, g in enumerate(group_ids)}, aggregate=aggregate)
