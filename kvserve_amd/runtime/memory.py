"""Memory plan of the fixed-profile runtime (kvserve_v1/compression/runtime/memory.py:72-453).

Sizes every buffer a runtime owns before the KV cache is allocated: the layout's
arenas, the transformed-row scratch of the quantizer, the codec's output capacity
and scratch (this engine's rANS: known in closed form, so nothing is probed on the
device), head orders and signs.  One runtime carves all of it from a single byte
tensor in the order `slot_regions` lists.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass, replace
from typing import Dict, List, Optional, Tuple

import torch

from .. import _lib
from .config import CompressionConfig
from .layout import ALIGNMENT, CompressionLayout, build_compression_layout
from .scores import HeadSelection, build_head_selection, load_scores
from .spec import CacheSpec, round_up

logger = logging.getLogger("kvserve_amd.runtime")


@dataclass(frozen=True)
class CompressionMemoryPlan:
    config: CompressionConfig
    layout: CompressionLayout
    head_selection: HeadSelection
    codec_workspace_bytes: int
    codec_max_output_bytes: Tuple[int, int]
    blocks_per_logical: int
    metadata_bytes: int
    retained_driver_bytes: int
    guard_bytes: int
    reserved_bytes: int


class FixedWorkspaceAllocator:
    """The codec scratch of one slot.  The rANS kernels take it whole; nothing is
    allocated while a chunk is coded (memory.py:417-453 serves nvCOMP's requests
    from the same kind of fixed buffer)."""

    def __init__(self, buffer: torch.Tensor):
        self.buffer = buffer


def codec_capacity(packed_bytes: int) -> Tuple[int, int]:
    """(stream capacity, scratch bytes) of the rANS codec over `packed_bytes` bytes."""
    lib = _lib.load()
    return int(lib.kvmi_rans_max_bytes(packed_bytes, 8)), int(lib.kvmi_rans_scratch_bytes(packed_bytes, 8))


def canonical_bytes(layout: CompressionLayout) -> int:
    """Scratch of the quantizing encode (transformed rows or per-workgroup column
    statistics, kvmi_rt_scratch_bytes) for every layer of the larger KV part at the
    chunk's full capacity."""
    lib = _lib.load()
    per_part = []
    for k in (0, 1):
        total = 0
        for p in layout.parts(k):
            rows = p.raw_bytes // (2 * p.num_heads * p.head_size)
            total += int(lib.kvmi_rt_scratch_bytes(1, rows, p.num_heads, p.head_size))
        per_part.append(total)
    return max(per_part)


def index_rows(layout: CompressionLayout) -> int:
    return max(len(layout.index_rows_by_group), len({p.layer_name for p in layout.layer_parts}), 1)


def slot_regions(config: CompressionConfig, layout: CompressionLayout, blocks_per_logical: int) -> List[Tuple[str, int]]:
    """Byte regions of one slot, in carving order."""
    physical = config.logical_blocks_per_chunk * blocks_per_logical
    return [("arena_a", layout.arena_bytes),
            ("arena_b", 0 if config.uses_aggregate else layout.arena_bytes),
            ("aux", layout.aux_arena_bytes),
            ("raw_tail", layout.raw_tail_capacity),
            ("indices", physical * index_rows(layout) * 8),
            ("canonical", canonical_bytes(layout) if config.uses_quantizer else 0)]


def metadata_regions(config: CompressionConfig, layout: CompressionLayout) -> List[Tuple[Tuple[str, ...], int]]:
    """Head orders (int64 for callers, int32 for the kernels) and signs, shared by all slots."""
    regions: List[Tuple[Tuple[str, ...], int]] = []
    seen = set()
    for p in layout.layer_parts:
        if p.layer_name not in seen:
            seen.add(p.layer_name)
            regions.append((("order64", p.layer_name), p.num_heads * 8))
            regions.append((("order32", p.layer_name), p.num_heads * 4))
        if config.uses_transformer:
            regions.append((("signs", p.layer_name, str(p.kv_part)), p.num_heads * p.head_size * 2))
    return regions


def _carved(sizes) -> int:
    total = 0
    for size in sizes:
        total = round_up(total, ALIGNMENT) + size
    return round_up(total, ALIGNMENT)


def build_memory_plan(config: CompressionConfig, specs: Dict[str, CacheSpec], *, blocks_per_logical: int = 1,
                      tp_size: int = 1, tp_rank: int = 0, num_layers: int = 0,
                      device: Optional[torch.device] = None,
                      warm_cpp_backend: bool = False) -> Optional[CompressionMemoryPlan]:
    """Same signature and decisions as memory.py:233-403; `device` and
    `warm_cpp_backend` are accepted for callers and unused (nothing is probed)."""
    if not config.available:
        return None
    if config.is_raw_aggregate:
        logger.info("KVServe raw_aggregate transport: slot_count=%d logical_blocks_per_chunk=%d",
                    config.slot_count, config.logical_blocks_per_chunk)
    scores = (load_scores(config.score_path)
              if config.uses_quantizer and config.split_type == "head" and config.score_path else None)
    planning = config if "quantizer" in config.pipeline else replace(config, split_type="layer")
    selection = build_head_selection(specs, planning, tp_rank, tp_size, scores)
    num_layers = num_layers or max(selection.low_counts, default=-1) + 1
    layout = build_compression_layout(specs, planning, selection.low_counts, num_layers)
    if any(p.block_size % blocks_per_logical for p in layout.layer_parts):
        raise ValueError("Logical attention blocks must contain whole kernel blocks.")
    if config.uses_codec:
        caps = [codec_capacity(n) for n in layout.packed_bytes_by_part]
        max_out = (caps[0][0], caps[1][0])
        per_slot = round_up(max(c[1] for c in caps), ALIGNMENT)
        layout = replace(layout, arena_bytes=round_up(max(layout.arena_bytes, *max_out), ALIGNMENT))
    else:
        max_out, per_slot = (0, 0), 0
    workspace = per_slot * config.slot_count
    metadata = _carved(size for _, size in metadata_regions(config, layout))
    slot = _carved(size for _, size in slot_regions(config, layout, blocks_per_logical))
    reserved = config.slot_count * slot + workspace + metadata
    logger.info("KVServe runtime plan: pipeline=%s slots=%d arena=%d aux=%d workspace=%d reserved=%d",
                config.pipeline, config.slot_count, layout.arena_bytes, layout.aux_arena_bytes, workspace, reserved)
    return CompressionMemoryPlan(config=config, layout=layout, head_selection=selection,
                                 codec_workspace_bytes=workspace, codec_max_output_bytes=max_out,
                                 blocks_per_logical=blocks_per_logical, metadata_bytes=metadata,
                                 retained_driver_bytes=0, guard_bytes=0, reserved_bytes=reserved)
