"""The fixed-profile runtime object (kvserve_v1/compression/runtime/manager.py:31-494).

`CompressionRuntime` owns one byte tensor carved into per-slot arenas, one stream
and one pipeline per slot, the head orders and Hadamard signs, and the optional
encoded-output banks.  The caller owns slot scheduling: it fences the returned
events before reading a slot's buffers or reusing the slot.

Streams keep the default priority (the reference asks for high-priority streams,
manager.py:148-153; prioritised streams are avoided on this platform).
"""

from __future__ import annotations

import hashlib
import json
import logging
from dataclasses import asdict, replace
from typing import Dict, List, Optional, Tuple

import torch

from .. import _lib
from .codec import ANSCodec, EncodedChunk, SlotEvent
from .layout import ALIGNMENT, KVPart, LayerPartLayout
from .memory import (CompressionMemoryPlan, FixedWorkspaceAllocator, metadata_regions, slot_regions)
from .pipeline import CacheBinding, CompressionPipeline, CompressionSlotBuffers
from .spec import round_up

logger = logging.getLogger("kvserve_amd.runtime")


def build_signs(part: LayerPartLayout, order: Tuple[int, ...], seed: int, *, pin_memory: bool = False) -> torch.Tensor:
    """±1 per (output head, channel) (manager.py:31-49).  The row of output head h is
    drawn from torch's CPU generator seeded with seed ^ (layer << 16) ^ original head,
    so a producer and a consumer with the same profile agree bit for bit."""
    out = torch.empty((part.num_heads, part.head_size), dtype=part.dtype, pin_memory=pin_memory)
    generator = torch.Generator(device="cpu")
    for output_head, original_head in enumerate(order):
        generator.manual_seed(seed ^ (part.layer_index << 16) ^ original_head)
        bits = torch.randint(0, 2, (part.head_size,), generator=generator, dtype=torch.int8)
        out[output_head].copy_(bits).mul_(2).sub_(1)
    return out.view(1, 1, part.num_heads, part.head_size)


class _Carver:
    def __init__(self, buffer: torch.Tensor):
        self.buffer = buffer
        self.offset = 0

    def take(self, nbytes: int) -> torch.Tensor:
        self.offset = round_up(self.offset, ALIGNMENT)
        out = self.buffer[self.offset:self.offset + nbytes]
        self.offset += nbytes
        return out


class CompressionRuntime:
    def __init__(self, plan: CompressionMemoryPlan, kv_cache_layout: str, blocks_per_logical: int,
                 device: torch.device, *, codec_factory=None, external_execution: bool = False,
                 execution: str = "both", pipeline_backend: Optional[str] = None):
        if execution not in ("both", "encode", "decode"):
            raise ValueError("Unknown KVServe execution capability")
        if pipeline_backend not in (None, "python", "cpp", "hip"):
            raise ValueError("Unknown KVServe pipeline backend")
        _lib.load()  # the pipeline runs only on the HIP library
        self.execution = execution
        self.plan = plan
        self.config = plan.config
        self.layout = plan.layout
        self.output_slots: List[Tuple[torch.Tensor, torch.Tensor]] = []
        self._output_slots_allocated = False
        self._external_execution = external_execution
        self._metadata_initialized = False
        self.wire_profile: Optional[str] = None
        device = torch.device(device)
        regions = slot_regions(self.config, self.layout, blocks_per_logical)
        meta = metadata_regions(self.config, self.layout)
        per_slot_ws = plan.codec_workspace_bytes // max(self.config.slot_count, 1)
        total = 0
        for size in ([s for _, s in regions] * self.config.slot_count
                     + [per_slot_ws] * (self.config.slot_count if self.config.uses_codec else 0)
                     + [s for _, s in meta]):
            total = round_up(total, ALIGNMENT) + size
        # zeroed once; encode skips clearing the payload of chunks that fill it
        self.bulk = torch.zeros(round_up(total, ALIGNMENT), dtype=torch.uint8, device=device)
        carver = _Carver(self.bulk)
        physical = self.config.logical_blocks_per_chunk * blocks_per_logical
        self.slots: List[CompressionSlotBuffers] = []
        for _ in range(self.config.slot_count):
            taken = {name: carver.take(size) for name, size in regions}
            rows = taken["indices"].numel() // (8 * physical)
            self.slots.append(CompressionSlotBuffers(
                arena_a=taken["arena_a"], arena_b=taken["arena_b"], aux=taken["aux"],
                block_indices=taken["indices"].view(torch.int64).view(rows, physical),
                completion_event=SlotEvent(), host_indices=None, raw_tail=taken["raw_tail"],
                canonical=taken["canonical"] if taken["canonical"].numel() else None))
        self.streams = [torch.cuda.Stream(device=device) for _ in self.slots]
        self.workspace_allocators: List[FixedWorkspaceAllocator] = []
        if self.config.uses_codec:
            self.workspace_allocators = [FixedWorkspaceAllocator(carver.take(per_slot_ws)) for _ in self.slots]
        orders64: Dict[str, torch.Tensor] = {}
        orders32: Dict[str, torch.Tensor] = {}
        signs: Dict[Tuple[str, int], torch.Tensor] = {}
        for key, size in meta:
            view = carver.take(size)
            if key[0] == "order64":
                orders64[key[1]] = view.view(torch.int64)
            elif key[0] == "order32":
                orders32[key[1]] = view.view(torch.int32)
            else:
                part = next(p for p in self.layout.layer_parts if p.layer_name == key[1] and str(p.kv_part) == key[2])
                signs[(key[1], part.kv_part)] = view.view(part.dtype).view(1, 1, part.num_heads, part.head_size)
        self.pipelines: List[CompressionPipeline] = []
        for index, stream in enumerate(self.streams):
            codec = None
            if self.config.uses_codec:
                workspace = self.workspace_allocators[index].buffer
                codec = (ANSCodec(stream, self.layout.packed_bytes_by_part, workspace) if codec_factory is None
                         else codec_factory(stream, self.layout.packed_bytes_by_part, workspace))
            self.pipelines.append(CompressionPipeline(
                layout=self.layout, kv_cache_layout=kv_cache_layout, blocks_per_logical=blocks_per_logical,
                slots=self.slots, codec=codec, stream=stream, signs=signs, head_orders=orders64,
                stages=self.config.pipeline, pipeline_backend=pipeline_backend, order_indices=orders32))
        self.stream = self.streams[0]
        self.head_orders = orders64
        self.signs = signs
        init = torch.cuda.Event()
        init.record(torch.cuda.current_stream(device))
        for stream in self.streams:
            stream.wait_event(init)
        logger.info("KVServe runtime initialized: layout=%s pipeline=%s slots=%d bulk_bytes=%d arena_bytes=%d "
                    "aux_arena_bytes=%d workspace_bytes=%d blocks_per_logical=%d", kv_cache_layout,
                    self.config.pipeline, self.config.slot_count, self.bulk.numel(), self.layout.arena_bytes,
                    self.layout.aux_arena_bytes, plan.codec_workspace_bytes, blocks_per_logical)

    @property
    def fa_group_indices(self):
        return self.layout.fa_group_indices

    # ------------------------------------------------------------------ binding
    def bind_kv_caches(self, kv_caches: Dict[str, CacheBinding], group_indices: Dict[str, int]) -> None:
        """manager.py:229-345: regroup the layout, bind every pipeline, upload the
        head orders and signs once, and hash the wire profile."""
        parts = tuple(replace(p, group_index=group_indices[p.layer_name]) for p in self.layout.layer_parts)
        self.layout = replace(self.layout, layer_parts=parts,
                              fa_group_indices=frozenset(group_indices[p.layer_name] for p in parts),
                              index_rows_by_group={g: r for r, g in
                                                   enumerate(sorted({p.group_index for p in parts}))})
        orders = self.plan.head_selection.local_orders
        if not self._metadata_initialized:
            device = self.bulk.device
            for name, part in {p.layer_name: p for p in parts}.items():
                order = torch.tensor(orders[part.layer_index], dtype=torch.int64)
                self.head_orders[name].copy_(order.to(device))
                self.pipelines[0].order_indices[name].copy_(order.to(torch.int32).to(device))
            if self.config.uses_transformer:
                for part in parts:
                    sign = build_signs(part, orders[part.layer_index], self.config.seed)
                    self.signs[(part.layer_name, part.kv_part)].copy_(sign.to(device))
            identity = {p.layer_name for p in parts if tuple(orders[p.layer_index]) == tuple(range(p.num_heads))}
            torch.cuda.synchronize(device)
            for pipeline in self.pipelines:
                pipeline.identity_orders = identity
            self._metadata_initialized = True
        for pipeline in self.pipelines:
            pipeline.layout = self.layout
            pipeline.bind_kv_caches(kv_caches, prepare_backend=not self._external_execution)
        config = asdict(self.config)
        for key in ("score_path", "slot_count"):
            config.pop(key, None)
        description = asdict(self.layout)
        description["fa_group_indices"] = sorted(self.layout.fa_group_indices)
        wire = {"version": 2, "config": config, "layout": description,
                "cache_layout": self.pipelines[0].kv_cache_layout,
                "blocks_per_logical": self.pipelines[0].blocks_per_logical,
                "orders": {p.layer_name: orders[p.layer_index] for p in parts}}
        self.wire_profile = hashlib.sha256(json.dumps(wire, sort_keys=True, default=str).encode()).hexdigest()
        logger.info("KVServe runtime KV caches bound: layers=%d fa_groups=%s", len(parts) // 2,
                    sorted(self.layout.fa_group_indices))

    # ------------------------------------------------------------------ sizes
    def data_bytes(self, kv_part: int, tokens: Optional[Dict[int, int]] = None) -> int:
        """manager.py:347-366."""
        if self.config.uses_aggregate:
            if tokens is None:
                return self.layout.raw_bytes_by_part[kv_part]
            total = 0
            for part in self.layout.parts(kv_part):
                blocks = (tokens.get(part.group_index, 0) + part.block_size - 1) // part.block_size
                total += blocks * part.num_heads * part.block_size * part.head_size * 2
            return total
        if tokens is not None and not self.layout.has_body(tokens):
            return 0
        return (self.layout.u8_bytes_by_part if "quantizer" in self.config.pipeline
                else self.layout.raw_bytes_by_part)[kv_part]

    def aux_bytes(self, kv_part: int, tokens: Optional[Dict[int, int]] = None) -> int:
        if tokens is not None and not self.layout.has_body(tokens):
            return 0
        return self.layout.aux_bytes_by_part[kv_part] if "quantizer" in self.config.pipeline else 0

    def registered_memory(self) -> Tuple[List[int], List[int]]:
        storage = self.bulk.untyped_storage()
        pointers, sizes = [storage.data_ptr()], [storage.nbytes()]
        for payload, auxiliary in self.output_slots:
            for tensor in (payload, auxiliary):
                size = tensor.numel() * tensor.element_size()
                if size:
                    pointers.append(tensor.data_ptr())
                    sizes.append(size)
        return pointers, sizes

    def allocate_output_slots(self, count: int) -> None:
        """Reserve encoded-output banks before binding (manager.py:383-396)."""
        if type(count) is not int or not 0 <= count <= 16:
            raise ValueError("Encoded output slot count must be 0..16")
        if self._output_slots_allocated or self._metadata_initialized:
            raise RuntimeError("Encoded output banks must be reserved once before binding")
        self.output_slots = [(torch.empty_like(self.slots[0].arena_a), torch.empty_like(self.slots[0].aux))
                             for _ in range(count)]
        extra = sum(t.numel() * t.element_size() for bank in self.output_slots for t in bank)
        self.plan = replace(self.plan, reserved_bytes=self.plan.reserved_bytes + extra)
        self._output_slots_allocated = True

    def _validate_output_bank(self, slot_id, output, auxiliary) -> CompressionSlotBuffers:
        if type(slot_id) is not int or not 0 <= slot_id < len(self.slots):
            raise ValueError("Invalid compression slot")
        slot = self.slots[slot_id]
        pairs = [(slot.arena_a, slot.aux), *self.output_slots]
        if not any(output is payload and auxiliary is aux for payload, aux in pairs):
            raise ValueError("Encoded output and auxiliary must be one Runtime-owned bank")
        return slot

    def _require_execution(self, operation: str) -> None:
        if self.execution not in ("both", operation):
            raise RuntimeError(f"KVServe {self.execution}-only runtime cannot {operation}")

    def _check_slot(self, slot_id) -> None:
        if type(slot_id) is not int or not 0 <= slot_id < len(self.slots):
            raise ValueError("Invalid compression slot")
        if not self._metadata_initialized:
            raise RuntimeError("bind_kv_caches must run before encode / decode")

    # ------------------------------------------------------------------ execution
    def encode_into(self, slot_id, logical_ids_by_group, kv_part, *, valid_tokens_by_group, output,
                    auxiliary) -> EncodedChunk:
        """Encode, then copy payload and aux into a runtime-owned bank (manager.py:406-444)."""
        self._require_execution("encode")
        slot = self._validate_output_bank(slot_id, output, auxiliary)
        stream = self.streams[slot_id]
        aux_bytes = self.aux_bytes(kv_part, valid_tokens_by_group)
        for tensor, capacity in ((output, slot.arena_a.numel()), (auxiliary, aux_bytes)):
            if (tensor.device != slot.arena_a.device or tensor.dtype != torch.uint8 or not tensor.is_contiguous()
                    or tensor.numel() < capacity):
                raise ValueError("Invalid encoded output or auxiliary bank")
        encoded = self.encode(slot_id, logical_ids_by_group, kv_part, valid_tokens_by_group=valid_tokens_by_group)
        encoded.event.synchronize()
        if encoded.raw_tail_bytes:
            raise ValueError("Leased output requires a complete compressed token body")
        size = encoded.codec_bytes
        if not 0 < size <= output.numel():
            raise ValueError("Encoded payload exceeds output bank")
        with torch.cuda.stream(stream):
            if output is not slot.arena_a:
                output[:size].copy_(slot.arena_a[:size], non_blocking=True)
                auxiliary[:aux_bytes].copy_(slot.aux[:aux_bytes], non_blocking=True)
            slot.completion_event.record(stream)
        return EncodedChunk(encoded.array, slot.completion_event, encoded.u8_bytes, payload_bytes=size)

    def encode(self, slot_id: int, logical_ids_by_group: List[List[int]], kv_part: KVPart, *,
               valid_tokens_by_group: Dict[int, int]) -> EncodedChunk:
        self._require_execution("encode")
        self._check_slot(slot_id)
        return self.pipelines[slot_id].encode(slot_id, logical_ids_by_group, kv_part,
                                              valid_tokens_by_group=valid_tokens_by_group)

    def decode(self, slot_id: int, logical_ids_by_group: List[List[int]], kv_part: KVPart, codec_bytes: int,
               u8_bytes: int, *, valid_tokens_by_group: Dict[int, int]) -> torch.cuda.Event:
        """Size checks of manager.py:462-488, then the slot's pipeline."""
        self._require_execution("decode")
        self._check_slot(slot_id)
        if u8_bytes != self.data_bytes(kv_part, valid_tokens_by_group):
            raise ValueError("Compressed chunk has an incompatible decoded size")
        if not 0 <= codec_bytes <= self.slots[slot_id].arena_a.numel():
            raise ValueError("Compressed chunk exceeds receive buffer capacity")
        if "codec" not in self.config.pipeline and codec_bytes != u8_bytes:
            raise ValueError("Unencoded chunk payload size does not match its layout")
        return self.pipelines[slot_id].decode(slot_id, logical_ids_by_group, kv_part, codec_bytes, u8_bytes,
                                              valid_tokens_by_group=valid_tokens_by_group)

    def shutdown(self) -> None:
        for stream in self.streams:
            stream.synchronize()
        self.pipelines.clear()
        self.output_slots.clear()


def create_runtime(plan: CompressionMemoryPlan, cache_layout: str, blocks_per_logical: int, device, *,
                   backend: str = "auto", output_slots: int = 0, graph_lengths=None, execution: str = "both",
                   standard_backend: Optional[str] = None) -> CompressionRuntime:
    """fused_runtime.py:374-413.  Every backend name selects the one HIP runtime:
    its encode is already a fused per-part launch set; `graph_lengths` is accepted
    and unused."""
    if backend not in ("auto", "standard", "fused"):
        raise ValueError("Unknown KVServe execution backend")
    if execution not in ("both", "encode", "decode"):
        raise ValueError("Unknown KVServe execution capability")
    if standard_backend not in (None, "python", "cpp"):
        raise ValueError("Unknown KVServe standard pipeline backend")
    runtime = CompressionRuntime(plan, cache_layout, blocks_per_logical, device, execution=execution,
                                 pipeline_backend=standard_backend)
    runtime.allocate_output_slots(output_slots)
    return runtime
