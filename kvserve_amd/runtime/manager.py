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


class _OutputBank:
    """A payload / auxiliary tensor pair that an encode may leave its result in."""

    def __init__(self, payload: torch.Tensor, aux: torch.Tensor, owner: Optional[int]):
        self.payload, self.aux = payload, aux
        self.owner = owner  # slot index of a slot's own arena pair; None for a lease

    def spans(self) -> List[Tuple[int, int]]:
        return [(t.data_ptr(), t.numel() * t.element_size()) for t in (self.payload, self.aux) if t.numel()]

    def holds(self, device: torch.device, payload_bytes: int, aux_bytes: int) -> bool:
        """Both tensors are contiguous uint8 on `device` with room for the chunk."""
        return all(t.device == device and t.dtype == torch.uint8 and t.is_contiguous() and t.numel() >= need
                   for t, need in ((self.payload, payload_bytes), (self.aux, aux_bytes)))

    def take_from(self, slot: CompressionSlotBuffers, payload_bytes: int, aux_bytes: int) -> None:
        """Copy a finished chunk out of `slot`'s arenas (enqueued on the current stream)."""
        self.payload[:payload_bytes].copy_(slot.arena_a[:payload_bytes], non_blocking=True)
        self.aux[:aux_bytes].copy_(slot.aux[:aux_bytes], non_blocking=True)


class _BankTable:
    """The runtime-owned output banks: every slot's own arena pair plus the leases.
    Banks are found by the identity of both tensors, so a view, a slice or a copy of
    a bank (which could alias a live arena) is never accepted."""

    def __init__(self, slots: List[CompressionSlotBuffers]):
        self._by_identity: Dict[Tuple[int, int], _OutputBank] = {}
        self.leases: List[_OutputBank] = []
        self.sealed = False
        for index, slot in enumerate(slots):
            self._enter(_OutputBank(slot.arena_a, slot.aux, index))

    def _enter(self, bank: _OutputBank) -> None:
        self._by_identity[(id(bank.payload), id(bank.aux))] = bank

    def find(self, payload, aux) -> Optional[_OutputBank]:
        bank = self._by_identity.get((id(payload), id(aux)))
        return bank if bank is not None and bank.payload is payload and bank.aux is aux else None

    def reserve(self, count: int, like: CompressionSlotBuffers) -> int:
        """Allocate `count` leases shaped like `like`'s arenas; returns their bytes."""
        self.sealed = True
        for _ in range(count):
            bank = _OutputBank(torch.empty_like(like.arena_a), torch.empty_like(like.aux), None)
            self.leases.append(bank)
            self._enter(bank)
        return sum(size for bank in self.leases for _, size in bank.spans())

    def release_leases(self) -> None:
        for bank in self.leases:
            self._by_identity.pop((id(bank.payload), id(bank.aux)), None)
        self.leases.clear()


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
        self._banks = _BankTable(self.slots)
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
    @property
    def _quantized(self) -> bool:
        return "quantizer" in self.config.pipeline

    def data_bytes(self, kv_part: int, tokens: Optional[Dict[int, int]] = None) -> int:
        """Stored (decoded) bytes of one chunk of `kv_part` (manager.py:343-359):
        `tokens` maps FA group -> valid tokens, None means a full chunk."""
        layout = self.layout
        if self.config.uses_aggregate:
            # the aggregate transport ships every layer's whole raw blocks
            if tokens is None:
                return layout.raw_bytes_by_part[kv_part]
            return sum(p.block_size * p.token_bytes * -(-tokens.get(p.group_index, 0) // p.block_size)
                       for p in layout.parts(kv_part))
        if not self._has_body(tokens):
            return 0
        return (layout.u8_bytes_by_part if self._quantized else layout.raw_bytes_by_part)[kv_part]

    def aux_bytes(self, kv_part: int, tokens: Optional[Dict[int, int]] = None) -> int:
        """Quantization-table bytes of one chunk (manager.py:361-368)."""
        return self.layout.aux_bytes_by_part[kv_part] if self._quantized and self._has_body(tokens) else 0

    def _has_body(self, tokens: Optional[Dict[int, int]]) -> bool:
        return tokens is None or self.layout.has_body(tokens)

    # ------------------------------------------------------------------ output banks
    @property
    def output_slots(self) -> List[Tuple[torch.Tensor, torch.Tensor]]:
        """The leased (payload, auxiliary) banks, in reservation order."""
        return [(bank.payload, bank.aux) for bank in self._banks.leases]

    def registered_memory(self) -> Tuple[List[int], List[int]]:
        """Device ranges a transport registers (manager.py:370-379): the bulk
        allocation, then every non-empty lease tensor."""
        storage = self.bulk.untyped_storage()
        spans = [(storage.data_ptr(), storage.nbytes())]
        spans += [span for bank in self._banks.leases for span in bank.spans()]
        return [ptr for ptr, _ in spans], [size for _, size in spans]

    def allocate_output_slots(self, count: int) -> None:
        """Reserve `count` encoded-output leases, once and before binding
        (manager.py:381-394); each is shaped like a slot's payload and aux arenas."""
        if type(count) is not int or not 0 <= count <= 16:
            raise ValueError("Encoded output slot count must be 0..16")
        if self._banks.sealed or self._metadata_initialized:
            raise RuntimeError("Encoded output banks must be reserved once before binding")
        added = self._banks.reserve(count, self.slots[0])
        self.plan = replace(self.plan, reserved_bytes=self.plan.reserved_bytes + added)

    def _check_slot_id(self, slot_id) -> CompressionSlotBuffers:
        if type(slot_id) is not int or not 0 <= slot_id < len(self.slots):
            raise ValueError("Invalid compression slot")
        return self.slots[slot_id]

    def _require_execution(self, operation: str) -> None:
        if self.execution not in ("both", operation):
            raise RuntimeError(f"KVServe {self.execution}-only runtime cannot {operation}")

    def _check_slot(self, slot_id) -> None:
        self._check_slot_id(slot_id)
        if not self._metadata_initialized:
            raise RuntimeError("bind_kv_caches must run before encode / decode")

    # ------------------------------------------------------------------ execution
    def encode_into(self, slot_id, logical_ids_by_group, kv_part, *, valid_tokens_by_group, output,
                    auxiliary) -> EncodedChunk:
        """Encode one chunk and leave it in a runtime-owned bank (manager.py:396-444):
        the slot's own arena pair, or a lease the result is copied into on the slot's
        stream.  The codec's byte count is read on the host, so this waits for the
        encode; the returned event closes the copy.  The caller must not reuse the
        bank before that event."""
        self._require_execution("encode")
        slot = self._check_slot_id(slot_id)
        bank = self._banks.find(output, auxiliary)
        if bank is None or bank.owner not in (None, slot_id):
            raise ValueError("Encoded output and auxiliary must be one Runtime-owned bank")
        aux_bytes = self.aux_bytes(kv_part, valid_tokens_by_group)
        if not (bank.holds(slot.arena_a.device, slot.arena_a.numel(), aux_bytes)):
            raise ValueError("Invalid encoded output or auxiliary bank")
        chunk = self.encode(slot_id, logical_ids_by_group, kv_part, valid_tokens_by_group=valid_tokens_by_group)
        chunk.event.synchronize()
        if chunk.raw_tail_bytes:
            raise ValueError("Leased output requires a complete compressed token body")
        size = chunk.codec_bytes
        if size <= 0 or size > bank.payload.numel():
            raise ValueError("Encoded payload exceeds output bank")
        stream = self.streams[slot_id]
        with torch.cuda.stream(stream):
            if bank.owner is None:
                bank.take_from(slot, size, aux_bytes)
            slot.completion_event.record(stream)
        return EncodedChunk(chunk.array, slot.completion_event, chunk.u8_bytes, payload_bytes=size)

    def encode(self, slot_id: int, logical_ids_by_group: List[List[int]], kv_part: KVPart, *,
               valid_tokens_by_group: Dict[int, int]) -> EncodedChunk:
        self._require_execution("encode")
        self._check_slot(slot_id)
        return self.pipelines[slot_id].encode(slot_id, logical_ids_by_group, kv_part,
                                              valid_tokens_by_group=valid_tokens_by_group)

    def decode(self, slot_id: int, logical_ids_by_group: List[List[int]], kv_part: KVPart, codec_bytes: int,
               u8_bytes: int, *, valid_tokens_by_group: Dict[int, int]) -> torch.cuda.Event:
        """Reject a chunk whose sizes do not fit this runtime's layout and slot
        (manager.py:462-488), then run the slot's pipeline."""
        self._require_execution("decode")
        self._check_slot(slot_id)
        capacity = self.slots[slot_id].arena_a.numel()
        rules = (
            (u8_bytes == self.data_bytes(kv_part, valid_tokens_by_group),
             "Compressed chunk has an incompatible decoded size"),
            (0 <= codec_bytes <= capacity, "Compressed chunk exceeds receive buffer capacity"),
            ("codec" in self.config.pipeline or codec_bytes == u8_bytes,
             "Unencoded chunk payload size does not match its layout"),
        )
        for holds, message in rules:
            if not holds:
                raise ValueError(message)
        return self.pipelines[slot_id].decode(slot_id, logical_ids_by_group, kv_part, codec_bytes, u8_bytes,
                                              valid_tokens_by_group=valid_tokens_by_group)

    def shutdown(self) -> None:
        """Drain every slot stream and drop the pipelines and leases."""
        for stream in self.streams:
            stream.synchronize()
        self.pipelines.clear()
        self._banks.release_leases()


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
