"""Per-slot execution of the fixed-profile runtime (kvserve_v1/compression/runtime/pipeline.py:19-804).

Encode of one KV part of one chunk, on the slot's stream:

  1. clear the packed region and the aux region the chunk sends (pipeline.py:601-614);
  2. upload the physical block ids, one row per KV-cache group (:183-222);
  3. copy the raw tail of every layer, tokens of an incomplete logical block in the
     cache's own [heads, tokens, channels] order (:353-390);
  4. one `kvmi_rt_encode` launch set per (group, geometry): gather through the head
     order, signs, bf16-per-stage FWHT, section min / max, quantize -- all layers of
     the part in one grid, written at the layout's offsets (:624-651);
  5. rANS over the packed bytes into arena A, or the packed bytes written straight
     into arena A when the pipeline has no codec (:652-669).

Decode runs the inverse (rANS, `kvmi_rt_decode`, raw tails).  Layer tables
(`kvmi_rt_layer`: cache pointer and strides, signs, head order, offsets, sections)
are built once per `bind_kv_caches` and live on the device.  The aggregate stage
(lossless native-layout copy, :471-555) keeps the reference's index_select /
index_copy_ over the cache views.
"""

from __future__ import annotations

import array
import contextlib
import ctypes
import logging
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple, Union

import numpy as np
import torch

from .. import _lib
from ._hip import H2D, memcpy_async
from .codec import ANSCodec, EncodedChunk
from .layout import CompressionLayout, KVPart, LayerPartLayout

logger = logging.getLogger("kvserve_amd.runtime")

_AXIS = {"channel": 0, "token": 1, "tensor": 2}

CacheBinding = Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]


@dataclass
class CompressionSlotBuffers:
    arena_a: torch.Tensor
    arena_b: torch.Tensor
    aux: torch.Tensor
    block_indices: torch.Tensor
    completion_event: torch.cuda.Event
    host_indices: Optional[torch.Tensor] = None
    raw_tail: Optional[torch.Tensor] = None
    canonical: Optional[torch.Tensor] = None


@dataclass
class _Launch:
    """One kvmi_rt_encode / kvmi_rt_decode call: the layers of one KV part that share
    a cache group and a geometry."""

    group_index: int
    block_size: int
    geometry: _lib.RtGeometry
    table: torch.Tensor  # device copy of kvmi_rt_layer[num_layers]
    num_layers: int


def hadamard_transform(inputs: torch.Tensor, outputs: torch.Tensor) -> None:
    """Normalized FWHT of bf16 rows [..., D] with bf16 rounding after every butterfly
    stage, on the current stream (runtime cpp_backend.hadamard_transform).  `outputs`
    may be `inputs` itself, and must not partly overlap it."""
    if inputs.dtype is not torch.bfloat16 or outputs.dtype is not torch.bfloat16:
        raise ValueError("The runtime transform takes BF16 rows")
    if inputs.shape != outputs.shape or not inputs.is_contiguous() or not outputs.is_contiguous():
        raise ValueError("The runtime transform needs contiguous inputs and outputs of one shape")
    if not inputs.is_cuda or inputs.device != outputs.device:
        raise ValueError("The runtime transform runs on one GPU")
    d = inputs.shape[-1] if inputs.dim() else 1
    nbytes = inputs.numel() * 2
    a, b = inputs.data_ptr(), outputs.data_ptr()
    if a != b and a < b + nbytes and b < a + nbytes:
        raise ValueError("The runtime transform inputs and outputs overlap")
    if d < 1 or d > 2048 or d & (d - 1):
        raise ValueError("The runtime transform needs a power-of-two head size up to 2048")
    rows = inputs.numel() // d if d else 0
    stream = torch.cuda.current_stream(inputs.device).cuda_stream
    _lib.check(_lib.load().kvmi_rt_hadamard(a, b, rows, d, ctypes.c_void_p(stream)), "kvmi_rt_hadamard")


class CompressionPipeline:
    def __init__(self, layout: CompressionLayout, kv_cache_layout: str, blocks_per_logical: int,
                 slots: List[CompressionSlotBuffers], codec: Optional[ANSCodec], stream: torch.cuda.Stream,
                 signs: Dict[Tuple[str, int], torch.Tensor], head_orders: Dict[str, torch.Tensor],
                 stages: Tuple[str, ...] = ("transformer", "quantizer", "codec"), pipeline_backend: Optional[str] = None,
                 order_indices: Optional[Dict[str, torch.Tensor]] = None):
        # "python" / "cpp" name the reference's two standard backends; both run the
        # same HIP kernels here.
        if pipeline_backend not in (None, "python", "cpp", "hip"):
            raise ValueError("Unknown KVServe pipeline backend")
        if kv_cache_layout == "LBHNC":
            kv_cache_layout = "HND"
        if kv_cache_layout != "HND":
            raise ValueError("KVServe compression requires LBHNC/HND KV cache layout.")
        self.layout = layout
        self.kv_cache_layout = kv_cache_layout
        self.blocks_per_logical = blocks_per_logical
        self.slots = slots
        self.codec = codec
        self.stream = stream
        self.signs = signs
        self.head_orders = head_orders
        self.order_indices = order_indices if order_indices is not None else {}
        self.stages = tuple(stages)
        self.pipeline_backend = pipeline_backend
        self.identity_orders: set = set()
        self.kv_caches: Dict[str, CacheBinding] = {}
        self._cache_parts: Dict[Tuple[str, int], torch.Tensor] = {}
        self._bases: Dict[Tuple[str, int], Tuple[torch.Tensor, int]] = {}
        self._num_blocks = 0
        self._launches: Dict[int, List[_Launch]] = {0: [], 1: []}
        # "auto": the row kernels where they apply; "generic": the multi-kernel path
        # everywhere (identical results; kept selectable for tests)
        self.kernel_path = "auto"
        self._lib = _lib.load()

    @staticmethod
    def _hadamard_transform(inputs: torch.Tensor, outputs: torch.Tensor, block_size: int) -> None:
        """pipeline.py:264-309's entry point, on the HIP kernel."""
        if inputs.shape[-1] != block_size:
            raise ValueError("Row width differs from the transform size")
        hadamard_transform(inputs, outputs)

    # ------------------------------------------------------------------ binding
    def bind_kv_caches(self, kv_caches: Dict[str, CacheBinding], *, prepare_backend: bool = True) -> None:
        """Validate HND bindings (pipeline.py:104-181) and build the layer tables."""
        value_sizes = {p.layer_name: p.head_size for p in self.layout.parts(1)}
        kernel_tokens = lambda part: part.block_size // self.blocks_per_logical  # noqa: E731
        for part in self.layout.parts(0):
            cache = kv_caches[part.layer_name]
            if isinstance(cache, tuple):
                if len(cache) != 2:
                    raise ValueError("Separate KV binding requires a K/V pair")
                for tensor, size in zip(cache, (part.head_size, value_sizes[part.layer_name])):
                    if (tensor.dtype is not part.dtype or tensor.ndim != 4
                            or tuple(tensor.shape[1:]) != (part.num_heads, kernel_tokens(part), size)
                            or tensor.stride(-1) != 1 or tensor.device != self.stream.device):
                        raise ValueError("Separate KV binding requires dense BF16 HND views")
                if cache[0].shape[0] != cache[1].shape[0]:
                    raise ValueError("K and V must contain the same number of blocks")
                continue
            expected = (part.num_heads, kernel_tokens(part), part.head_size + value_sizes[part.layer_name])
            if (cache.dtype is not part.dtype or cache.ndim != 4 or tuple(cache.shape[1:]) != expected
                    or cache.stride(-1) != 1 or cache.device != self.stream.device):
                raise ValueError(f"Unsupported compression cache for {part.layer_name}: expected [blocks, {expected}] "
                                 f"with dense BF16 content, got {tuple(cache.shape)} / {cache.dtype}.")
        key_sizes = {p.layer_name: p.head_size for p in self.layout.parts(0)}
        self.kv_caches = {name: kv_caches[name] for name in key_sizes}
        self._cache_parts = {}
        self._bases = {}
        for part in self.layout.layer_parts:
            cache = self.kv_caches[part.layer_name]
            if isinstance(cache, tuple):
                view, offset = cache[part.kv_part], 0
            else:
                offset = 0 if part.kv_part == 0 else key_sizes[part.layer_name]
                view = cache.narrow(-1, offset, part.head_size)
            self._cache_parts[(part.layer_name, part.kv_part)] = view
            self._bases[(part.layer_name, part.kv_part)] = (cache[part.kv_part] if isinstance(cache, tuple) else cache,
                                                            offset)
        self._num_blocks = min(v.shape[0] for v in self._cache_parts.values())
        self._build_tables()

    def _build_tables(self) -> None:
        transform = "transformer" in self.stages and "aggregate" not in self.stages
        quantize = "quantizer" in self.stages and "aggregate" not in self.stages
        # per KV part and cache group: (group, block size, raw-tail bytes per token,
        # chunk capacity in tokens), the sums layout.py's per-layer loops compute
        self._groups = {}
        for kv in (0, 1):
            acc: Dict[int, List[int]] = {}
            for part in self.layout.parts(kv):
                entry = acc.setdefault(part.group_index, [part.block_size, 0,
                                                           part.raw_bytes // (2 * part.num_heads * part.head_size)])
                entry[1] += part.num_heads * part.head_size * 2
            self._groups[kv] = tuple((g, bs, per_token, cap) for g, (bs, per_token, cap) in acc.items())
        self._aux_clean: Dict[int, int] = {}  # slot -> KV part whose aux layout it holds, gaps zero
        self._launches = {0: [], 1: []}
        if "aggregate" in self.stages:
            return
        for kv in (0, 1):
            groups: Dict[Tuple[int, int, int, int], List[LayerPartLayout]] = {}
            for part in self.layout.parts(kv):
                key = (part.group_index, part.num_heads, part.head_size, part.block_size)
                groups.setdefault(key, []).append(part)
            for (group, heads, size, block_size), parts in groups.items():
                rows = (_lib.RtLayer * len(parts))()
                axes = 0
                aligned = True
                for i, part in enumerate(parts):
                    base, offset = self._bases[(part.layer_name, part.kv_part)]
                    aligned &= (base.data_ptr() % 16 == 0 and offset % 8 == 0
                                and all(st % 8 == 0 for st in base.stride()[:3]))
                    entry = rows[i]
                    entry.cache = base.data_ptr()
                    entry.block_stride, entry.head_stride, entry.token_stride = (base.stride(0), base.stride(1),
                                                                                 base.stride(2))
                    entry.channel_offset = offset
                    entry.signs = self.signs[(part.layer_name, kv)].data_ptr() if transform else None
                    entry.head_order = self.order_indices[part.layer_name].data_ptr()
                    entry.u8_offset = part.u8_offset
                    entry.num_sections = len(part.sections) if quantize else 0
                    for j, s in enumerate(part.sections if quantize else ()):
                        entry.sections[j] = _lib.RtSection(s.head_start, s.head_count, s.num_levels, _AXIS[s.axis],
                                                           s.aux_min_offset, s.aux_scale_offset)
                        axes |= 1 << _AXIS[s.axis]
                host = torch.frombuffer(bytearray(bytes(rows)), dtype=torch.uint8)
                table = host.to(self.stream.device)
                flags = ((_lib.RT_TRANSFORM if transform else 0) | (_lib.RT_QUANTIZE if quantize else 0)
                         | (_lib.RT_ALIGNED if aligned else 0) | (_lib.RT_GENERIC if self.kernel_path == "generic" else 0))
                geometry = _lib.RtGeometry(heads, size, block_size // self.blocks_per_logical, flags, axes)
                self._launches[kv].append(_Launch(group, block_size, geometry, table, len(parts)))

    # ------------------------------------------------------------------ indices
    _STAGING_DEPTH = 4  # uploads of block ids kept in flight per pipeline

    def _physical_ids(self, logical_ids) -> np.ndarray:
        if isinstance(logical_ids, torch.Tensor):
            ids = logical_ids.detach().to("cpu", torch.int64).numpy()
        elif isinstance(logical_ids, np.ndarray):
            ids = logical_ids.astype(np.int64, copy=False)
        else:
            ids = np.frombuffer(array.array("q", logical_ids), dtype=np.int64)
        f = self.blocks_per_logical
        if f == 1:
            return ids
        return (ids[:, None] * f + np.arange(f, dtype=np.int64)[None, :]).reshape(-1)

    def _staging_rows(self, slot: CompressionSlotBuffers) -> Tuple[np.ndarray, torch.Tensor, int]:
        """A pinned staging generation for the id uploads of one call.  A generation is
        reused only after the copies queued from it have run (its event)."""
        if getattr(self, "_staging", None) is None or self._staging.shape[1:] != slot.block_indices.shape:
            self._staging = torch.empty((self._STAGING_DEPTH, *slot.block_indices.shape), dtype=torch.int64,
                                        pin_memory=True)
            self._staging_np = self._staging.numpy()
            self._staging_events = [None] * self._STAGING_DEPTH
            self._staging_next = 0
        g = self._staging_next
        self._staging_next = (g + 1) % self._STAGING_DEPTH
        if self._staging_events[g] is not None:
            self._staging_events[g].synchronize()
        return self._staging_np[g], self._staging[g], g

    def _group_indices(self, slot: CompressionSlotBuffers, logical_ids_by_group
                       ) -> Dict[int, Tuple[torch.Tensor, np.ndarray]]:
        """Device ids (one upload per group, pipeline.py:183-222) and host ids."""
        out = {}
        staged = None
        for group, logical_ids in enumerate(logical_ids_by_group):
            if not len(logical_ids) or group not in self.layout.index_rows_by_group:
                continue
            row = self.layout.index_rows_by_group[group]
            physical = self._physical_ids(logical_ids)
            storage = slot.block_indices if slot.block_indices.ndim == 1 else slot.block_indices[row]
            n = physical.size
            if n > storage.numel():
                raise ValueError("Compressed chunk exceeds logical_blocks_per_chunk")
            if physical.min() < 0 or physical.max() >= self._num_blocks:
                raise ValueError(f"Block id out of range for KV caches of {self._num_blocks} blocks")
            if staged is None:
                staged = self._staging_rows(slot)
            host_np, host, g = staged
            hrow_np = host_np if host_np.ndim == 1 else host_np[row]
            hrow = host if host.ndim == 1 else host[row]
            hrow_np[:n] = physical
            indices = storage[:n]
            memcpy_async(indices.data_ptr(), hrow.data_ptr(), 8 * n, H2D, self.stream.cuda_stream)
            out[group] = (indices, physical)
        if staged is not None:
            event = self._staging_events[staged[2]] or torch.cuda.Event()
            event.record(self.stream)
            self._staging_events[staged[2]] = event
        return out

    # ------------------------------------------------------------------ raw tails
    def _cache_part(self, part: LayerPartLayout) -> torch.Tensor:
        return self._cache_parts[(part.layer_name, part.kv_part)]

    def _tail_blocks(self, part: LayerPartLayout, physical: np.ndarray, valid_tokens: int):
        """(physical block, token count) of the incomplete logical block."""
        tail = valid_tokens % part.block_size
        if not tail:
            return []
        kernel_tokens = part.block_size // self.blocks_per_logical
        out = []
        for i, block in enumerate(physical[-self.blocks_per_logical:].tolist()):
            out.append((block, max(0, min(tail - i * kernel_tokens, kernel_tokens))))
        return out

    def _pack_raw_tail(self, slot, part, physical, valid_tokens, offset) -> int:
        """pipeline.py:353-390: [heads, count, channels] of each tail block, packed."""
        cache = self._cache_part(part)
        for block, count in self._tail_blocks(part, physical, valid_tokens):
            if count <= 0:
                break
            source = cache[block, :, :count, :]
            nbytes = source.numel() * 2
            slot.raw_tail[offset:offset + nbytes].view(source.dtype).view_as(source).copy_(source)
            offset += nbytes
        return offset

    def _apply_raw_tail(self, slot, part, physical, valid_tokens, offset) -> int:
        """pipeline.py:392-428: the tail blocks are cleared first, so no stale tokens
        of either side survive past the tail."""
        cache = self._cache_part(part)
        for block, count in self._tail_blocks(part, physical, valid_tokens):
            target = cache[block]
            target.zero_()
            if count <= 0:
                continue
            destination = target[:, :count, :]
            nbytes = destination.numel() * 2
            destination.copy_(slot.raw_tail[offset:offset + nbytes].view(destination.dtype).view_as(destination))
            offset += nbytes
        return offset

    # ------------------------------------------------------------------ aggregate
    def _aggregate_segments(self, logical_ids_by_group, kv_part):
        segments, offset = [], 0
        for row, part in enumerate(self.layout.parts(kv_part)):
            ids = logical_ids_by_group[part.group_index] if part.group_index < len(logical_ids_by_group) else []
            blocks = len(ids) * self.blocks_per_logical
            cache = self._cache_part(part)
            nbytes = blocks * (cache.numel() // cache.shape[0]) * cache.element_size()
            segments.append((row, part, offset, nbytes, blocks))
            offset += nbytes
        return segments, offset

    def _aggregate_view(self, buffer, offset, nbytes, blocks, part):
        cache = self._cache_part(part)
        return buffer[offset:offset + nbytes].view(part.dtype).view(blocks, *cache.shape[1:])

    def _encode_aggregate(self, slot, logical_ids_by_group, kv_part) -> EncodedChunk:
        segments, payload = self._aggregate_segments(logical_ids_by_group, kv_part)
        with torch.cuda.stream(self.stream):
            index = self._group_indices(slot, logical_ids_by_group)
            for _row, part, offset, nbytes, blocks in segments:
                if not blocks:
                    continue
                out = self._aggregate_view(slot.arena_a, offset, nbytes, blocks, part)
                torch.index_select(self._cache_part(part), 0, index[part.group_index][0], out=out)
            slot.completion_event.record(self.stream)
        return EncodedChunk(None, slot.completion_event, payload, payload, 0, 0)

    def _decode_aggregate(self, slot, logical_ids_by_group, kv_part) -> torch.cuda.Event:
        segments, _ = self._aggregate_segments(logical_ids_by_group, kv_part)
        with torch.cuda.stream(self.stream):
            index = self._group_indices(slot, logical_ids_by_group)
            for _row, part, offset, nbytes, blocks in segments:
                if not blocks:
                    continue
                value = self._aggregate_view(slot.arena_a, offset, nbytes, blocks, part)
                self._cache_part(part).index_copy_(0, index[part.group_index][0], value)
            slot.completion_event.record(self.stream)
        return slot.completion_event

    # ------------------------------------------------------------------ body
    @property
    def _stream_ptr(self) -> ctypes.c_void_p:
        ptr = self.__dict__.get("_stream_ptr_cache")
        if ptr is None:
            ptr = self.__dict__["_stream_ptr_cache"] = ctypes.c_void_p(self.stream.cuda_stream)
        return ptr

    def _body(self, launch: _Launch, index, valid_tokens_by_group) -> Optional[Tuple[torch.Tensor, int]]:
        entry = index.get(launch.group_index)
        tokens = valid_tokens_by_group.get(launch.group_index, 0)
        blocks = tokens // launch.block_size * self.blocks_per_logical
        if entry is None or not blocks:
            return None
        return entry[0], blocks

    def encode(self, slot_id: int, logical_ids_by_group: List[List[int]], kv_part: KVPart, *,
               valid_tokens_by_group: Dict[int, int]) -> EncodedChunk:
        slot = self.slots[slot_id]
        tokens = valid_tokens_by_group
        groups = self._groups[kv_part]
        raw_tail_bytes = sum((tokens.get(g, 0) % bs) * per_token for g, bs, per_token, _ in groups)
        if logger.isEnabledFor(logging.DEBUG):
            logger.debug("KVServe runtime encode: slot=%d kv_part=%d logical_ids=%s", slot_id, kv_part,
                         [g for g in logical_ids_by_group if len(g)])
        if "aggregate" in self.stages:
            return self._encode_aggregate(slot, logical_ids_by_group, kv_part)
        quantized = "quantizer" in self.stages
        u8_bytes = (self.layout.u8_bytes_by_part if quantized else self.layout.raw_bytes_by_part)[kv_part]
        aux_bytes = self.layout.aux_bytes_by_part[kv_part] if quantized else 0
        if not any(tokens.get(g, 0) >= bs for g, bs, _, _ in self._groups[0]):  # layout.has_body
            u8_bytes = aux_bytes = 0
        coded = bool(u8_bytes) and "codec" in self.stages
        packed = slot.arena_b[self.layout.u8_base:] if coded else slot.arena_a
        tail_addr = slot.raw_tail.data_ptr() if slot.raw_tail is not None else 0
        # A chunk that fills every layer's capacity overwrites the whole payload (the
        # layers' symbol ranges tile it) and every aux entry; the aux arena's
        # alignment gaps stay zero unless the other KV part's sections or a received
        # chunk were written there since it was last cleared.
        full = all(tokens.get(g, 0) == cap for g, _, _, cap in groups)
        clear_aux = bool(aux_bytes) and not (full and self._aux_clean.get(slot_id) == kv_part)
        torch_ops = not full or clear_aux or raw_tail_bytes
        with torch.cuda.stream(self.stream) if torch_ops else contextlib.nullcontext():
            if not full:
                # capacities are planned for the largest chunk: a short chunk must not
                # carry the previous owner's bytes
                packed[:u8_bytes].zero_()
            if clear_aux:
                slot.aux[:aux_bytes].zero_()
            if aux_bytes:
                self._aux_clean[slot_id] = kv_part
            index = self._group_indices(slot, logical_ids_by_group)
            offset = 0
            if raw_tail_bytes:
                for part in self.layout.parts(kv_part):
                    entry = index.get(part.group_index)
                    if entry is not None:
                        offset = self._pack_raw_tail(slot, part, entry[1], tokens[part.group_index], offset)
            canonical = slot.canonical.data_ptr() if slot.canonical is not None else None
            for launch in self._launches[kv_part]:
                body = self._body(launch, index, tokens)
                if body is None:
                    continue
                ids, blocks = body
                rc = self._lib.kvmi_rt_encode(ctypes.byref(launch.geometry), launch.table.data_ptr(), launch.num_layers,
                                              ids.data_ptr(), blocks, canonical, packed.data_ptr(),
                                              slot.aux.data_ptr() if quantized else None,
                                              self.layout.aux_arena_bytes // 2, self._stream_ptr)
                _lib.check(rc, "kvmi_rt_encode")
            if not coded:
                slot.completion_event.record(self.stream)
                return EncodedChunk(None, slot.completion_event, u8_bytes, u8_bytes, raw_tail_bytes, tail_addr)
            encoded = self.codec.encode(packed, slot.arena_a, u8_bytes, slot.completion_event)
        encoded.raw_tail_bytes = offset
        encoded.raw_tail_addr = tail_addr
        return encoded

    def decode(self, slot_id: int, logical_ids_by_group: List[List[int]], kv_part: KVPart, codec_bytes: int,
               u8_bytes: int, *, valid_tokens_by_group: Dict[int, int]) -> torch.cuda.Event:
        slot = self.slots[slot_id]
        if "aggregate" in self.stages:
            return self._decode_aggregate(slot, logical_ids_by_group, kv_part)
        if logger.isEnabledFor(logging.DEBUG):
            logger.debug("KVServe runtime decode: slot=%d kv_part=%d codec_bytes=%d u8_bytes=%d", slot_id, kv_part,
                         codec_bytes, u8_bytes)
        quantized = "quantizer" in self.stages
        coded = bool(u8_bytes) and "codec" in self.stages
        packed = slot.arena_b[self.layout.u8_base:] if coded else slot.arena_a
        tokens = valid_tokens_by_group
        tails = any(tokens.get(g, 0) % bs for g, bs, _, _ in self._groups[kv_part])
        self._aux_clean.pop(slot_id, None)  # the received aux replaced the slot's own
        with torch.cuda.stream(self.stream) if tails else contextlib.nullcontext():
            if coded:
                self.codec.decode(slot.arena_a, packed, codec_bytes, u8_bytes, slot.completion_event)
            index = self._group_indices(slot, logical_ids_by_group)
            for launch in self._launches[kv_part]:
                body = self._body(launch, index, tokens)
                if body is None:
                    continue
                ids, blocks = body
                rc = self._lib.kvmi_rt_decode(ctypes.byref(launch.geometry), launch.table.data_ptr(), launch.num_layers,
                                              ids.data_ptr(), blocks, packed.data_ptr(),
                                              slot.aux.data_ptr() if quantized else None, self._stream_ptr)
                _lib.check(rc, "kvmi_rt_decode")
            offset = 0
            if tails:
                for part in self.layout.parts(kv_part):
                    entry = index.get(part.group_index)
                    if entry is not None:
                        offset = self._apply_raw_tail(slot, part, entry[1], tokens[part.group_index], offset)
            slot.completion_event.record(self.stream)
        return slot.completion_event
