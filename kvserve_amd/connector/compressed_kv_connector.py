"""CompressedKVConnector: vLLM v1 KV connector for prefill/decode disaggregation
with KV compression on MI355X (kvserve_v1/connector/compressed_kv_connector.py:126-685).

Same class, constructor, roles, metadata types, environment knobs and transport
protocol as the reference; the worker side runs the fused gfx950 codec on the
paged caches themselves:

  save_kv_layer   records the layer's cache for each scheduled request (the
                  reference copies the request's blocks out here, :377-391).  The
                  cache is read in wait_for_save of the same forward pass; no
                  layer writes another layer's cache and the request's blocks
                  cannot change before the step ends, so the bytes read are the
                  same.
  wait_for_save   layers in sorted(layer_name) order -- the reference's layer id is
                  the index in that order (:425-427) -- are compressed straight
                  from the caches by the fused paged kernels (no per-layer gather,
                  no stack), bundled by `build_wire` and sent with the
                  "__compressed__" sentinel in front of the layer names (:393-497).
                  Compression off, below `min_compress_size` or failed: the blocks
                  are gathered straight into one stacked tensor and sent raw.
  start_load_kv   restores the bundle and decompresses straight into the decode
                  caches at the scheduled block ids (:235-371); raw payloads are
                  scattered per layer.  Layers absent from the forward context are
                  skipped, as in the reference.

vLLM is not a dependency: where it is importable the connector subclasses its
KVConnectorBase_V1; otherwise a stand-in with the same metadata binding methods is
used, so the connector runs in tests and single-process pipelines.
"""

from __future__ import annotations

import enum
import json
import logging
import os
import time
from collections import defaultdict, deque
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import torch

from ..compression.compression_manager import FusedCompressionManager
from ..compression.manager import add_sentinel, is_compressed_layer_names, strip_sentinel
from ..compression.wire import CompressedWire, build_wire, restore_from_wire
from .kv_utils import (extract_kv_from_layer_by_blocks, inject_kv_into_layer_by_blocks, is_flash_layout,
                       make_slot_mapping)

try:  # pragma: no cover - vLLM is not installed in the build image
    from vllm.distributed.kv_transfer.kv_connector.v1.base import (KVConnectorBase_V1, KVConnectorMetadata,
                                                                   KVConnectorRole)
    HAS_VLLM = True
except ImportError:
    HAS_VLLM = False

    class KVConnectorRole(enum.Enum):
        SCHEDULER = 0
        WORKER = 1

    class KVConnectorMetadata:
        """Per-step metadata the scheduler hands to the workers."""

    class KVConnectorBase_V1:
        """The parts of vLLM's connector base class this connector relies on."""

        def __init__(self, vllm_config, role, kv_cache_config=None):
            self._connector_metadata: Optional[KVConnectorMetadata] = None
            self._vllm_config = vllm_config
            self._role = role
            self._kv_cache_config = kv_cache_config

        @property
        def role(self):
            return self._role

        def bind_connector_metadata(self, connector_metadata: KVConnectorMetadata) -> None:
            self._connector_metadata = connector_metadata

        def clear_connector_metadata(self) -> None:
            self._connector_metadata = None

        def _get_connector_metadata(self) -> KVConnectorMetadata:
            assert self._connector_metadata is not None
            return self._connector_metadata

        def register_kv_caches(self, kv_caches: Dict[str, torch.Tensor]) -> None:
            return None

logger = logging.getLogger("kvserve_amd.connector")
_warned: set = set()


def _warn_once(msg: str, *args) -> None:
    if msg not in _warned:
        _warned.add(msg)
        logger.warning(msg, *args)


try:
    _LOAD_TIMEOUT_S = float(os.environ.get("KVSERVE_LOAD_TIMEOUT_S", "60"))
except ValueError:
    _LOAD_TIMEOUT_S = 60.0
_DEFAULT_MAX_NCCL_CHUNK_BYTES = 512 * 1024 * 1024


def _sorted_rids(rids) -> List[str]:
    return sorted(rids)


def _write_compression_stats(request_id: str, transfer_id: str, original_bytes: int, compressed_bytes: int) -> None:
    """One JSON line per compressed send to $KVSERVE_COMPRESSION_STATS_PATH (:57-78)."""
    path = os.environ.get("KVSERVE_COMPRESSION_STATS_PATH")
    if not path or original_bytes <= 0 or compressed_bytes <= 0:
        return
    row = {"request_id": request_id, "transfer_id": transfer_id, "original_bytes": original_bytes,
           "compressed_bytes": compressed_bytes}
    try:
        with open(path, "a") as f:
            f.write(json.dumps(row, sort_keys=True) + "\n")
    except OSError as e:
        _warn_once("[Connector] Failed to write compression stats to %s: %s", path, e)


def _max_nccl_chunk_bytes() -> int:
    """$KVSERVE_MAX_NCCL_CHUNK_BYTES, a positive integer, else 512 MiB (:81-97)."""
    raw = os.environ.get("KVSERVE_MAX_NCCL_CHUNK_BYTES")
    if not raw:
        return _DEFAULT_MAX_NCCL_CHUNK_BYTES
    try:
        value = int(raw)
    except ValueError:
        _warn_once("Invalid KVSERVE_MAX_NCCL_CHUNK_BYTES=%r; using default %d", raw, _DEFAULT_MAX_NCCL_CHUNK_BYTES)
        return _DEFAULT_MAX_NCCL_CHUNK_BYTES
    if value <= 0:
        _warn_once("KVSERVE_MAX_NCCL_CHUNK_BYTES must be positive; using default %d", _DEFAULT_MAX_NCCL_CHUNK_BYTES)
        return _DEFAULT_MAX_NCCL_CHUNK_BYTES
    return value


@dataclass
class ReqMeta:
    request_id: str
    transfer_id: str
    token_ids: List[int]
    block_ids: List[int]
    slot_mapping: torch.Tensor  # CPU int64 [num_tokens]


@dataclass
class CompressedKVConnectorMetadata(KVConnectorMetadata):
    requests: List[ReqMeta] = field(default_factory=list)

    def add_request(self, request_id: str, transfer_id: str, token_ids: List[int], block_ids: List[int],
                    block_size: int) -> None:
        self.requests.append(ReqMeta(request_id=request_id, transfer_id=transfer_id, token_ids=token_ids,
                                     block_ids=block_ids,
                                     slot_mapping=make_slot_mapping(token_ids, block_ids, block_size)))


def _truthy(v: Optional[str]) -> bool:
    return (v or "").strip().lower() in {"1", "true", "yes", "on"}


class CompressedKVConnector(KVConnectorBase_V1):
    """KV connector: compressed transfer of a request's prompt KV from the prefill
    (producer) instance to the decode (consumer) instance.

    `kv_connector_extra_config` keys: "compression" (None, "default" or a profile
    dict, as for KVCompressionAdapter), "transport_class" ("module:Class" of a
    transport with the NcclTransport surface, or "loopback"), and, without vLLM,
    "tp_rank" / "tp_size".
    """

    def __init__(self, vllm_config, role, kv_cache_config=None):
        super().__init__(vllm_config, role, kv_cache_config)
        cfg = vllm_config.kv_transfer_config
        extra = dict(getattr(cfg, "kv_connector_extra_config", None) or {})
        self.is_producer = bool(cfg.is_kv_producer)
        self._block_size = vllm_config.cache_config.block_size
        self._async_send = _truthy(os.environ.get("KVSERVE_ASYNC_SEND", "0"))
        configured = max(1, int(cfg.kv_buffer_size))
        try:
            self._max_inflight_bytes = int(os.environ.get("KVSERVE_MAX_INFLIGHT_BYTES", str(configured)))
        except ValueError:
            self._max_inflight_bytes = configured

        # scheduler side
        self._requests_need_load: Dict[str, Tuple[Any, List[int]]] = {}
        self._request_transfer_ids: Dict[str, str] = {}
        self.chunked_prefill: Dict[str, Tuple[List[int], List[int]]] = {}
        # worker side
        self._worker_received_kv: Dict[str, deque] = defaultdict(deque)
        self._layer_buffers: Dict[str, Dict[str, torch.Tensor]] = {}
        self._save_block_ids: Dict[str, List[int]] = {}

        mc = vllm_config.model_config
        self._num_kv_heads: int = mc.get_num_kv_heads(vllm_config.parallel_config)
        self._head_size: int = mc.get_head_size()
        self._model_name: str = os.path.basename(str(mc.model).rstrip("/"))
        self._tp_rank = int(extra.get("tp_rank", 0))
        self._tp_size = int(extra.get("tp_size", 1))
        self._compressor: Optional[Any] = None
        self._compression_cfg = extra.get("compression")
        self._transport_spec = extra.get("transport_class")

        if role == KVConnectorRole.WORKER:
            local_rank = int(os.environ.get("LOCAL_RANK", "0"))
            if HAS_VLLM:  # pragma: no cover
                from vllm.distributed.parallel_state import (get_tensor_model_parallel_rank,
                                                             get_tensor_model_parallel_world_size, get_world_group)
                local_rank = get_world_group().local_rank
                self._tp_rank = get_tensor_model_parallel_rank()
                self._tp_size = get_tensor_model_parallel_world_size()
            self._transport = self._build_transport(cfg, local_rank=local_rank, channel_rank=self._tp_rank,
                                                    spec=self._transport_spec)
            logger.info("[CompressedKVConnector] WORKER init: is_producer=%s local_rank=%d tp_rank=%d tp_size=%d "
                        "compression=%s", self.is_producer, local_rank, self._tp_rank, self._tp_size,
                        "enabled" if self._compression_cfg else "disabled")

    @classmethod
    def get_required_kvcache_layout(cls, vllm_config) -> Optional[str]:
        """NHD for the compressed path; MLA keeps vLLM's default (:216-231)."""
        if getattr(vllm_config, "model_config", None) is None:
            _warn_once("Unable to detect current VLLM config. Fallback to default KV cache layout.")
            return None
        if getattr(vllm_config.model_config, "use_mla", False):
            _warn_once("CompressedKVConnector has not validated MLA KV cache layout; "
                       "falling back to vLLM default layout.")
            return None
        return "NHD"

    # ------------------------------------------------------------------ worker: load
    def start_load_kv(self, forward_context, **kwargs) -> None:
        """Consume every scheduled request's payload as it arrives, in arrival
        order, and write it into the decode caches (:235-371)."""
        if self.is_producer:
            return
        for rid, payloads in self._transport.drain_received().items():
            self._worker_received_kv[rid].extend(payloads)
        meta = self._get_connector_metadata()
        if not isinstance(meta, CompressedKVConnectorMetadata):
            return

        pending = list(meta.requests)
        self._transport.set_expected_requests([r.transfer_id for r in pending])
        load_t0 = time.perf_counter()
        deadline = time.monotonic() + _LOAD_TIMEOUT_S
        while pending:
            for key, payloads in self._transport.drain_received().items():
                self._worker_received_kv[key].extend(payloads)
            req = next((r for r in pending if self._worker_received_kv.get(r.transfer_id)), None)
            if req is None:
                if time.monotonic() > deadline:
                    for missing in pending:
                        self._transport.record_stat({
                            "direction": "load_wait", "kind": "timeout", "request_id": missing.transfer_id,
                            "scheduler_request_id": missing.request_id,
                            "receive_wait_s": time.perf_counter() - load_t0})
                    self._transport.set_expected_requests([])
                    raise TimeoutError("Timed out waiting for KV transfers: " +
                                       ", ".join(r.transfer_id for r in pending))
                time.sleep(0.005)
                continue
            pending.remove(req)
            rid, transfer_id = req.request_id, req.transfer_id
            layer_names, payload = self._worker_received_kv[transfer_id].popleft()
            receive_wait_s = time.perf_counter() - load_t0
            if not self._worker_received_kv[transfer_id]:
                self._worker_received_kv.pop(transfer_id, None)
            payload_bytes = self._transport.payload_nbytes(payload)
            try:
                if payload is None:
                    self._transport.record_stat({"direction": "load_wait", "kind": "failed",
                                                 "request_id": transfer_id, "scheduler_request_id": rid,
                                                 "receive_wait_s": receive_wait_s})
                    logger.error("[Connector] transport reported failure for rid=%s transfer_id=%s", rid,
                                 transfer_id)
                    raise RuntimeError(f"KV transport failed for {transfer_id}")
                compressed_payload = is_compressed_layer_names(layer_names)
                layer_names = strip_sentinel(layer_names)
                caches = self._decode_caches(forward_context, layer_names)
                if compressed_payload:
                    self._load_compressed(payload, layer_names, caches, req)
                else:
                    for i, cache in enumerate(caches):
                        if cache is not None:
                            inject_kv_into_layer_by_blocks(cache, payload[i], req.block_ids, rid)
                self._transport.record_stat({
                    "direction": "load_wait", "kind": "compressed" if compressed_payload else "raw",
                    "request_id": transfer_id, "scheduler_request_id": rid, "receive_wait_s": receive_wait_s,
                    "start_load_total_s": time.perf_counter() - load_t0})
            finally:
                # the staging credit covers the payload until the GPU has read it
                if self._transport.device.type == "cuda":
                    torch.cuda.current_stream(self._transport.device).synchronize()
                self._transport.release_received(transfer_id, payload_bytes)
        self._transport.set_expected_requests([])

    @staticmethod
    def _decode_caches(forward_context, layer_names: Sequence[str]) -> List[Optional[torch.Tensor]]:
        out: List[Optional[torch.Tensor]] = []
        for name in layer_names:
            layer = forward_context.no_compile_layers.get(name)
            kv = getattr(layer, "kv_cache", None) if layer is not None else None
            out.append(None if kv is None else kv[forward_context.virtual_engine])
        return out

    def _load_compressed(self, payload, layer_names, caches, req: ReqMeta) -> None:
        rid, transfer_id = req.request_id, req.transfer_id
        compressor = self._get_compressor()
        if compressor is None:
            logger.error("[Connector] Received compressed KV but no compressor configured for %s", rid)
            raise RuntimeError(f"No KV decompressor configured for {transfer_id}")
        if not isinstance(payload, dict) or not payload.get("__bundle__"):
            logger.error("[Connector] Invalid compressed payload for %s", rid)
            raise RuntimeError(f"Invalid compressed KV payload for {transfer_id}")
        compressed = restore_from_wire(CompressedWire(meta=payload["meta"], body_chunks=payload["body_chunks"],
                                                      aux_tensors=payload["aux_tensors"]))
        if not req.block_ids:
            return
        if self._paged_ok(compressor, caches):
            try:
                compressor.decompress_paged(compressed, caches, req.block_ids)
            except Exception as e:
                logger.error("[Connector] Decompression failed for %s: %s", rid, e)
                raise RuntimeError(f"KV decompression failed for {transfer_id}") from e
            return
        stacked = compressor.decompress(compressed)
        if stacked is None:
            logger.error("[Connector] Decompression failed for %s", rid)
            raise RuntimeError(f"KV decompression failed for {transfer_id}")
        for i, cache in enumerate(caches):
            if cache is not None:
                inject_kv_into_layer_by_blocks(cache, stacked[i], req.block_ids, rid)

    @staticmethod
    def _paged_ok(compressor, caches: Sequence[Optional[torch.Tensor]]) -> bool:
        """The fused paged kernels apply: every layer present, NHD bf16 caches of
        one shape on one GPU, and a pipeline with a quantizer."""
        if not caches or any(c is None for c in caches):
            return False
        if not isinstance(getattr(compressor, "_manager", None), FusedCompressionManager):
            return False
        c0 = caches[0]
        return all(is_flash_layout(c) and c.dtype == torch.bfloat16 and c.shape[2:] == c0.shape[2:]
                   and c.device == c0.device for c in caches)

    def wait_for_layer_load(self, layer_name: str) -> None:
        return None

    # ------------------------------------------------------------------ worker: save
    def save_kv_layer(self, layer_name: str, kv_layer: torch.Tensor, attn_metadata, **kwargs) -> None:
        if not self.is_producer:
            return
        meta = self._get_connector_metadata()
        if not isinstance(meta, CompressedKVConnectorMetadata):
            return
        for req in meta.requests:
            self._layer_buffers.setdefault(req.request_id, {})[layer_name] = kv_layer
            self._save_block_ids[req.request_id] = list(req.block_ids)

    def wait_for_save(self) -> None:
        if not self.is_producer:
            return
        meta = self._get_connector_metadata()
        if not isinstance(meta, CompressedKVConnectorMetadata):
            return
        current = {r.request_id for r in meta.requests}
        transfer_ids = [r.transfer_id for r in meta.requests]
        stale = set(self._layer_buffers) - current
        if stale:
            logger.warning("[Connector] Dropping stale layer buffers: %s", stale)
            for rid in stale:
                self._layer_buffers.pop(rid, None)
                self._save_block_ids.pop(rid, None)

        for req in meta.requests:
            rid, transfer_id = req.request_id, req.transfer_id
            layer_kv = self._layer_buffers.pop(rid, None)
            block_ids = self._save_block_ids.pop(rid, list(req.block_ids))
            if not layer_kv:
                continue
            names = sorted(layer_kv)
            caches = [layer_kv[n] for n in names]
            compressor = self._get_compressor()
            if compressor is not None:
                t0 = time.monotonic()
                compressed, raw_bytes = self._compress(compressor, caches, block_ids, rid)
                if compressed is not None:
                    wire = build_wire(compressed, _max_nccl_chunk_bytes())
                    self._transport.send_bundle(transfer_id, add_sentinel(names), wire.meta, wire.body_chunks,
                                                wire.aux_tensors)
                    _write_compression_stats(rid, transfer_id, raw_bytes, wire.nbytes)
                    compressor.update_controller(rid, (time.monotonic() - t0) * 1e3)
                    logger.debug("[Connector] Sent compressed KV for %s (%d layers, %.2f MB -> %.2f MB)", rid,
                                 len(names), raw_bytes / 1e6, wire.nbytes / 1e6)
                    continue
                logger.warning("[Connector] Compression returned None for %s, falling back to raw send", rid)
            self._transport.send(transfer_id, names, self._stack(caches, block_ids))

        if self._async_send:
            before = self._transport.pending_bytes()
            wait_s = self._transport.wait_for_below(self._max_inflight_bytes)
            if transfer_ids:
                self._transport.record_stat({
                    "direction": "backpressure", "kind": "producer", "request_id": transfer_ids[0],
                    "scheduled_requests": len(transfer_ids), "blocked": before > self._max_inflight_bytes,
                    "pending_before_bytes": before, "pending_after_bytes": self._transport.pending_bytes(),
                    "limit_bytes": self._max_inflight_bytes, "wait_s": wait_s})
        else:
            self._transport.wait_for_sent()

    def _compress(self, compressor, caches: List[torch.Tensor], block_ids: List[int], rid: str):
        """(payload or None, raw bytes).  Paged kernels on the caches when they
        apply, else the reference's gather + stack + compress."""
        if not block_ids:
            return None, 0
        if self._paged_ok(compressor, caches):
            c0 = caches[0]
            raw = len(caches) * 2 * len(block_ids) * (c0[0, 0].numel()) * c0.element_size()
            return compressor.compress_paged(caches, block_ids, rid), raw
        stacked = self._stack(caches, block_ids)
        return compressor.compress(stacked, rid), stacked.numel() * stacked.element_size()

    @staticmethod
    def _stack(caches: List[torch.Tensor], block_ids: List[int]) -> torch.Tensor:
        """[L, 2, nb, ...] of the request's blocks, each layer gathered straight into
        its slice (the reference's extract + torch.stack, :377-391, :425-427)."""
        first = extract_kv_from_layer_by_blocks(caches[0], block_ids)
        out = torch.empty((len(caches),) + tuple(first.shape), dtype=first.dtype, device=first.device)
        out[0].copy_(first)
        for i in range(1, len(caches)):
            if tuple(caches[i].shape[2:]) != tuple(caches[0].shape[2:]) or caches[i].dtype != first.dtype:
                raise RuntimeError("layers of one request must share one KV cache shape")
            extract_kv_from_layer_by_blocks(caches[i], block_ids, out=out[i])
        return out

    def get_finished(self, finished_req_ids: set) -> Tuple[Optional[set], Optional[set]]:
        return None, None

    def shutdown(self) -> None:
        transport = getattr(self, "_transport", None)
        if self.is_producer and transport is not None:
            transport.wait_for_sent()

    # ------------------------------------------------------------------ scheduler
    def get_num_new_matched_tokens(self, request, num_computed_tokens: int) -> Tuple[int, bool]:
        """The consumer takes all prompt tokens but the last from the producer;
        vLLM must compute at least one token itself (:514-524)."""
        if self.is_producer:
            return 0, False
        n = len(request.prompt_token_ids) - 1 - num_computed_tokens
        return (n, False) if n > 0 else (0, False)

    def update_state_after_alloc(self, request, blocks, num_external_tokens: int) -> None:
        self._resolve_transfer_id(request.request_id, request)
        if not self.is_producer and num_external_tokens > 0:
            self._requests_need_load[request.request_id] = (request, blocks.get_block_ids()[0])

    def build_connector_meta(self, scheduler_output) -> CompressedKVConnectorMetadata:
        """This step's transfers (:535-614).  Producer: a request is sent once its
        whole prompt has been prefilled, chunked prefills accumulating their block
        ids across steps.  Consumer: the requests waiting for a load, new or
        resumed after preemption."""
        meta = CompressedKVConnectorMetadata()
        for new in scheduler_output.scheduled_new_reqs:
            prompt = new.prompt_token_ids or []
            if self.is_producer:
                n = scheduler_output.num_scheduled_tokens[new.req_id] + new.num_computed_tokens
                if n < len(prompt):
                    self.chunked_prefill[new.req_id] = (new.block_ids[0], prompt)
                    continue
                meta.add_request(new.req_id, self._resolve_transfer_id(new.req_id), prompt, new.block_ids[0],
                                 self._block_size)
            elif new.req_id in self._requests_need_load:
                meta.add_request(new.req_id, self._resolve_transfer_id(new.req_id), prompt, new.block_ids[0],
                                 self._block_size)
                self._requests_need_load.pop(new.req_id)

        cached = scheduler_output.scheduled_cached_reqs
        resumed_ids = getattr(cached, "resumed_req_ids", set())
        for i, req_id in enumerate(cached.req_ids):
            computed = cached.num_computed_tokens[i]
            new_blocks = cached.new_block_ids[i]
            resumed = req_id in resumed_ids
            if self.is_producer:
                n = scheduler_output.num_scheduled_tokens[req_id] + computed
                assert req_id in self.chunked_prefill and new_blocks is not None
                block_ids = new_blocks[0]
                if not resumed:
                    block_ids = self.chunked_prefill[req_id][0] + block_ids
                prompt = self.chunked_prefill[req_id][1]
                if n < len(prompt):
                    self.chunked_prefill[req_id] = (block_ids, prompt)
                    continue
                meta.add_request(req_id, self._resolve_transfer_id(req_id), prompt, block_ids, self._block_size)
                self.chunked_prefill.pop(req_id, None)
                continue
            if not resumed:  # resumed requests come first in the cached list
                break
            if req_id in self._requests_need_load:
                request, _ = self._requests_need_load.pop(req_id)
                assert new_blocks is not None
                meta.add_request(req_id, self._resolve_transfer_id(req_id, request),
                                 request.all_token_ids[:computed + 1], new_blocks[0], self._block_size)
        return meta

    def request_finished(self, request, block_ids: List[int]) -> Tuple[bool, Optional[Dict[str, Any]]]:
        self.chunked_prefill.pop(request.request_id, None)
        self._request_transfer_ids.pop(request.request_id, None)
        if not self.is_producer:
            self._requests_need_load.pop(request.request_id, None)
        return False, None

    # ------------------------------------------------------------------ internals
    def _get_compressor(self):
        """KVCompressionAdapter built on first use; None without a compression spec."""
        if self._compression_cfg is None:
            return None
        if self._compressor is None:
            from ..compression.manager import KVCompressionAdapter
            self._compressor = KVCompressionAdapter(compression_spec=self._compression_cfg,
                                                    num_kv_heads=self._num_kv_heads, head_size=self._head_size,
                                                    model_name=self._model_name, tp_rank=self._tp_rank,
                                                    tp_size=self._tp_size)
        return self._compressor

    def _resolve_transfer_id(self, request_id: str, request=None) -> str:
        """The router's kv_transfer_params["transfer_id"], shared by both sides;
        the local request id when the router gave none (:650-664)."""
        if request is not None:
            params = getattr(request, "kv_transfer_params", None)
            if params and params.get("transfer_id"):
                self._request_transfer_ids[request_id] = str(params["transfer_id"])
            else:
                _warn_once("Missing transfer_id in kv_transfer_params from router; falling back to local "
                           "request_id. This is only safe for single-process tests.")
        return self._request_transfer_ids.get(request_id, request_id)

    @staticmethod
    def _build_transport(cfg, local_rank: int = 0, channel_rank: int = 0, spec: Optional[str] = None):
        """The transport named by `spec` ("loopback" or "module:Class"), built with
        the reference's NcclTransport constructor arguments (:666-675)."""
        kwargs = dict(is_sender=bool(cfg.is_kv_producer), host=cfg.kv_ip, port=int(cfg.kv_port),
                      local_rank=local_rank, channel_rank=channel_rank,
                      recv_buffer_size=max(1, int(cfg.kv_buffer_size)))
        if spec is None:
            raise NotImplementedError(
                "the ZMQ + NCCL network transport is not part of this engine: set "
                "kv_connector_extra_config['transport_class'] to 'loopback' or to 'module:Class' of a "
                "transport with the NcclTransport methods")
        if spec == "loopback":
            from .transport import LoopbackTransport
            return LoopbackTransport(**kwargs)
        import importlib
        mod, _, name = str(spec).partition(":")
        if not name:
            raise ValueError(f"transport_class must be 'module:Class', got {spec!r}")
        return getattr(importlib.import_module(mod), name)(**kwargs)
