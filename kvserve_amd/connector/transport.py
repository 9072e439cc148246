"""Transports for the compressed-KV connector.

The connector talks to its transport through the method surface of the
reference's NcclTransport (kvserve_v1/transport/nccl_transport.py:83-593):

  producer  send(request_id, layer_names, stacked_kv)
            send_bundle(request_id, layer_names, meta, body_chunks, aux_tensors)
            wait_for_sent(), wait_for_below(max_pending_bytes) -> seconds waited,
            pending_bytes()
  consumer  drain_received() -> {request_id: [(layer_names, payload), ...]}
            payload_nbytes(payload), release_received(request_id, nbytes),
            set_expected_requests(request_ids)
  both      record_stat(row), device

A received bundle is the dict ``{"__bundle__": True, "meta", "body_chunks",
"aux_tensors"}`` (nccl_transport.py:729-735); a failed transfer is delivered as
``([], None)`` (nccl_transport.py:59-60, :562-568).

The ZMQ + NCCL transport itself (a socket control channel and a send thread) is
network plumbing and not part of this engine; a deployment plugs its own class in
through ``kv_connector_extra_config["transport_class"]``.  `LoopbackTransport`
hands payloads from a producer to a consumer inside one process (single-process
disaggregation, benchmarks): the consumer receives the producer's tensors themselves
(copied only when the consumer names another device) and the metadata dict itself.
The hand-off is zero-copy: a producer must not write a sent buffer again, and a
consumer must not mutate the received metadata (the connector does neither).
"""

from __future__ import annotations

import json
import os
import threading
import time
from collections import defaultdict, deque
from typing import Any, Deque, Dict, List, Optional, Tuple

import torch

FAILED_LAYER_NAMES: List[str] = []
FAILED_PAYLOAD: Any = None


def _tensor_nbytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


def payload_nbytes(payload: Any) -> int:
    """Bytes a received payload holds in staging (nccl_transport.py:72-80)."""
    if isinstance(payload, torch.Tensor):
        return _tensor_nbytes(payload)
    if isinstance(payload, dict) and payload.get("__bundle__"):
        return sum(_tensor_nbytes(t) for t in payload["body_chunks"] + payload["aux_tensors"])
    return 0


class _Channel:
    """State shared by the two ends of one loopback channel."""

    def __init__(self, capacity: int):
        self.cv = threading.Condition()
        # sent, not yet admitted by the receiver: (request_id, layer_names, payload, nbytes)
        self.pending: Deque[Tuple[str, List[str], Any, int]] = deque()
        self.pending_bytes = 0
        self.received: Dict[str, Deque[Tuple[List[str], Any]]] = defaultdict(deque)
        self.capacity = capacity
        self.reserved = 0
        self.expected: set = set()
        self.priority: Optional[str] = None
        self.stats: List[Dict[str, Any]] = []


class LoopbackTransport:
    """In-process hand-off between a producer and a consumer connector.

    Both ends name the same (host, port, channel_rank).  `device` is where the
    consumer wants received tensors (its GPU); a payload already there is handed
    over as it is, so the producer must not write a sent buffer again (the
    connector sends freshly allocated ones).  Every send is admitted at once.
    """

    _registry: Dict[Tuple[str, int, int], _Channel] = {}
    _registry_lock = threading.Lock()

    def __init__(self, is_sender: bool, host: str = "127.0.0.1", port: int = 0, local_rank: int = 0,
                 channel_rank: int = 0, recv_buffer_size: int = 1_000_000_000,
                 device: Optional[torch.device] = None):
        self.is_sender = is_sender
        self.local_rank = local_rank
        self.channel_rank = channel_rank
        self.port = port + channel_rank
        if device is None:
            device = torch.device(f"cuda:{local_rank}") if torch.cuda.is_available() else torch.device("cpu")
        self.device = torch.device(device)
        self._stats_path = os.environ.get("KVSERVE_TRANSPORT_STATS_PATH")
        key = (str(host), int(port), int(channel_rank))
        with LoopbackTransport._registry_lock:
            ch = LoopbackTransport._registry.get(key)
            if ch is None:
                ch = LoopbackTransport._registry[key] = _Channel(max(1, int(recv_buffer_size)))
            if not is_sender:
                ch.capacity = max(1, int(recv_buffer_size))
        self._ch = ch
        self._copy_events: List[Any] = []

    @classmethod
    def reset_channels(cls) -> None:
        """Forget every channel (between tests)."""
        with LoopbackTransport._registry_lock:
            LoopbackTransport._registry.clear()

    # ------------------------------------------------------------------ stats
    def record_stat(self, row: Dict[str, Any]) -> None:
        """Append a connector or transport event (nccl_transport.py:447-469); rows
        also go, as JSON lines, to $KVSERVE_TRANSPORT_STATS_PATH when it is set."""
        with self._ch.cv:
            self._stat_locked(row)

    def _stat_locked(self, row: Dict[str, Any]) -> None:
        row = dict(row)
        row.setdefault("time_s", time.time())
        self._ch.stats.append(row)
        if self._stats_path:
            clean = {k: v for k, v in row.items() if not k.startswith("_")}
            try:
                with open(self._stats_path, "a") as f:
                    f.write(json.dumps(clean, sort_keys=True, default=str) + "\n")
            except OSError:
                pass

    @property
    def stats(self) -> List[Dict[str, Any]]:
        with self._ch.cv:
            return list(self._ch.stats)

    # ------------------------------------------------------------------ producer
    def _stage(self, tensors: List[torch.Tensor]) -> List[torch.Tensor]:
        """The tensors as the consumer receives them: themselves on its device, else
        copies there (enqueued on the current stream)."""
        out = []
        for t in tensors:
            if t.device == self.device:
                out.append(t)
                continue
            r = torch.empty(t.shape, dtype=t.dtype, device=self.device)
            r.copy_(t.contiguous(), non_blocking=True)
            out.append(r)
            if t.device.type == "cuda" or self.device.type == "cuda":
                ev = torch.cuda.Event()
                ev.record(torch.cuda.current_stream(t.device if t.device.type == "cuda" else self.device))
                self._copy_events.append(ev)
        return out

    def _post(self, request_id: str, layer_names: List[str], payload: Any, nbytes: int, kind: str) -> None:
        ch = self._ch
        with ch.cv:
            ch.pending.append((request_id, list(layer_names), payload, nbytes))
            ch.pending_bytes += nbytes
            depth, queued = len(ch.pending), ch.pending_bytes
            self._stat_locked({"direction": "send", "kind": kind, "request_id": request_id, "payload_bytes": nbytes,
                               "queue_depth_at_submit": depth, "queued_bytes_at_submit": queued})
            ch.cv.notify_all()

    def send(self, request_id: str, layer_names: List[str], stacked_kv: torch.Tensor) -> None:
        """Queue a raw stacked KV tensor (nccl_transport.py:181-197)."""
        assert self.is_sender
        (t,) = self._stage([stacked_kv])
        self._post(request_id, layer_names, t, _tensor_nbytes(t), "tensor")

    def _meta(self, meta: Dict[str, Any]) -> Dict[str, Any]:
        """The metadata as the consumer receives it: the dict itself (a hand-off)."""
        return meta

    def send_bundle(self, request_id: str, layer_names: List[str], meta: Dict[str, Any],
                    body_chunks: List[torch.Tensor], aux_tensors: List[torch.Tensor]) -> None:
        """Queue a compressed bundle (nccl_transport.py:199-223)."""
        assert self.is_sender
        payload = {"__bundle__": True, "meta": self._meta(meta), "body_chunks": self._stage(list(body_chunks)),
                   "aux_tensors": self._stage(list(aux_tensors))}
        self._post(request_id, layer_names, payload, payload_nbytes(payload), "bundle")

    def wait_for_sent(self) -> None:
        """Block until every queued copy has finished on the device."""
        assert self.is_sender
        for ev in self._copy_events:
            ev.synchronize()
        self._copy_events.clear()

    def wait_for_below(self, max_pending_bytes: int, timeout_s: Optional[float] = None) -> float:
        """Block while more than `max_pending_bytes` wait for the receiver
        (nccl_transport.py:232-239); the consumer takes them from another thread."""
        assert self.is_sender
        t0 = time.perf_counter()
        with self._ch.cv:
            self._ch.cv.wait_for(lambda: self._ch.pending_bytes <= max_pending_bytes, timeout=timeout_s)
        return time.perf_counter() - t0

    def pending_bytes(self) -> int:
        assert self.is_sender
        with self._ch.cv:
            return self._ch.pending_bytes

    def mark_failed(self, request_id: str) -> None:
        """Deliver a failure marker for `request_id` (nccl_transport.py:562-568)."""
        with self._ch.cv:
            self._ch.received[request_id].append((list(FAILED_LAYER_NAMES), FAILED_PAYLOAD))

    # ------------------------------------------------------------------ consumer
    def _admit(self) -> None:
        """Move sent payloads into the received set, in order (all of them: a
        hand-off needs no staging credit).  Called with the channel lock held."""
        ch = self._ch
        while ch.pending:
            rid, names, payload, nbytes = ch.pending.popleft()
            ch.pending_bytes -= nbytes
            ch.received[rid].append((names, payload))
        ch.cv.notify_all()

    def drain_received(self) -> Dict[str, List[Tuple[List[str], Any]]]:
        """Received payloads per request id, each list in arrival order (nccl_transport.py:471-479)."""
        assert not self.is_sender
        with self._ch.cv:
            self._admit()
            out = {k: list(v) for k, v in self._ch.received.items() if v}
            self._ch.received.clear()
        return out

    @staticmethod
    def payload_nbytes(payload: Any) -> int:
        return payload_nbytes(payload)

    def release_received(self, request_id: str, payload_bytes: int) -> None:
        """A payload has been consumed (nccl_transport.py:485-506); a hand-off holds
        no staging to give back."""
        assert not self.is_sender

    def set_expected_requests(self, request_ids: List[str]) -> None:
        """The requests of this step (nccl_transport.py:508-517)."""
        with self._ch.cv:
            self._ch.expected = set(request_ids)
            self._admit()
