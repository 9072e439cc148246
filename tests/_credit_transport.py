"""Test transport: a loopback that adds what a network transport does on the way.

The metadata goes through msgpack (as on the control channel of
kvserve_v1/transport/nccl_transport.py), the consumer copies every payload into
staging on its device, and admits it only with receive credit by the rules of
nccl_transport.py:508-560.  The connector's load loop and the wire's msgpack safety
are tested against it; it is not part of the engine.
"""

from __future__ import annotations

from typing import Any, Dict, List

import msgpack
import torch

from kvserve_amd.connector.transport import LoopbackTransport


class CreditLoopbackTransport(LoopbackTransport):
    """Test infrastructure: a loopback whose consumer copies every payload into
    staging on its device and admits it only with receive credit, by the rules of
    nccl_transport.py:508-560 -- admitted when the staging is empty, when it fits, or
    once as the scheduled request allowed past the budget (`recv_buffer_size` is the
    staging capacity).  The metadata goes through msgpack as on the network
    transport's control channel, so a bundle that would not serialize fails here.
    The connector's load loop is tested against these rules."""

    def _meta(self, meta: Dict[str, Any]) -> Dict[str, Any]:
        return msgpack.unpackb(msgpack.packb(meta, use_bin_type=True), raw=False)

    def _stage(self, tensors: List[torch.Tensor]) -> List[torch.Tensor]:
        out = []
        for t in tensors:
            r = torch.empty(t.shape, dtype=t.dtype, device=self.device)
            r.copy_(t.contiguous(), non_blocking=True)
            out.append(r)
        if self.device.type == "cuda":
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(self.device))
            self._copy_events.append(ev)
        return out

    def _try_reserve(self, request_id: str, nbytes: int) -> bool:
        """Called with the channel lock held."""
        ch = self._ch
        over = ch.reserved > 0 and ch.reserved + nbytes > ch.capacity
        if over:
            if request_id in ch.expected and ch.priority is None:
                ch.priority = request_id
            else:
                return False
        before = ch.reserved
        ch.reserved += nbytes
        self._stat_locked({"direction": "recv_credit", "kind": "reserve", "request_id": request_id,
                           "payload_bytes": nbytes, "blocked": over, "reserved_before_bytes": before,
                           "reserved_after_bytes": ch.reserved, "capacity_bytes": ch.capacity,
                           "oversize": nbytes > ch.capacity, "priority_overflow": request_id == ch.priority})
        return True

    def _admit(self) -> None:
        ch = self._ch
        while ch.pending:
            rid, names, payload, nbytes = ch.pending[0]
            if not self._try_reserve(rid, nbytes):
                break
            ch.pending.popleft()
            ch.pending_bytes -= nbytes
            ch.received[rid].append((names, payload))
        ch.cv.notify_all()

    def release_received(self, request_id: str, payload_bytes: int) -> None:
        """Return staging credit once a payload has been consumed (nccl_transport.py:485-506)."""
        assert not self.is_sender
        if payload_bytes <= 0:
            return
        ch = self._ch
        with ch.cv:
            before = ch.reserved
            ch.reserved = max(0, ch.reserved - int(payload_bytes))
            if request_id == ch.priority:
                ch.priority = None
            self._stat_locked({"direction": "recv_credit_release", "kind": "release", "request_id": request_id,
                               "payload_bytes": int(payload_bytes), "reserved_before_bytes": before,
                               "reserved_after_bytes": ch.reserved, "capacity_bytes": ch.capacity})
            self._admit()
