"""Codec stage of the fixed-profile runtime (kvserve_v1/compression/runtime/codec.py:15-105).

`EncodedChunk` keeps the reference's fields.  The ANS stage is this engine's rANS
over bytes (w = 8) in the place of nvCOMP ANS.  The stream length is data-dependent:
the encoder writes it on the device, the runtime stream copies it to pinned host
memory, and `codec_bytes` reads it after the chunk's event.  Decoding flags a
corrupt stream the same way; the slot event raises it on `synchronize()`.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Callable, Optional

import torch

from .. import _lib
from ._hip import D2H, H2D, memcpy_async

_RING = 64  # lengths kept in flight per codec


@dataclass
class EncodedChunk:
    array: object
    event: torch.cuda.Event
    u8_bytes: int
    payload_bytes: Optional[int] = None
    raw_tail_bytes: int = 0
    raw_tail_addr: int = 0

    @property
    def codec_bytes(self) -> int:
        if self.payload_bytes is not None:
            return self.payload_bytes
        return int(self.array.buffer_size)  # type: ignore[attr-defined]


class SlotEvent(torch.cuda.Event):
    """Completion event of a slot; `synchronize()` also reports a decode error
    found by the codec for the work the event closes."""

    def __init__(self):
        super().__init__()
        self.check: Optional[Callable[[], None]] = None

    def synchronize(self) -> None:
        super().synchronize()
        check, self.check = self.check, None
        if check is not None:
            check()


class _StreamLength:
    def __init__(self, host: torch.Tensor, index: int, event: torch.cuda.Event):
        self._host, self._index, self._event, self._value = host, index, event, None

    @property
    def buffer_size(self) -> int:
        if self._value is None:
            torch.cuda.Event.synchronize(self._event)
            self._value = int(self._host[self._index])
        return self._value


class ANSCodec:
    """rANS over the packed bytes of one KV part, on the runtime stream, with the
    slot's fixed scratch."""

    def __init__(self, stream: torch.cuda.Stream, packed_sizes, workspace: torch.Tensor):
        self.stream = stream
        self.workspace = workspace
        device = workspace.device
        self._lengths = torch.zeros(_RING, dtype=torch.int64, device=device)
        self._host_lengths = torch.zeros(_RING, dtype=torch.int64, pin_memory=True)
        self._err = torch.zeros(1, dtype=torch.int32, device=device)
        self._host_err = torch.zeros(2, dtype=torch.int32, pin_memory=True)  # [flag, zero]
        self._next = 0
        self._stream_ptr = ctypes.c_void_p(stream.cuda_stream)
        self._lib = _lib.load()
        self._enc_jobs = {}
        self.capacities = {n: int(self._lib.kvmi_rans_max_bytes(n, 8)) for n in set(packed_sizes)}

    def encode(self, source: torch.Tensor, output: torch.Tensor, u8_bytes: int,
               event: torch.cuda.Event) -> EncodedChunk:
        i = self._next
        self._next = (i + 1) % _RING
        length = self._lengths.data_ptr() + 8 * i
        key = (source.data_ptr(), u8_bytes, output.data_ptr(), output.numel())
        job = self._enc_jobs.get(key)
        if job is None:
            job = self._enc_jobs[key] = _lib.RansEncJob(source.data_ptr(), u8_bytes, output.data_ptr(),
                                                        output.numel(), self.workspace.data_ptr(),
                                                        self.workspace.numel(), length)
        job.out_len = length
        _lib.check(self._lib.kvmi_rans_encode_batch(ctypes.byref(job), 1, 8, self._stream_ptr),
                   "kvmi_rans_encode_batch")
        memcpy_async(self._host_lengths.data_ptr() + 8 * i, length, 8, D2H, self.stream.cuda_stream)
        event.record(self.stream)
        return EncodedChunk(_StreamLength(self._host_lengths, i, event), event, u8_bytes)

    def decode(self, source: torch.Tensor, output: torch.Tensor, codec_bytes: int, u8_bytes: int,
               event: torch.cuda.Event) -> torch.cuda.Event:
        sp = self.stream.cuda_stream
        # the error flag starts from zero: a copy of the pinned zero word
        memcpy_async(self._err.data_ptr(), self._host_err.data_ptr() + 4, 4, H2D, sp)
        job = _lib.RansDecJob(source.data_ptr(), codec_bytes, u8_bytes, output.data_ptr())
        _lib.check(self._lib.kvmi_rans_decode_batch(ctypes.byref(job), 1, 8, self._err.data_ptr(), self._stream_ptr),
                   "kvmi_rans_decode_batch")
        memcpy_async(self._host_err.data_ptr(), self._err.data_ptr(), 4, D2H, sp)
        if isinstance(event, SlotEvent):
            event.check = self.check
        event.record(self.stream)
        return event

    def check(self) -> None:
        """Raise when the last decode (already synchronized) met a corrupt stream."""
        from ..engine import raise_device_error

        code = int(self._host_err[0])
        if code:
            raise_device_error(code)
