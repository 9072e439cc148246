"""CPU restatement of the fixed-profile runtime's numerics -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker.  The product (kvserve_amd.runtime) never does.

numpy, float32 arithmetic with an explicit round-to-nearest-even to bf16 after every
operation the reference performs on bf16 tensors:

  gather / head order   kvserve_v1/compression/runtime/pipeline.py:224-262
  signs, FWHT           pipeline.py:264-309 (two-buffer butterflies, bf16 per stage,
                        increasing index bit, then * (1 / sqrt(D)))
  quantize              pipeline.py:430-469 (amin / amax, rn(max - min) floored at
                        1e-5, scale = rn(raw / (L - 1)), inverse = rn(1 / scale),
                        q = clamp(round(rn(rn(x - min) * inverse)), 0, L - 1))
  aux                   min / scale at the section offsets, first half of the arena
  raw tails             pipeline.py:353-428 ([heads, count, channels] per tail block;
                        decode clears the tail blocks first)
  dequantize, inverse   pipeline.py:671-703 (rn(rn(q * scale) + min), FWHT, signs,
                        scatter through the head order)

Pinned by tests/test_runtime_oracle.py against the reference's own CPU runtime
(tests/golden/runtime.npz, written by tests/golden/make_runtime_golden.py), the
Sylvester closed form, the Walsh functions of unit vectors, and the reference
tests' quantizer formulas (tests/runtime/test_gpu.py:412-535).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

import numpy as np

AXES = ("channel", "token", "tensor")


def rn(x) -> np.ndarray:
    """float32 -> nearest bf16 (ties to even), returned as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)).view(np.float32)
    return np.where(np.isnan(x), x, r)


def from_bits(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def to_bits(x) -> np.ndarray:
    return (rn(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def fwht(rows: np.ndarray) -> np.ndarray:
    """Normalized FWHT over the last axis, bf16 after every butterfly stage (pipeline.py:285-309)."""
    v = rn(rows)
    d = v.shape[-1]
    lead = v.shape[:-1]
    step = 1
    while step < d:
        pairs = v.reshape(*lead, d // (2 * step), 2, step)
        a, b = pairs[..., 0, :], pairs[..., 1, :]
        v = np.stack((rn(a + b), rn(a - b)), axis=-2).reshape(*lead, d)
        step *= 2
    return rn(v * np.float32(1.0 / np.sqrt(np.float64(d))))


def quant_params(mn: np.ndarray, mx: np.ndarray, levels: int) -> Tuple[np.ndarray, np.ndarray]:
    """(scale, inverse) of pipeline.py:455-460."""
    raw = rn(np.float32(mx) - np.float32(mn))
    raw = np.where(raw < np.float32(1e-5), rn(np.float32(1e-5)), raw)
    scale = rn(raw / np.float32(levels - 1))
    return scale, rn(np.float32(1.0) / scale)


def quantize(x: np.ndarray, mn: np.ndarray, inverse: np.ndarray, levels: int) -> np.ndarray:
    q = np.rint(rn(rn(x - mn) * inverse))
    return np.clip(q, 0, levels - 1).astype(np.uint8)


def dequantize(q: np.ndarray, mn: np.ndarray, scale: np.ndarray) -> np.ndarray:
    return rn(rn(q.astype(np.float32) * scale) + mn)


@dataclass
class Section:
    head_start: int
    head_count: int
    levels: int
    axis: str
    aux_min_offset: int
    aux_scale_offset: int


@dataclass
class LayerPart:
    """One layer's K or V part.  `cache` holds bf16 bits [blocks, heads, kernel_tokens,
    channels]; the part is channels [channel_offset, channel_offset + head_size)."""

    cache: np.ndarray
    channel_offset: int
    head_size: int
    order: Sequence[int]
    u8_offset: int
    signs: Optional[np.ndarray] = None  # [heads, head_size] of +-1 in output-head order
    sections: List[Section] = field(default_factory=list)


def _tail_blocks(phys: Sequence[int], tokens: int, block_size: int, bpl: int):
    tail = tokens % block_size
    if not tail:
        return []
    kt = block_size // bpl
    return [(b, max(0, min(tail - i * kt, kt))) for i, b in enumerate(phys[-bpl:])]


def _aux_put(aux: np.ndarray, offset: int, values: np.ndarray) -> None:
    b = to_bits(values).reshape(-1).view(np.uint8)
    aux[offset:offset + b.size] = b


def _aux_get(aux: np.ndarray, offset: int, count: int) -> np.ndarray:
    return from_bits(aux[offset:offset + 2 * count].view(np.uint16))


def _canonical(part: LayerPart, ids: Sequence[int]) -> np.ndarray:
    x = from_bits(part.cache[list(ids)][..., part.channel_offset:part.channel_offset + part.head_size])
    return x[:, list(part.order)].transpose(0, 2, 1, 3)  # [blocks, tokens, heads, channels]


def encode_part(parts: Sequence[LayerPart], phys: Sequence[int], tokens: int, block_size: int, bpl: int,
                transform: bool, quantize_: bool, u8_bytes: int, aux_bytes: int
                ) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(payload[u8_bytes], aux[aux_bytes], raw tail) of one KV part of one chunk
    (pipeline.py:557-669 without the codec stage)."""
    payload = np.zeros(u8_bytes, dtype=np.uint8)
    aux = np.zeros(aux_bytes, dtype=np.uint8)
    tails = []
    body_blocks = tokens // block_size * bpl
    for part in parts:
        for b, count in _tail_blocks(phys, tokens, block_size, bpl):
            if count <= 0:
                break
            window = part.cache[b][:, :count, part.channel_offset:part.channel_offset + part.head_size]
            tails.append(np.ascontiguousarray(window).view(np.uint8).reshape(-1))
        if not body_blocks or not u8_bytes:
            continue
        x = _canonical(part, phys[:body_blocks])
        if transform:
            x = fwht(rn(x * part.signs.astype(np.float32)))
        if not quantize_:
            b = to_bits(x).reshape(-1).view(np.uint8)
            payload[2 * part.u8_offset:2 * part.u8_offset + b.size] = b
            continue
        q = np.zeros(x.shape, dtype=np.uint8)
        for s in part.sections:
            sub = x[:, :, s.head_start:s.head_start + s.head_count, :]
            axes = {"channel": (0, 1), "token": (2, 3), "tensor": (0, 1, 2, 3)}[s.axis]
            mn, mx = sub.min(axis=axes, keepdims=True), sub.max(axis=axes, keepdims=True)
            scale, inverse = quant_params(mn, mx, s.levels)
            q[:, :, s.head_start:s.head_start + s.head_count, :] = quantize(sub, mn, inverse, s.levels)
            _aux_put(aux, s.aux_min_offset, mn)
            _aux_put(aux, s.aux_scale_offset, scale)
        flat = q.reshape(-1)
        payload[part.u8_offset:part.u8_offset + flat.size] = flat
    tail = np.concatenate(tails) if tails else np.zeros(0, dtype=np.uint8)
    return payload, aux, tail


def decode_part(parts: Sequence[LayerPart], phys: Sequence[int], tokens: int, block_size: int, bpl: int,
                transform: bool, quantize_: bool, payload: np.ndarray, aux: np.ndarray, tail: np.ndarray) -> None:
    """Restore one KV part of one chunk into each part's `cache` in place (pipeline.py:705-804)."""
    body_blocks = tokens // block_size * bpl
    offset = 0
    for part in parts:
        c0, c1 = part.channel_offset, part.channel_offset + part.head_size
        if body_blocks and payload.size:
            ids = list(phys[:body_blocks])
            kt = part.cache.shape[2]
            heads = part.cache.shape[1]
            shape = (body_blocks, kt, heads, part.head_size)
            if quantize_:
                n = int(np.prod(shape))
                q = payload[part.u8_offset:part.u8_offset + n].reshape(shape)
                y = np.zeros(shape, dtype=np.float32)
                for s in part.sections:
                    hs = slice(s.head_start, s.head_start + s.head_count)
                    if s.axis == "channel":
                        pshape, count = (1, 1, s.head_count, part.head_size), s.head_count * part.head_size
                    elif s.axis == "token":
                        pshape, count = (body_blocks, kt, 1, 1), body_blocks * kt
                    else:
                        pshape, count = (1, 1, 1, 1), 1
                    mn = _aux_get(aux, s.aux_min_offset, count).reshape(pshape)
                    scale = _aux_get(aux, s.aux_scale_offset, count).reshape(pshape)
                    y[:, :, hs, :] = dequantize(q[:, :, hs, :], mn, scale)
            else:
                n = int(np.prod(shape))
                y = from_bits(payload[2 * part.u8_offset:2 * part.u8_offset + 2 * n].view(np.uint16)).reshape(shape)
            if transform:
                y = rn(fwht(y) * part.signs.astype(np.float32))
            restored = to_bits(y).transpose(0, 2, 1, 3)  # [blocks, heads(output order), tokens, channels]
            for j, b in enumerate(ids):
                for h, original in enumerate(part.order):
                    part.cache[b, original, :, c0:c1] = restored[j, h]
        for b, count in _tail_blocks(phys, tokens, block_size, bpl):
            part.cache[b, :, :, c0:c1] = 0
            if count <= 0:
                continue
            heads = part.cache.shape[1]
            n = heads * count * part.head_size * 2
            part.cache[b, :, :count, c0:c1] = tail[offset:offset + n].view(np.uint16).reshape(heads, count,
                                                                                               part.head_size)
            offset += n
