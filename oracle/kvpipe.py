"""numpy restatement of KVServe's modular compression pipeline (test oracle).

TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.  bf16 tensors are carried as
uint16 bit patterns; every elementwise bf16 op of the reference is computed in
float32 (IEEE round-to-nearest-even, as torch does on CPU and GPU) and rounded to
bf16 before the next op.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

HEADER_BYTES = 16
MAGIC = 0x0150424B
CHUNK_THRESHOLD_BYTES = 500 * 1024 * 1024  # compression_manager.py:230-231
CHUNK_LAYERS = 8  # compression_manager.py:235


# ------------------------------------------------------------------ bf16
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round-to-nearest-even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u >> 16) & 1) + np.uint32(0x7FFF)
    return ((u + r) >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rbf(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bf16 values (kept as float32)."""
    return bf16_to_f32(f32_to_bf16(x))


# ------------------------------------------------------------------ signs
def rademacher_signs(base_seed: int, layer_id: int, num_heads: int, head_dim: int) -> np.ndarray:
    """[H, D] float32 of +-1.  hadamard_func.py:33-48 and :137-152: one CPU generator
    re-seeded with base_seed ^ (layer << 16) ^ head, then randint(0, 2, (D,), int8)*2-1."""
    import torch

    gen = torch.Generator(device="cpu")
    rows = []
    for h in range(num_heads):
        gen.manual_seed(base_seed ^ (layer_id << 16) ^ h)
        s = torch.randint(0, 2, (head_dim,), generator=gen, dtype=torch.int8)
        rows.append(s.numpy().astype(np.float32) * 2 - 1)
    return np.stack(rows)


def sign_bits(signs: np.ndarray) -> np.ndarray:
    """[H, D] +-1 -> [H, ceil(D/32)] uint32, bit (d % 32) of word d // 32 set when the
    sign is -1 (bits past D are 0)."""
    H, D = signs.shape
    W = (D + 31) // 32
    neg = np.zeros((H, W * 32), np.uint64)
    neg[:, :D] = signs < 0
    w = neg.reshape(H, W, 32) << np.arange(32, dtype=np.uint64)
    return w.sum(axis=2).astype(np.uint32)


# ------------------------------------------------------------------ FWHT
def fwht_f32(x: np.ndarray) -> np.ndarray:
    """Unnormalised Walsh-Hadamard transform over the last axis in float32, natural
    (Sylvester) order, radix-2 stages from the lowest index bit up."""
    y = np.array(x, dtype=np.float32, copy=True)
    D = y.shape[-1]
    assert D & (D - 1) == 0, "power-of-two head_dim"
    lead = y.shape[:-1]
    h = 1
    while h < D:
        v = y.reshape(*lead, D // (2 * h), 2, h)
        a = v[..., 0, :].copy()
        b = v[..., 1, :]
        v[..., 0, :] = a + b
        v[..., 1, :] = a - b
        h *= 2
    return y


def _scale(D: int) -> np.float32:
    return np.float32(1.0 / math.sqrt(D))  # hadamard_func.py:98 scale=1/sqrt(size)


def pow2_chunks(D: int) -> List[int]:
    """hadamard_func.py:50-71: D as descending powers of two (96 -> [64, 32])."""
    return [1 << b for b in range(D.bit_length() - 1, -1, -1) if D >> b & 1]


def fwht_scaled_f32(x: np.ndarray) -> np.ndarray:
    """hadamard_func.py:73-103 before the bf16 rounding: each power-of-two chunk of the
    last axis transformed on its own (fwht_f32) and scaled by 1/sqrt(chunk)."""
    out, start = [], 0
    for c in pow2_chunks(x.shape[-1]):
        out.append(fwht_f32(x[..., start:start + c]) * _scale(c))
        start += c
    return np.concatenate(out, axis=-1)


def hadamard_forward(x_bits: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """bf16 [..., H, D] -> bf16.  hadamard_func.py:161-197: x*s (exact in bf16), FWHT of
    each power-of-two chunk with scale 1/sqrt(chunk) in fp32, one bf16 rounding."""
    x = bf16_to_f32(x_bits) * signs
    return f32_to_bf16(fwht_scaled_f32(x))


def hadamard_inverse(y_bits: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """hadamard_func.py:199-231: chunked FWHT (rounded to bf16) first, then * signs."""
    z = rbf(fwht_scaled_f32(bf16_to_f32(y_bits)))
    return f32_to_bf16(z * signs)


# ------------------------------------------------------------------ quantizer
_FLOOR = float(bf16_to_f32(f32_to_bf16(np.array([1e-5], np.float32)))[0])


def section_scale(mn: np.ndarray, mx: np.ndarray, max_value: int) -> np.ndarray:
    """quantizer_func.py:56: bf16 (max-min).clamp_(min=1e-5).div_(max_value-1)."""
    d = rbf(mx - mn)
    d = np.where(d < np.float32(1e-5), np.float32(_FLOOR), d).astype(np.float32)
    return rbf(d / np.float32(max_value - 1))


def quantize(max_value: int, x: np.ndarray, axis: str) -> Tuple[np.ndarray, Optional[np.ndarray], Optional[np.ndarray]]:
    """quantizer_func.py:9-75 on a bf16-valued float32 tensor [B, S, Hg, D].
    Returns (uint8 symbols, min, scale) with min/scale keepdim-shaped bf16 values,
    or (empty, None, None) for an empty section."""
    if x.size == 0:
        return x.astype(np.uint8), None, None
    dims = {"channel": (0, 1), "token": (2, 3), "tensor": (0, 1, 2, 3)}[axis]
    mx = x.max(axis=dims, keepdims=True)
    mn = x.min(axis=dims, keepdims=True)
    sc = section_scale(mn, mx, max_value)
    t = rbf(x - mn)
    q = rbf(t / sc)
    sym = np.clip(np.rint(q), 0, max_value).astype(np.uint8)
    return sym, mn, sc


def dequantize(sym: np.ndarray, mn: Optional[np.ndarray], sc: Optional[np.ndarray]) -> np.ndarray:
    """quantizer_func.py:77-113: bf16(bf16(q * scale) + min)."""
    q = sym.astype(np.float32)
    if mn is None:
        return q
    return rbf(rbf(q * sc) + mn)


# ------------------------------------------------------------------ masks / profiles
def head_mask_from_scores(scores: np.ndarray, hybrid_ratio: float) -> np.ndarray:
    """kvserve_quantizer.py:58-63: the round(numel*ratio) lowest scores are low precision."""
    n_low = int(round(scores.size * hybrid_ratio))
    flat = np.argsort(scores.reshape(-1), kind="stable")[:n_low]
    mask = np.zeros(scores.size, dtype=bool)
    mask[flat] = True
    return mask.reshape(scores.shape)


def layer_mask(num_layers: int) -> np.ndarray:
    """kvserve_quantizer.py:65-68: the last round(0.33*L) layers are low precision."""
    m = np.zeros(num_layers, dtype=bool)
    n = int(round(num_layers * 0.33))
    if n:
        m[-n:] = True
    return m


@dataclass
class PartProfile:
    """Output head order, levels and V statistic groups of one part of one layer."""

    order: List[int]   # source head at output position j
    levels: List[int]  # max_value at output position j
    group: List[int]   # statistic group of output position j (contiguous runs)


@dataclass
class LayerProfile:
    k: PartProfile
    v: PartProfile


def head_split_profile(low_mask_row: Sequence[bool], hk: int, hv: int, lk: int, lv: int) -> LayerProfile:
    """split_func.py:40-72 + kvserve_quantizer.py:210-220: [low asc, high asc]."""
    low = [h for h, m in enumerate(low_mask_row) if m]
    high = [h for h, m in enumerate(low_mask_row) if not m]
    order = low + high
    grp = [0] * len(low) + [1 if low else 0] * len(high)
    return LayerProfile(
        PartProfile(order, [lk] * len(low) + [hk] * len(high), grp),
        PartProfile(order, [lv] * len(low) + [hv] * len(high), grp),
    )


def layer_split_profile(is_low: bool, H: int, hk: int, hv: int, lk: int, lv: int) -> LayerProfile:
    """split_func.py:9-38: the whole layer is one section."""
    order = list(range(H))
    return LayerProfile(
        PartProfile(order, [lk if is_low else hk] * H, [0] * H),
        PartProfile(order, [lv if is_low else hv] * H, [0] * H),
    )


# ------------------------------------------------------------------ one layer
AXES = ("channel", "token", "tensor")
DEFAULT_AXES = ("channel", "token")  # (axis_key, axis_value), kvserve_quantizer.py defaults


@dataclass
class LayerMeta:
    """Quantization metadata of one layer as bf16 values (float32 arrays), per part by
    its axis: "channel" [H', D] by output position; "token" [G, B*S] by statistic
    group; "tensor" [G, 1] by group.  (kmin, kscale) for K, (vmin, vscale) for V."""

    kmin: np.ndarray
    kscale: np.ndarray
    vmin: np.ndarray
    vscale: np.ndarray


def _group_runs(part: PartProfile) -> List[Tuple[int, int]]:
    """[lo, hi) output positions of each statistic group, in group order."""
    runs = []
    for g in sorted(set(part.group)):
        js = [j for j, gg in enumerate(part.group) if gg == g]
        assert js == list(range(js[0], js[-1] + 1)), "groups are contiguous runs of output positions"
        runs.append((js[0], js[-1] + 1))
    return runs


def quantize_part(x: np.ndarray, part: PartProfile, axis: str) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """KVServeQuantizer.quantize's section loop (kvserve_quantizer.py:202-214) for one
    part: x bf16-valued float32 [B, S, H, D] in output order; quantizer_func.quantize on
    each section with its axis (quantizer_func.py:41-49).  A channel-axis section has
    per-(head, channel) statistics, so each head is its own section there."""
    B, S, H, D = x.shape
    out = np.empty(x.shape, np.uint8)
    if axis == "channel":
        mn_t, sc_t = np.empty((H, D), np.float32), np.empty((H, D), np.float32)
        for j in range(H):
            sym, mn, sc = quantize(part.levels[j], x[:, :, j:j + 1, :], "channel")
            out[:, :, j:j + 1, :] = sym
            mn_t[j], sc_t[j] = mn[0, 0, 0], sc[0, 0, 0]
        return out, mn_t, sc_t
    runs = _group_runs(part)
    n = B * S if axis == "token" else 1
    mn_t, sc_t = np.empty((len(runs), n), np.float32), np.empty((len(runs), n), np.float32)
    for g, (lo, hi) in enumerate(runs):
        sym, mn, sc = quantize(part.levels[lo], x[:, :, lo:hi, :], axis)
        out[:, :, lo:hi, :] = sym
        mn_t[g], sc_t[g] = mn.reshape(-1), sc.reshape(-1)
    return out, mn_t, sc_t


def dequantize_part(sym: np.ndarray, part: PartProfile, axis: str, mn_t: np.ndarray,
                    sc_t: np.ndarray) -> np.ndarray:
    """quantizer_func.dequantize (quantizer_func.py:77-113) of each section of one part;
    returns bf16-valued float32 [B, S, H, D] in output order."""
    B, S, H, D = sym.shape
    if axis == "channel":
        return dequantize(sym, mn_t[None, None], sc_t[None, None])
    out = np.empty(sym.shape, np.float32)
    for g, (lo, hi) in enumerate(_group_runs(part)):
        shape = (B, S, 1, 1) if axis == "token" else (1, 1, 1, 1)
        out[:, :, lo:hi, :] = dequantize(sym[:, :, lo:hi, :], mn_t[g].reshape(shape), sc_t[g].reshape(shape))
    return out


def quantize_layer(y: np.ndarray, prof: LayerProfile,
                   axes: Tuple[str, str] = DEFAULT_AXES) -> Tuple[np.ndarray, LayerMeta]:
    """KVServeQuantizer.quantize (kvserve_quantizer.py:171-233) generalised to any
    number of contiguous statistic groups: K with axes[0], V with axes[1] (default K
    per channel, V per token over the heads of a group).  y: bf16-valued float32
    [2, B, S, H, D].  Returns uint8 [2, B, S, H', D] with heads in output order, and
    metadata."""
    out = np.empty(y.shape, dtype=np.uint8)
    out[0], kmin, ksc = quantize_part(y[0][:, :, prof.k.order, :], prof.k, axes[0])
    out[1], vmin, vsc = quantize_part(y[1][:, :, prof.v.order, :], prof.v, axes[1])
    return out, LayerMeta(kmin, ksc, vmin, vsc)


def dequantize_layer(sym: np.ndarray, meta: LayerMeta, prof: LayerProfile,
                     axes: Tuple[str, str] = DEFAULT_AXES) -> np.ndarray:
    """KVServeQuantizer.dequantize (kvserve_quantizer.py:235-294): returns bf16-valued
    float32 [2, B, S, H, D] in source head order."""
    out = np.empty(sym.shape, np.float32)
    out[0][:, :, prof.k.order, :] = dequantize_part(sym[0], prof.k, axes[0], meta.kmin, meta.kscale)
    out[1][:, :, prof.v.order, :] = dequantize_part(sym[1], prof.v, axes[1], meta.vmin, meta.vscale)
    return out


# ------------------------------------------------------------------ bitpack
def bitpack_encode(sym: np.ndarray, bits: int) -> np.ndarray:
    """bitpack_codec.py:24-47,100-110: header + LSB-first packing of the flattened symbols."""
    s = np.ascontiguousarray(sym, dtype=np.uint8).reshape(-1)
    if np.any(s >> bits):
        raise ValueError("symbol exceeds bitpack_bits")
    n = s.size
    hdr = np.zeros(HEADER_BYTES, np.uint8)
    hdr[0:4] = np.frombuffer(np.uint32(MAGIC).tobytes(), np.uint8)
    hdr[4] = bits
    hdr[8:16] = np.frombuffer(np.uint64(n).tobytes(), np.uint8)
    if n == 0:
        return hdr
    bitsarr = np.unpackbits(s[:, None], axis=1, count=bits, bitorder="little").reshape(-1)
    payload = np.packbits(bitsarr, bitorder="little")
    assert payload.size == (n * bits + 7) // 8
    return np.concatenate([hdr, payload])


def bitpack_decode(stream: np.ndarray, n: int, bits: int) -> np.ndarray:
    """bitpack_codec.py:50-69,112-135 (header and length checked)."""
    stream = np.asarray(stream, np.uint8)
    if stream.size != HEADER_BYTES + (n * bits + 7) // 8:
        raise ValueError("BitPackCodec payload length does not match shape and bit width")
    expect = bitpack_encode(np.zeros(0, np.uint8), bits)
    expect[8:16] = np.frombuffer(np.uint64(n).tobytes(), np.uint8)
    if not np.array_equal(stream[:HEADER_BYTES], expect):
        raise ValueError("invalid bitpack header or decode configuration")
    if n == 0:
        return np.zeros(0, np.uint8)
    b = np.unpackbits(stream[HEADER_BYTES:], bitorder="little")[: n * bits].reshape(n, bits)
    return (b.astype(np.uint8) << np.arange(bits, dtype=np.uint8)).sum(axis=1).astype(np.uint8)


# ------------------------------------------------------------------ paged I/O
def gather_blocks(pool: np.ndarray, block_ids: Sequence[int]) -> np.ndarray:
    """kv_utils.py:59-80 (FlashAttention NHD layout): kv[:, idx].clone()."""
    return pool[:, np.asarray(block_ids, dtype=np.int64)].copy()


def scatter_blocks(pool: np.ndarray, payload: np.ndarray, block_ids: Sequence[int]) -> None:
    """kv_utils.py:83-119: kv[:, idx[:num_blocks]] = payload."""
    idx = np.asarray(block_ids, dtype=np.int64)[: payload.shape[1]]
    pool[:, idx] = payload


# ------------------------------------------------------------------ request level
def chunk_ranges(num_layers: int, raw_bytes: int) -> List[Tuple[int, int]]:
    """compression_manager.py:229-235, :383-390: one chunk, or 8-layer chunks above 500 MiB."""
    if raw_bytes > CHUNK_THRESHOLD_BYTES:
        return [(s, min(s + CHUNK_LAYERS, num_layers)) for s in range(0, num_layers, CHUNK_LAYERS)]
    return [(0, num_layers)]


@dataclass
class Chunk:
    start: int
    stop: int
    symbols: np.ndarray       # uint8 codec buffer [l, 2, H', B, S, D] (permuted) or [l,2,B,S,H',D]
    stream: np.ndarray        # packed bytes with header
    metas: List[LayerMeta]


def compress_request(
    pools: Sequence[np.ndarray],
    block_ids: Sequence[int],
    profiles: Sequence[LayerProfile],
    base_seed: int,
    bits: int,
    transform: bool = True,
    layout: str = "permuted",
    layer_ids: Optional[Sequence[int]] = None,
    chunks: Optional[Sequence[Tuple[int, int]]] = None,
    axes: Tuple[str, str] = DEFAULT_AXES,
) -> List[Chunk]:
    """Gather every layer (kv_utils.py:59-80), then compress_all_layers
    (compression_manager.py:200-537): per layer transform (KVServeTransformer,
    kvserve_transformer.py:268-274) and quantize, codec-buffer layout (:155-164),
    and one bitpack stream per chunk.  layer_ids: sign seed layer of each pool
    (default 0..L-1); chunks: explicit layer ranges (default: the reference's rule)."""
    L = len(pools)
    _, _, S, H, D = pools[0].shape
    B = len(block_ids)
    raw = L * 2 * B * S * H * D * 2
    lids = list(range(L)) if layer_ids is None else list(layer_ids)
    out = []
    for s, e in (chunk_ranges(L, raw) if chunks is None else chunks):
        syms, metas = [], []
        for l in range(s, e):
            x = gather_blocks(pools[l], block_ids)
            if transform:
                sg = rademacher_signs(base_seed, lids[l], H, D)
                y = np.stack([bf16_to_f32(hadamard_forward(x[p], sg)) for p in (0, 1)])
            else:
                y = bf16_to_f32(x)
            sym, meta = quantize_layer(y, profiles[l], axes)
            syms.append(sym.transpose(0, 3, 1, 2, 4) if layout == "permuted" else sym)
            metas.append(meta)
        buf = np.ascontiguousarray(np.stack(syms))
        out.append(Chunk(s, e, buf, bitpack_encode(buf, bits), metas))
    return out


def decompress_request(
    chunks: Sequence[Chunk],
    pools: Sequence[np.ndarray],
    block_ids: Sequence[int],
    profiles: Sequence[LayerProfile],
    base_seed: int,
    bits: int,
    transform: bool = True,
    layout: str = "permuted",
    layer_ids: Optional[Sequence[int]] = None,
    axes: Tuple[str, str] = DEFAULT_AXES,
) -> None:
    """decompress_all_layers (compression_manager.py:539-757) then
    inject_kv_into_layer_by_blocks (kv_utils.py:83-119), into `pools` in place."""
    lids = list(range(len(pools))) if layer_ids is None else list(layer_ids)
    for ch in chunks:
        shape = ch.symbols.shape
        buf = bitpack_decode(ch.stream, int(np.prod(shape)), bits).reshape(shape)
        for i, l in enumerate(range(ch.start, ch.stop)):
            sym = buf[i].transpose(0, 2, 3, 1, 4) if layout == "permuted" else buf[i]
            x = dequantize_layer(sym, ch.metas[i], profiles[l], axes)
            H, D = x.shape[-2], x.shape[-1]
            if transform:
                sg = rademacher_signs(base_seed, lids[l], H, D)
                xb = np.stack([hadamard_inverse(f32_to_bf16(x[p]), sg) for p in (0, 1)])
            else:
                xb = f32_to_bf16(x)
            scatter_blocks(pools[l], xb, block_ids)
