"""numpy restatement of KVServe's TileLang fused quantizer numerics (test oracle).

TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.  This is the arithmetic of
quantizer_config.impl = "tilelang_fused": KVHadamardQuantOp.compress_v3 /
decompress_v3 (kvserve_v1/tilelang_ops/kv_hadamard_quant.py:1519-1599, :1645-1750)
behind TileLangFusedQuantizer (kvserve_v1/compression/quantizer/tilelang_quantizer.py).
It differs from the modular quantizer (oracle/kvpipe.py):

  transform  y = FWHT_fp32(x * s) * (1/sqrt(D)), kept in fp32       :521-596, :598-663
             had = bf16(y) is what gets quantized                     :583-586, :647-650
  K          per-(head, channel) min / max of the fp32 y over all rows :571-594, :1303-1304
             sc = max(max - min, 1e-5) / (L - 1)  (fp32)               :894-899, :1313
  V          per-(row, head) min / max of y over D                    :652-659
             grouped over the heads of equal L (first-occurrence order) :1382-1397, :1143-1156
             sc = max(gmax - gmin, 1e-5) / (L - 1)  (fp32)             :1158-1163
  quantize   q = clamp(round((f32(had) - min) / sc), 0, L)             :914-919, :1172-1178
             no head reordering; L per head from the CSV mask
  wire meta  min / scale converted to float16 (tilelang_quantizer.py:23-53)
  dequant    x = q * sc16 + min16 in fp32, FWHT_fp32, * (1/sqrt(D)) * s, bf16 :685-716

Two choices are made by the TileLang / nvcc lowering, not by the reference's source,
and are therefore parity-unpinned here: T.round is taken as round-half-away-from-zero
(TVM lowers tir.round to roundf for CUDA), and the dequant q * sc + min as one fused
multiply-add (nvcc contracts a*b + c by default).  Both only decide exact ties.
"""

from __future__ import annotations

import math
from typing import Dict, Sequence, Tuple

import numpy as np

from .kvpipe import bf16_to_f32, f32_to_bf16, fwht_f32

FLOOR = np.float32(1e-5)  # T.max(..., 1e-5) / clamp_(min=1e-5) on float32


def round_half_away(v: np.ndarray) -> np.ndarray:
    """roundf: nearest integer, ties away from zero (computed exactly in float64)."""
    d = np.asarray(v, dtype=np.float64)
    return (np.sign(d) * np.floor(np.abs(d) + 0.5)).astype(np.float32)


def group_map(max_vals: Sequence[float]) -> np.ndarray:
    """Group id of every head: heads with equal L share a group, ids in order of
    first occurrence (kv_hadamard_quant.py:1382-1390)."""
    ids: Dict[float, int] = {}
    return np.array([ids.setdefault(float(v), len(ids)) for v in max_vals], dtype=np.int32)


def transform(x_bits: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """bf16 [..., H, D] -> fp32 y = FWHT(x * s) * (1/sqrt(D))."""
    D = x_bits.shape[-1]
    return fwht_f32(bf16_to_f32(x_bits) * signs) * np.float32(1.0 / math.sqrt(D))


def _scale(mn: np.ndarray, mx: np.ndarray, levels: np.ndarray) -> np.ndarray:
    return np.maximum(mx - mn, FLOOR) / (np.asarray(levels, np.float32) - np.float32(1.0))


def _quantize(had: np.ndarray, mn: np.ndarray, sc: np.ndarray, levels: np.ndarray) -> np.ndarray:
    q = round_half_away((had - mn) / sc)
    return np.minimum(np.maximum(q, np.float32(0.0)), np.asarray(levels, np.float32)).astype(np.uint8)


def compress_layer(x_bits: np.ndarray, signs: np.ndarray, k_levels: Sequence[float],
                   v_levels: Sequence[float]) -> Tuple[np.ndarray, Dict[str, np.ndarray]]:
    """One layer [2, R, H, D] (bf16 bits, R = blocks * block_size rows) ->
    (uint8 [2, R, H, D], fp32 metadata {kmin, kscale [H, D], vmin, vscale [R, H]})."""
    kl = np.asarray(k_levels, np.float32)
    vl = np.asarray(v_levels, np.float32)
    y = transform(x_bits, signs)
    had = bf16_to_f32(f32_to_bf16(y))
    # K: channel statistics over all rows
    kmn, kmx = y[0].min(axis=0), y[0].max(axis=0)
    ksc = _scale(kmn, kmx, kl[:, None])
    qk = _quantize(had[0], kmn, ksc, kl[:, None])
    # V: row statistics over D, reduced over the heads of each group
    rmn, rmx = y[1].min(axis=-1), y[1].max(axis=-1)  # [R, H]
    gm = group_map(v_levels)
    gmn, gmx = np.empty_like(rmn), np.empty_like(rmx)
    for g in np.unique(gm):
        heads = gm == g
        gmn[:, heads] = rmn[:, heads].min(axis=1, keepdims=True)
        gmx[:, heads] = rmx[:, heads].max(axis=1, keepdims=True)
    vsc = _scale(gmn, gmx, vl[None, :])
    qv = _quantize(had[1], gmn[..., None], vsc[..., None], vl[None, :, None])
    return np.stack([qk, qv]), {"kmin": kmn, "kscale": ksc, "vmin": gmn, "vscale": vsc}


def _fma_f32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """float32(a * b + c) with a single rounding: the float64 value is exact for a
    byte times a float16 plus a float16."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(np.float32)


def decompress_layer(q: np.ndarray, kmin16: np.ndarray, kscale16: np.ndarray, vmin16: np.ndarray,
                     vscale16: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """uint8 [2, R, H, D] with float16 metadata -> bf16 bits [2, R, H, D]."""
    D = q.shape[-1]
    f = lambda t: np.asarray(t, np.float16).astype(np.float32)
    xk = _fma_f32(q[0], f(kscale16)[None], f(kmin16)[None])
    xv = _fma_f32(q[1], f(vscale16)[..., None], f(vmin16)[..., None])
    y = fwht_f32(np.stack([xk, xv])) * np.float32(1.0 / math.sqrt(D))
    return f32_to_bf16(y * signs)
