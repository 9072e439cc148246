"""Head selection of the fixed-profile runtime (kvserve_v1/compression/runtime/scores.py:16-112).

The low-precision heads are the lowest ``round(candidates * hybrid_ratio)`` scores
over all (layer, head) pairs of the bound layers (stable order); each layer's heads
are reordered [low ascending, high ascending].  Score tables wider than the local
heads are sliced by tensor-parallel rank, and a score column is shared by replicated
KV heads.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from .config import CompressionConfig
from .spec import CacheSpec


@dataclass(frozen=True)
class HeadSelection:
    low_counts: Dict[int, int]
    local_orders: Dict[int, Tuple[int, ...]]


def load_scores(path: str) -> np.ndarray:
    """.npy (no pickles), .pt / .pth (weights only), .json, or CSV."""
    p = Path(path)
    suffix = p.suffix.lower()
    if suffix == ".npy":
        values = np.load(p, allow_pickle=False)
    elif suffix in (".pt", ".pth"):
        loaded = torch.load(p, map_location="cpu", weights_only=True)
        if isinstance(loaded, dict):
            loaded = loaded.get("scores", loaded.get("head_scores"))
        values = loaded.float().numpy()
    elif suffix == ".json":
        values = np.asarray(json.loads(p.read_text()), dtype=np.float32)
    else:
        values = np.genfromtxt(p, delimiter=",", dtype=np.float32)
        if values.ndim == 2:
            values = values[~np.all(np.isnan(values), axis=1)]
            values = values[:, ~np.all(np.isnan(values), axis=0)]
    return np.asarray(values, dtype=np.float32)


def build_head_selection(specs: Dict[str, CacheSpec], config: CompressionConfig, tp_rank: int, tp_size: int,
                         scores: Optional[np.ndarray] = None) -> HeadSelection:
    items = list(specs.items())
    if config.split_type == "layer":
        return HeadSelection(low_counts={s.layer_index: 0 for _, s in items},
                             local_orders={s.layer_index: tuple(range(s.num_kv_heads)) for _, s in items})
    if scores is None:
        if not config.score_path:
            raise ValueError("Head split requires a score_path or head scores.")
        scores = load_scores(config.score_path)
    if scores.ndim != 2 or not np.isfinite(scores).all():
        raise ValueError("Head scores must be a finite 2D array of layers and KV heads.")
    rows, width = scores.shape
    candidates = []
    for _, spec in items:
        li = spec.layer_index
        if not 0 <= li < rows:
            raise ValueError(f"Head scores have no row for layer {li}.")
        candidates.extend(range(li * width, (li + 1) * width))
    cand = np.asarray(candidates, dtype=np.int64)
    mask = np.zeros(scores.size, dtype=bool)
    n_low = round(cand.size * config.hybrid_ratio)
    if n_low:
        picked = np.argsort(scores.reshape(-1)[cand], kind="stable")[:n_low]
        mask[cand[picked]] = True
    mask = mask.reshape(scores.shape)
    low_counts, orders = {}, {}
    for _, spec in items:
        li, local = spec.layer_index, spec.num_kv_heads
        if width == local:
            start = 0
        elif width == local * tp_size:
            start = tp_rank * local
        elif local == 1 and 0 < width < tp_size and tp_size % width == 0:
            start = tp_rank // (tp_size // width)
        else:
            raise ValueError(f"Head score width {width} is incompatible with {local} local KV heads and "
                             f"TP size {tp_size}.")
        row = mask[li, start:start + local]
        low, high = np.flatnonzero(row).tolist(), np.flatnonzero(~row).tolist()
        low_counts[li] = len(low)
        orders[li] = tuple(low + high)
    return HeadSelection(low_counts=low_counts, local_orders=orders)
