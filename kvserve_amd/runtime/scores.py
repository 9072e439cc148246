"""Head selection of the fixed-profile runtime: which KV heads of each bound layer take
the low-precision levels (kvserve_v1/compression/runtime/scores.py:16-112).

The rule, which peers must reproduce exactly because it fixes the head order on the
wire:

* ``split_type = "layer"``: no head is low here (the layer split is applied by the
  layout) and every layer keeps its natural head order.
* ``split_type = "head"``: the score table has one row per model layer and one column
  per KV head of the whole model (or of this rank).  The candidates are the full rows of
  the bound layers, taken in binding order; the ``round(candidates * hybrid_ratio)``
  lowest scores (ties broken by candidate order) are low.  Each rank then looks at its
  own window of a row -- the whole row, its tensor-parallel slice, or the one column it
  shares with other ranks when KV heads are replicated -- and orders its heads
  [low ascending, high ascending].
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Callable, Dict, Optional, Tuple

import numpy as np
import torch

from .config import CompressionConfig
from .spec import CacheSpec


@dataclass(frozen=True)
class HeadSelection:
    low_counts: Dict[int, int]
    local_orders: Dict[int, Tuple[int, ...]]


def _scores_from_torch(path: Path) -> np.ndarray:
    obj = torch.load(path, map_location="cpu", weights_only=True)  # tensors only, nothing executed
    if isinstance(obj, dict):
        obj = obj.get("scores", obj.get("head_scores"))
    return obj.float().numpy()


def _scores_from_text(path: Path) -> np.ndarray:
    table = np.genfromtxt(path, delimiter=",", dtype=np.float32)
    if table.ndim == 2:  # drop rows and columns that hold no number (headers, trailing commas)
        table = table[~np.isnan(table).all(axis=1)]
        table = table[:, ~np.isnan(table).all(axis=0)]
    return table


_LOADERS: Dict[str, Callable[[Path], np.ndarray]] = {
    ".npy": lambda p: np.load(p, allow_pickle=False),
    ".pt": _scores_from_torch,
    ".pth": _scores_from_torch,
    ".json": lambda p: np.asarray(json.loads(p.read_text()), dtype=np.float32),
}


def load_scores(path: str) -> np.ndarray:
    """A score table from .npy (no pickles), .pt / .pth (weights only; a tensor or a dict
    with "scores" / "head_scores"), .json, or comma-separated text (any other suffix)."""
    p = Path(path)
    return np.asarray(_LOADERS.get(p.suffix.lower(), _scores_from_text)(p), dtype=np.float32)


def _window_start(width: int, local: int, tp_rank: int, tp_size: int) -> int:
    """First score column of this rank's heads in a row of `width` columns."""
    if width == local:                        # the table already holds this rank's heads
        return 0
    if width == local * tp_size:              # the model's heads, sliced by rank
        return tp_rank * local
    replicas = tp_size // width if 0 < width < tp_size else 0
    if local == 1 and replicas and width * replicas == tp_size:
        return tp_rank // replicas            # one KV head shared by `replicas` ranks
    raise ValueError(f"Head score width {width} is incompatible with {local} local KV heads and "
                     f"TP size {tp_size}.")


def _low_mask(scores: np.ndarray, rows: list, ratio: float) -> np.ndarray:
    """Boolean table shaped like `scores`: True where a candidate is among the lowest."""
    mask = np.zeros(scores.shape, dtype=bool)
    cand = scores[rows]                        # candidate rows in binding order (repeats allowed)
    n_low = round(cand.size * ratio)
    if n_low:
        flat = np.argsort(cand.reshape(-1), kind="stable")[:n_low]
        r, c = np.divmod(flat, scores.shape[1])
        mask[np.asarray(rows)[r], c] = True
    return mask


def build_head_selection(specs: Dict[str, CacheSpec], config: CompressionConfig, tp_rank: int, tp_size: int,
                         scores: Optional[np.ndarray] = None) -> HeadSelection:
    bound = list(specs.values())
    if config.split_type == "layer":
        return HeadSelection(low_counts={s.layer_index: 0 for s in bound},
                             local_orders={s.layer_index: tuple(range(s.num_kv_heads)) for s in bound})
    if scores is None:
        if not config.score_path:
            raise ValueError("Head split requires a score_path or head scores.")
        scores = load_scores(config.score_path)
    if scores.ndim != 2 or not np.isfinite(scores).all():
        raise ValueError("Head scores must be a finite 2D array of layers and KV heads.")
    missing = next((s.layer_index for s in bound if not 0 <= s.layer_index < scores.shape[0]), None)
    if missing is not None:
        raise ValueError(f"Head scores have no row for layer {missing}.")
    mask = _low_mask(scores, [s.layer_index for s in bound], config.hybrid_ratio)
    low_counts, orders = {}, {}
    for s in bound:
        start = _window_start(scores.shape[1], s.num_kv_heads, tp_rank, tp_size)
        is_low = mask[s.layer_index, start:start + s.num_kv_heads]
        heads = np.arange(s.num_kv_heads)
        low_counts[s.layer_index] = int(is_low.sum())
        orders[s.layer_index] = tuple(int(h) for h in np.concatenate([heads[is_low], heads[~is_low]]))
    return HeadSelection(low_counts=low_counts, local_orders=orders)
