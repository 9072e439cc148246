"""Quantization profiles and Rademacher signs for the fused engine.

A profile says, for each layer and part (K, V), which source head is stored at each
output position, its quantization levels (``max_value``) and its V statistic group.
It is the generalisation of KVServeQuantizer's head / layer split
(kvserve_v1/compression/quantizer/kvserve_quantizer.py:42-103, :171-233;
quantizer/split_func.py:9-72): the reference's two sections ``[low, high]`` are two
groups, and a per-(layer, head) level table needs no CSV at all.

Device layout (kvmi_layer_job::profile): uint8 [2 parts][3][H] =
order / levels / group.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, List, Optional, Sequence

import numpy as np

DUO_DIR = Path(__file__).resolve().parent / "compression" / "config" / "duo_config"


# ------------------------------------------------------------------ signs
def rademacher_sign_bits(base_seed: int, layer_id: int, num_heads: int, head_dim: int) -> np.ndarray:
    """uint32 [H, ceil(D/32)]: bit d%32 of word d//32 is set where the sign is -1 (bits
    past D are 0).

    Recipe of HadamardTransform.get_rademacher_signs (hadamard_func.py:33-48,
    :137-152): one CPU torch.Generator re-seeded per head with
    base_seed ^ (layer_id << 16) ^ head, then randint(0, 2, (D,), int8) * 2 - 1.
    """
    import torch

    if head_dim < 1:
        raise ValueError("head_dim must be positive")
    gen = torch.Generator(device="cpu")
    W = (head_dim + 31) // 32
    out = np.zeros((num_heads, W), dtype=np.uint32)
    for h in range(num_heads):
        gen.manual_seed(base_seed ^ (layer_id << 16) ^ h)
        s = torch.randint(0, 2, (head_dim,), generator=gen, dtype=torch.int8).numpy()
        neg = np.zeros(W * 32, np.uint64)
        neg[:head_dim] = s == 0  # 0 -> -1
        words = (neg.reshape(W, 32) << np.arange(32, dtype=np.uint64)).sum(axis=1)
        out[h] = words.astype(np.uint32)
    return out


# ------------------------------------------------------------------ DuoAttention scores
def scores_from_csv(model_name: str) -> np.ndarray:
    """float32 [layers, kv_heads] head-importance scores of a model.

    Search order as DuoConfigGenerator.get_scores_from_csv (duo_config/get_config.py:89-117):
    the package's duo_config directory, then the working directory, then
    $KVSERVE_DUO_CONFIG_DIR.
    """
    base = model_name.strip("/").split("/")[-1]
    name = f"{base}_scores.csv"
    paths = [DUO_DIR / name, Path.cwd() / name]
    env = os.environ.get("KVSERVE_DUO_CONFIG_DIR")
    if env:
        paths.append(Path(env) / name)
    for p in paths:
        if p.exists():
            rows = []
            for line in p.read_text().splitlines():
                line = line.strip()
                if not line:
                    continue
                vals = line.split(",")
                if any(v.strip() == "" for v in vals):
                    continue  # pandas .dropna() drops incomplete rows
                rows.append([float(v) for v in vals])
            return np.asarray(rows, dtype=np.float32)
    raise FileNotFoundError(f"head scores for {base} not found (checked {', '.join(map(str, paths))})")


def head_low_mask(scores: np.ndarray, hybrid_ratio: float) -> np.ndarray:
    """kvserve_quantizer.py:58-63: the round(numel * ratio) lowest-scoring
    (layer, head) pairs are low precision (torch.argsort, ascending)."""
    n_low = int(round(scores.size * hybrid_ratio))
    import torch

    order = torch.argsort(torch.from_numpy(np.ascontiguousarray(scores.reshape(-1))))[:n_low].numpy()
    mask = np.zeros(scores.size, dtype=bool)
    mask[order] = True
    return mask.reshape(scores.shape)


def layer_low_mask(num_rows: int) -> np.ndarray:
    """kvserve_quantizer.py:65-68: the last round(0.33 * rows) layers are low precision."""
    m = np.zeros(num_rows, dtype=bool)
    n = int(round(num_rows * 0.33))
    if n:
        m[-n:] = True
    return m


def tp_head_slice(mask: np.ndarray, num_heads: int, tp_size: int, tp_rank: int) -> np.ndarray:
    """kvserve_quantizer.py:76-103: this worker's KV-head columns of the mask."""
    total = mask.shape[1]
    if total == num_heads:
        return mask
    if total % num_heads:
        raise ValueError(f"Head mask size mismatch: mask_heads={total}, tensor_heads={num_heads}.")
    tp = tp_size or total // num_heads
    if tp * num_heads != total:
        raise ValueError(f"TP mismatch: tp_size={tp}, tensor_heads={num_heads}, total_heads={total}.")
    if tp_rank < 0 or tp_rank >= tp:
        raise ValueError(f"Invalid tp_rank={tp_rank} for tp_size={tp}.")
    return mask[:, tp_rank * num_heads:(tp_rank + 1) * num_heads]


# ------------------------------------------------------------------ profiles
@dataclass
class LayerProfile:
    """Profile of one layer: arrays of length H for K and V."""

    k_order: List[int]
    k_levels: List[int]
    v_order: List[int]
    v_levels: List[int]
    v_group: List[int]
    k_group: Optional[List[int]] = None  # K sections (metadata only: K stats are per channel)
    n_low: Optional[int] = None  # leading output positions forming the reference's "low" section

    def num_v_groups(self) -> int:
        return max(self.v_group) + 1

    def k_groups(self) -> List[int]:
        return self.k_group if self.k_group is not None else self.v_group

    def to_array(self) -> np.ndarray:
        H = len(self.k_order)
        a = np.zeros((2, 3, H), dtype=np.uint8)
        a[0, 0], a[0, 1], a[0, 2] = self.k_order, self.k_levels, self.k_groups()
        a[1, 0], a[1, 1], a[1, 2] = self.v_order, self.v_levels, self.v_group
        return a

    def validate(self, H: int, k_groups: bool = False) -> None:
        """k_groups: K shares statistics over its groups too (token / tensor axis), so
        its groups obey the rules of V's."""
        for name, arr in (("k_order", self.k_order), ("v_order", self.v_order)):
            if sorted(arr) != list(range(H)):
                raise ValueError(f"{name} must be a permutation of range({H})")
        for lv in list(self.k_levels) + list(self.v_levels):
            if not 2 <= int(lv) <= 255:
                raise ValueError("levels (max_value) must be in [2, 255]")
        parts = [("V", list(self.v_group), self.v_levels)]
        if k_groups:
            parts.append(("K", list(self.k_groups()), self.k_levels))
        for name, g, levels in parts:
            if len(g) != H or g[0] != 0 or any(b not in (a, a + 1) for a, b in zip(g, g[1:])):
                raise ValueError(f"{name} groups must be contiguous runs numbered from 0")
            for gi in set(g):
                if len({levels[j] for j in range(H) if g[j] == gi}) != 1:
                    raise ValueError(f"all heads of a {name} group share one level count")


def section_profile(low_mask_row: Sequence[bool], hk: int, hv: int, lk: int, lv: int) -> LayerProfile:
    """Head split (split_func.py:40-72): output order [low heads asc, high heads asc];
    low heads form group 0 and high heads the next group (kvserve_quantizer.py:210-220)."""
    low = [h for h, m in enumerate(low_mask_row) if m]
    high = [h for h, m in enumerate(low_mask_row) if not m]
    order = low + high
    grp = [0] * len(low) + [1 if low else 0] * len(high)
    return LayerProfile(order, [lk] * len(low) + [hk] * len(high), order, [lv] * len(low) + [hv] * len(high), grp,
                        n_low=len(low))


def whole_layer_profile(H: int, k_levels: int, v_levels: int, is_low: bool = False) -> LayerProfile:
    """Layer split (split_func.py:9-38): the layer is one section (low or high)."""
    order = list(range(H))
    return LayerProfile(order, [k_levels] * H, order, [v_levels] * H, [0] * H, n_low=H if is_low else 0)


def per_head_profile(k_levels: Sequence[int], v_levels: Sequence[int]) -> LayerProfile:
    """Per-(layer, head) levels: heads ordered by (V level, head), one V group per
    distinct V level; K heads keep the same order."""
    H = len(v_levels)
    distinct = sorted(set(int(x) for x in v_levels))
    order = sorted(range(H), key=lambda h: (distinct.index(int(v_levels[h])), h))
    grp = [distinct.index(int(v_levels[h])) for h in order]
    return LayerProfile(order, [int(k_levels[h]) for h in order], order, [int(v_levels[h]) for h in order], grp)


def profiles_from_quantizer_config(qc: Dict, num_layers: int, num_heads: int, tp_rank: int = 0,
                                   tp_size: int = 1) -> List[LayerProfile]:
    """Profiles of layers 0..num_layers-1 for a KVServeQuantizer config dict
    (kvserve_quantizer.py:42-68 defaults)."""
    model = qc.get("model_name", "Llama-3.1-8B-Instruct")
    ratio = qc.get("hybrid_ratio", 0.3)
    hk = qc.get("high_key_max_value", 16)
    hv = qc.get("high_value_max_value", 16)
    lk = qc.get("low_key_max_value", 12)
    lv = qc.get("low_value_max_value", 12)
    if qc.get("axis_key", "channel") != "channel" or qc.get("axis_value", "token") != "token":
        raise NotImplementedError("the fused engine quantizes K per channel and V per token")
    split = qc.get("split_type", "head")
    scores = scores_from_csv(model)
    if split == "head":
        mask = tp_head_slice(head_low_mask(scores, ratio), num_heads,
                             qc.get("tensor_parallel_size", tp_size), qc.get("tp_rank", tp_rank))
        if num_layers > mask.shape[0]:
            raise IndexError(f"head scores of {model} cover {mask.shape[0]} layers, got {num_layers}")
        return [section_profile(mask[l], hk, hv, lk, lv) for l in range(num_layers)]
    if split == "layer":
        lm = layer_low_mask(scores.shape[0])
        if num_layers > lm.shape[0]:
            raise IndexError(f"layer mask of {model} covers {lm.shape[0]} layers, got {num_layers}")
        return [whole_layer_profile(num_heads, lk if lm[l] else hk, lv if lm[l] else hv, bool(lm[l]))
                for l in range(num_layers)]
    raise ValueError(f"split_type must be 'head' or 'layer', got {split}")
