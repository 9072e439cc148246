"""Shared loaders for the fixed-profile runtime's golden cases (tests/golden/runtime.npz).

Each case holds the reference CPU runtime's inputs and outputs for one chunk: the
source blocks, the payload / aux / raw tail of both KV parts, the restored target
blocks, the head orders, signs and layout offsets.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Dict, List

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden" / "runtime.npz"
MINUS_NINE = 0xC110  # bf16 bits of -9.0


def load_cases() -> Dict[str, dict]:
    data = np.load(GOLDEN)
    cases: Dict[str, dict] = {}
    for key in data.files:
        if key.endswith("_meta"):
            name = key[:-5]
            meta = json.loads(bytes(data[key]).decode())
            case = {"name": name, "meta": meta}
            for k in data.files:
                if k.startswith(name + "_") and k != key:
                    case[k[len(name) + 1:]] = data[k]
            cases[name] = case
    return cases


def physical(meta: dict, logical: List[int]) -> List[int]:
    f = meta["blocks_per_logical"]
    return [b * f + i for b in logical for i in range(f)]


def full_caches(case: dict, fill_source: bool, seed: int = 0) -> List[np.ndarray]:
    """bf16 bits [total_blocks, heads, kernel_tokens, Dk + Dv] per layer: the golden
    source blocks at their physical ids and random blocks elsewhere (fill_source),
    or -9 everywhere (a consumer's cache)."""
    meta = case["meta"]
    rng = np.random.default_rng(seed)
    out = []
    for i in range(meta["layers"]):
        src = case[f"src{i}"]
        shape = (meta["total_blocks"], *src.shape[1:])
        if fill_source:
            cache = (rng.standard_normal(shape, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)
            cache[physical(meta, meta["src"])] = src
        else:
            cache = np.full(shape, MINUS_NINE, dtype=np.uint16)
        out.append(cache)
    return out


def extra_config(meta: dict) -> dict:
    return {"compression": {"enable-compression-pipeline": True, "logical_blocks_per_chunk": len(meta["src"]),
                            **meta["compression"]}}
