"""Synthetic paged-KV workloads of the benchmark configurations.

Every generator is seeded (torch.Generator) and returns the per-layer KV caches in
vLLM's FlashAttention NHD layout [2, P, S, H, D] (bf16), the block table of the
request(s) and the per-layer quantization profiles.  Data are synthetic: there is no
network for real model activations.

  1  1 layer x 8 heads x D=128 x 512 tokens, K/V ~ N(0,1), 4 outlier K channels per
     head x10, identity table; head split with the Llama-3.1-8B row-0 mask at
     hybrid 0.3, 16/16 levels, 4 bits.
  2  Llama-3-8B: 32 layers x 8192 tokens, same data law, first 512 ids of a seeded
     randperm(65536) for every layer; 16/16 levels, 4 bits, 4 chunks of 8 layers.
  3  16 requests, lengths U[1024, 16384], per-(layer, head) levels {6, 12} for K
     and V independently, 262144-block pool (aliased, see make_config3).
  4  Qwen2.5-72B: 80 layers x 32768 tokens, N(0,1) with 2% Student-t(3) outliers;
     layer split, levels 12/6/12/6..., 4 bits.
  5  256 requests x 256 tokens, 16 layers, D=64, 6/6 levels, 3 bits.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from .profiles import LayerProfile, per_head_profile, scores_from_csv, head_low_mask, section_profile, \
    whole_layer_profile

SEED_HADAMARD = 0xC0FEBABE  # configs/compression/original_top_nvcomp.json:6


@dataclass
class Request:
    pools: List[torch.Tensor]       # per layer [2, P, S, H, D] bf16 (may alias between requests)
    block_ids: torch.Tensor         # int32 [B] on the pools' device
    profiles: List[LayerProfile]
    layer_ids: List[int]


@dataclass
class Workload:
    name: str
    requests: List[Request]
    num_heads: int
    head_dim: int
    block_size: int
    bits: int
    seed: int

    def raw_bytes(self) -> int:
        tot = 0
        for r in self.requests:
            tot += len(r.pools) * 2 * r.block_ids.numel() * self.block_size * self.num_heads * self.head_dim * 2
        return tot


def kv_blocks(gen: torch.Generator, B: int, S: int, H: int, D: int, k_outliers: int = 4,
              t_outlier_frac: float = 0.0, device="cpu") -> torch.Tensor:
    """[2, B, S, H, D] bf16 with K, V ~ N(0, 1); `k_outliers` seeded K channels per head
    scaled x10; optionally a fraction of elements replaced by Student-t(3) draws."""
    x = torch.randn((2, B, S, H, D), generator=gen, device=device, dtype=torch.float32)
    if k_outliers:
        ch = torch.stack([torch.randperm(D, generator=gen, device=device)[:k_outliers] for _ in range(H)])
        scale = torch.ones((H, D), device=device)
        scale.scatter_(1, ch, 10.0)
        x[0] *= scale
    if t_outlier_frac > 0:
        m = torch.rand(x.shape, generator=gen, device=device) < t_outlier_frac
        # Student-t(3) = N / sqrt(chi2_3 / 3)
        z = torch.randn(x.shape, generator=gen, device=device)
        c = torch.randn((3,) + tuple(x.shape), generator=gen, device=device).square().sum(0) / 3
        x = torch.where(m, z / c.sqrt(), x)
    return x.to(torch.bfloat16)


def llama_row_profiles(num_layers: int, H: int, levels=(16, 16, 16, 16), ratio: float = 0.3) -> List[LayerProfile]:
    """Head split with the Llama-3.1-8B-Instruct DuoAttention mask (layer l uses row
    l % 32); levels = (high K, high V, low K, low V)."""
    mask = head_low_mask(scores_from_csv("Llama-3.1-8B-Instruct"), ratio)
    hk, hv, lk, lv = levels
    # more heads than the CSV's 8 (the wide-head benchmark variants): the row repeats
    return [section_profile(np.resize(mask[l % mask.shape[0]], H) if H > mask.shape[1] else mask[l % mask.shape[0]][:H],
                            hk, hv, lk, lv) for l in range(num_layers)]


def make_config1(device="cuda", seed: int = 1) -> Workload:
    gen = torch.Generator(device="cpu").manual_seed(seed)
    L, B, S, H, D = 1, 32, 16, 8, 128
    x = kv_blocks(gen, B, S, H, D)
    pool = x.to(device).contiguous()  # identity table: pool == request blocks
    ids = torch.arange(B, dtype=torch.int32, device=device)
    req = Request([pool], ids, llama_row_profiles(L, H), list(range(L)))
    return Workload("config1", [req], H, D, S, 4, SEED_HADAMARD)


def make_config2(device="cuda", seed: int = 2, num_layers: int = 32, pool_blocks: Optional[int] = None,
                 fill: str = "zeros", num_heads: int = 8, head_dim: int = 128) -> Workload:
    """Llama-3-8B-shaped request: 32 layers x 8192 tokens in a 65536-block pool per layer
    (4 GiB per layer, 128 GiB total).  Only the request's blocks hold data; the rest
    of each pool is `fill` ("zeros" or "empty").  `num_heads` / `head_dim` other than
    8 / 128 give the same request with wider rows (the pool keeps 4 GiB per layer)."""
    L, S, H, D, B = num_layers, 16, num_heads, head_dim, 512
    if pool_blocks is None:
        pool_blocks = 65536 * 8 * 128 // (H * D)
    gen = torch.Generator(device=device).manual_seed(seed)
    perm = torch.randperm(pool_blocks, generator=torch.Generator(device="cpu").manual_seed(seed))
    ids = perm[:B].to(torch.int32).to(device)
    pools = []
    for _ in range(L):
        p = (torch.zeros if fill == "zeros" else torch.empty)((2, pool_blocks, S, H, D), dtype=torch.bfloat16,
                                                              device=device)
        p[:, ids.long()] = kv_blocks(gen, B, S, H, D, device=device)
        pools.append(p)
    req = Request(pools, ids, llama_row_profiles(L, H), list(range(L)))
    return Workload("config2", [req], H, D, S, 4, SEED_HADAMARD)


def make_config5(device="cuda", seed: int = 5, num_requests: int = 256, pool_blocks: int = 8192) -> Workload:
    """256 requests x 256 tokens (16 blocks), 16 layers, H=8, D=64, 6/6 levels, 3 bits.
    All requests share the per-layer pools (disjoint seeded random blocks)."""
    L, S, H, D, B = 16, 16, 8, 64, 16
    gen = torch.Generator(device=device).manual_seed(seed)
    perm = torch.randperm(pool_blocks, generator=torch.Generator(device="cpu").manual_seed(seed))
    assert num_requests * B <= pool_blocks
    pools = [torch.zeros((2, pool_blocks, S, H, D), dtype=torch.bfloat16, device=device) for _ in range(L)]
    for p in pools:
        used = perm[: num_requests * B].to(device)
        p[:, used] = kv_blocks(gen, num_requests * B, S, H, D, k_outliers=0, device=device)
    prof = [whole_layer_profile(H, 6, 6) for _ in range(L)]
    reqs = [Request(pools, perm[r * B:(r + 1) * B].to(torch.int32).to(device), prof, list(range(L)))
            for r in range(num_requests)]
    return Workload("config5", reqs, H, D, S, 3, SEED_HADAMARD)


def make_config4(device="cuda", seed: int = 4, num_layers: int = 80, tokens: int = 32768) -> Workload:
    """Qwen2.5-72B-shaped long context: contiguous per-layer caches holding exactly the
    request (identity table), layer split with levels 12, 6, 12, 6, ..."""
    L, S, H, D = num_layers, 16, 8, 128
    B = tokens // S
    gen = torch.Generator(device=device).manual_seed(seed)
    pools = [kv_blocks(gen, B, S, H, D, k_outliers=0, t_outlier_frac=0.02, device=device) for _ in range(L)]
    ids = torch.arange(B, dtype=torch.int32, device=device)
    prof = [whole_layer_profile(H, 12 if l % 2 == 0 else 6, 12 if l % 2 == 0 else 6) for l in range(L)]
    return Workload("config4", [Request(pools, ids, prof, list(range(L)))], H, D, S, 4, SEED_HADAMARD)


def make_config3(device="cuda", seed: int = 3, num_requests: int = 16, num_layers: int = 32,
                 pool_blocks: int = 262144, physical_pools: int = 2) -> Workload:
    """16 variable-length requests with per-(layer, head) levels in {6, 12}.  A
    262144-block pool per layer would need 512 GiB for 32 layers, more than HBM, so the
    32 logical layer pools alias `physical_pools` physical pools (layer l uses pool
    l % physical_pools); every request's blocks are disjoint within a pool."""
    L, S, H, D = num_layers, 16, 8, 128
    g = torch.Generator(device="cpu").manual_seed(seed)
    lens = torch.randint(1024, 16385, (num_requests,), generator=g)
    blocks = [int((t + S - 1) // S) for t in lens]
    perm = torch.randperm(pool_blocks, generator=g)
    gen = torch.Generator(device=device).manual_seed(seed)
    phys = [torch.zeros((2, pool_blocks, S, H, D), dtype=torch.bfloat16, device=device)
            for _ in range(physical_pools)]
    total = sum(blocks)
    used = perm[:total].to(device)
    for p in phys:
        for c0 in range(0, total, 4096):
            sel = used[c0:c0 + 4096]
            p[:, sel] = kv_blocks(gen, sel.numel(), S, H, D, device=device)
    reqs, off = [], 0
    for r in range(num_requests):
        ids = perm[off:off + blocks[r]].to(torch.int32).to(device)
        off += blocks[r]
        kl = torch.randint(0, 2, (L, H), generator=g) * 6 + 6
        vl = torch.randint(0, 2, (L, H), generator=g) * 6 + 6
        prof = [per_head_profile(kl[l].tolist(), vl[l].tolist()) for l in range(L)]
        reqs.append(Request([phys[l % physical_pools] for l in range(L)], ids, prof, list(range(L))))
    return Workload("config3", reqs, H, D, S, 4, SEED_HADAMARD)
