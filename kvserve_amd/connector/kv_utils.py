"""Block-level KV extract / inject for the connector (kvserve_v1/utils/kv_utils.py:6-119).

FlashAttention caches ``[2, num_blocks, ...]`` and MLA / FlashInfer caches
``[num_blocks, 2, ...]`` that are contiguous 16-bit CUDA tensors go through the HIP
gather / scatter kernels (kvmi_gather_blocks / kvmi_gather_blocks_kv_adjacent and
the scatters); anything else is copied with device-side tensor indexing.  Only the
FlashAttention NHD layout takes the fused compression path (the reference requests
NHD, compressed_kv_connector.py:217-230).
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

from .. import ops


def make_slot_mapping(token_ids: Sequence[int], block_ids: Sequence[int], block_size: int) -> torch.Tensor:
    """Absolute slots block_ids[t // block_size] * block_size + t % block_size of the
    first len(token_ids) tokens, as a CPU int64 tensor (kv_utils.py:6-17)."""
    ids = torch.as_tensor(list(block_ids), dtype=torch.long)
    slots = (ids[:, None] * block_size + torch.arange(block_size, dtype=torch.long)[None, :]).reshape(-1)
    return slots[: len(token_ids)]


def is_flash_layout(kv_layer: torch.Tensor) -> bool:
    """[2, num_blocks, S, H, D] 16-bit contiguous CUDA cache: the layout the HIP
    kernels read and write."""
    return (kv_layer.dim() == 5 and kv_layer.shape[0] == 2 and kv_layer.element_size() == 2
            and kv_layer.is_contiguous() and kv_layer.is_cuda)


def _hip_copyable(kv_layer: torch.Tensor) -> bool:
    """A contiguous 16-bit CUDA cache whose blocks are whole 16-byte vectors."""
    return (kv_layer.dim() >= 3 and kv_layer.element_size() == 2 and kv_layer.is_contiguous() and kv_layer.is_cuda
            and (kv_layer[0, 0].numel() * 2) % 16 == 0)


def extract_kv_from_layer_by_blocks(kv_layer: torch.Tensor, block_ids: Sequence[int],
                                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """kv[:, block_ids] (FlashAttention) or kv[block_ids] (MLA) as a new tensor, or
    written into `out` (kv_utils.py:59-80)."""
    if kv_layer.shape[0] == 2:
        if len(block_ids) == 0:
            res = kv_layer[:, :0].clone()
        elif is_flash_layout(kv_layer):
            return ops.gather_blocks(kv_layer, block_ids, out=out)
        else:
            idx = torch.tensor(list(block_ids), dtype=torch.long, device=kv_layer.device)
            res = kv_layer[:, idx]
    elif kv_layer.dim() > 1 and kv_layer.shape[1] == 2:
        if len(block_ids) == 0:
            res = kv_layer[:0].clone()
        elif _hip_copyable(kv_layer):
            return ops.gather_blocks(kv_layer, block_ids, out=out)
        else:
            idx = torch.tensor(list(block_ids), dtype=torch.long, device=kv_layer.device)
            res = kv_layer[idx]
    else:
        raise RuntimeError(f"Unsupported KV layout shape: {tuple(kv_layer.shape)}")
    if out is None:
        return res  # advanced indexing (and the clone of the empty slice) made a copy
    out.copy_(res)
    return out


def inject_kv_into_layer_by_blocks(kv_cache_layer: torch.Tensor, kv_data: torch.Tensor, block_ids: Sequence[int],
                                   request_id: str = "") -> None:
    """Write a request's blocks back into a paged cache; with more ids than payload
    blocks only the first ones are written (kv_utils.py:83-119)."""
    if len(block_ids) == 0:
        return
    if kv_cache_layer.shape[0] == 2:
        if is_flash_layout(kv_cache_layer):
            ops.scatter_blocks(kv_cache_layer, kv_data, block_ids)
            return
        payload = kv_data.to(kv_cache_layer.device)
        idx = torch.tensor(list(block_ids), dtype=torch.long, device=kv_cache_layer.device)
        kv_cache_layer[:, idx[: payload.shape[1]]] = payload
        return
    if kv_cache_layer.dim() > 1 and kv_cache_layer.shape[1] == 2:
        if _hip_copyable(kv_cache_layer):
            ops.scatter_blocks(kv_cache_layer, kv_data, block_ids)
            return
        payload = kv_data.to(kv_cache_layer.device)
        idx = torch.tensor(list(block_ids), dtype=torch.long, device=kv_cache_layer.device)
        kv_cache_layer[idx[: payload.shape[0]]] = payload
        return
    raise RuntimeError(f"Unsupported KV layout for request {request_id}: {tuple(kv_cache_layer.shape)}")
