"""Conversion between the engine's flat metadata tables and the reference's
per-layer quantization dicts.

Engine tables (kvserve_amd.engine.Packet):
  kmeta bf16 [L, 2, H, D]   [l, 0] = per-channel min, [l, 1] = scale, by output position
  vmeta bf16 [L, 2, G, B*S] [l, 0] = per-token min, [l, 1] = scale, by V group
Reference dict of one layer (kvserve_quantizer.py:224-231, quantizer_func.py:67-73):
  {"high_key_meta", "high_value_meta", "low_key_meta", "low_value_meta": {
       "min_val": bf16 [1,1,Hg,D] (K) or [B,S,1,1] (V) | None, "quant_scale": same,
       "original_dtype": "bfloat16", "quant_dtype": "uint8"},
   "original_dtype": "bfloat16"}
The "low" section is the first n_low output positions and V group 0 when it exists.
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import torch

from ..profiles import LayerProfile

_SECTIONS = ("high_key_meta", "high_value_meta", "low_key_meta", "low_value_meta")


def _empty(dtype: str = "bfloat16") -> Dict:
    return {"min_val": None, "quant_scale": None, "original_dtype": dtype, "quant_dtype": "uint8"}


def _sec(mn: torch.Tensor, sc: torch.Tensor) -> Dict:
    return {"min_val": mn, "quant_scale": sc, "original_dtype": "bfloat16", "quant_dtype": "uint8"}


def layer_dict(kmeta_l: torch.Tensor, vmeta_l: torch.Tensor, prof: LayerProfile, B: int, S: int) -> Dict:
    """Reference-format metadata of one layer (views into the engine tables)."""
    H, D = kmeta_l.shape[1], kmeta_l.shape[2]
    n_low = prof.n_low if prof.n_low is not None else 0
    if prof.num_v_groups() > (2 if 0 < n_low < H else 1) or prof.k_order != prof.v_order:
        raise ValueError("this profile has no reference-format metadata (more than two sections)")
    out = {k: _empty() for k in _SECTIONS}
    out["original_dtype"] = "bfloat16"
    if n_low > 0:
        out["low_key_meta"] = _sec(kmeta_l[0, :n_low].view(1, 1, n_low, D), kmeta_l[1, :n_low].view(1, 1, n_low, D))
        out["low_value_meta"] = _sec(vmeta_l[0, 0].view(B, S, 1, 1), vmeta_l[1, 0].view(B, S, 1, 1))
    if n_low < H:
        nh = H - n_low
        g = 1 if n_low > 0 else 0
        out["high_key_meta"] = _sec(kmeta_l[0, n_low:].view(1, 1, nh, D), kmeta_l[1, n_low:].view(1, 1, nh, D))
        out["high_value_meta"] = _sec(vmeta_l[0, g].view(B, S, 1, 1), vmeta_l[1, g].view(B, S, 1, 1))
    return out


def tables_from_dicts(dicts: Sequence[Dict], H: int, D: int, B: int, S: int,
                      device) -> Tuple[torch.Tensor, torch.Tensor]:
    """Inverse of layer_dict for a list of layers: (kmeta [L,2,H,D], vmeta [L,2,G,B*S])."""
    L = len(dicts)
    G = 1
    for d in dicts:
        n = sum(1 for s in ("low_value_meta", "high_value_meta") if d[s]["min_val"] is not None)
        G = max(G, n)
    views = _table_views(dicts, H, D, B * S, G, device)
    if views is not None:
        return views
    kmeta = torch.empty((L, 2, H, D), dtype=torch.bfloat16, device=device)
    vmeta = torch.zeros((L, 2, G, B * S), dtype=torch.bfloat16, device=device)
    for l, d in enumerate(dicts):
        parts_k = [d[s] for s in ("low_key_meta", "high_key_meta") if d[s]["min_val"] is not None]
        parts_v = [d[s] for s in ("low_value_meta", "high_value_meta") if d[s]["min_val"] is not None]
        if not parts_k or not parts_v:
            raise ValueError("Missing quantization params")
        kmeta[l, 0] = torch.cat([p["min_val"].reshape(-1, D) for p in parts_k]).to(device, torch.bfloat16)
        kmeta[l, 1] = torch.cat([p["quant_scale"].reshape(-1, D) for p in parts_k]).to(device, torch.bfloat16)
        for g, p in enumerate(parts_v):
            vmeta[l, 0, g] = p["min_val"].reshape(-1).to(device, torch.bfloat16)
            vmeta[l, 1, g] = p["quant_scale"].reshape(-1).to(device, torch.bfloat16)
    return kmeta, vmeta


def _table_views(dicts: Sequence[Dict], H: int, D: int, BS: int, G: int,
                 device) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """kmeta / vmeta as views when every section tensor already sits where the
    engine's one-allocation layout puts it (kmeta [L,2,H,D] followed by vmeta
    [L,2,G,B*S], bf16) -- the case of a packet made by this engine, also after a
    wire round trip that shipped the allocation whole.  Pointer arithmetic only;
    None when any tensor is elsewhere (the caller then copies)."""
    L = len(dicts)
    if L == 0:
        return None
    first = dicts[0]["low_key_meta"]["min_val"]
    if first is None:
        first = dicts[0]["high_key_meta"]["min_val"]
    if first is None or first.dtype != torch.bfloat16 or first.device != torch.device(device):
        return None
    st = first.untyped_storage()
    sp, base = st.data_ptr(), first.data_ptr()
    kn, vn = L * 2 * H * D, L * 2 * G * BS
    if (base - sp) % 2 or base - sp + 2 * (kn + vn) > st.nbytes():
        return None
    vbase = base + 2 * kn

    def at(t, addr, numel) -> bool:
        return (t is not None and t.dtype == torch.bfloat16 and t.is_contiguous() and t.numel() == numel
                and t.data_ptr() == addr and t.untyped_storage().data_ptr() == sp)

    for l, d in enumerate(dicts):
        h = 0
        for s in ("low_key_meta", "high_key_meta"):
            mn = d[s]["min_val"]
            if mn is None:
                continue
            rows = mn.numel() // D
            if not (at(mn, base + 2 * ((2 * l) * H + h) * D, rows * D)
                    and at(d[s]["quant_scale"], base + 2 * ((2 * l + 1) * H + h) * D, rows * D)):
                return None
            h += rows
        if h != H:
            return None
        g = 0
        for s in ("low_value_meta", "high_value_meta"):
            mn = d[s]["min_val"]
            if mn is None:
                continue
            if not (at(mn, vbase + 2 * ((2 * l) * G + g) * BS, BS)
                    and at(d[s]["quant_scale"], vbase + 2 * ((2 * l + 1) * G + g) * BS, BS)):
                return None
            g += 1
    off = (base - sp) // 2
    kmeta = torch.empty(0, dtype=torch.bfloat16, device=device).set_(st, off, (L, 2, H, D))
    vmeta = torch.empty(0, dtype=torch.bfloat16, device=device).set_(st, off + kn, (L, 2, G, BS))
    return kmeta, vmeta
