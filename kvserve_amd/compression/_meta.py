"""Conversion between the engine's flat metadata tables and the reference's
per-layer quantization dicts.

Engine tables (kvserve_amd.engine.Packet), one per part, laid out by the part's axis:
  channel  bf16 [L, 2, H, D]    [l, 0] = per-channel min, [l, 1] = scale, by output position
  token    bf16 [L, 2, G, B*S]  per-token min / scale, by statistic group
  tensor   bf16 [L, 2, G, 1]    one min / scale per group
(K is on the channel axis and V on the token axis by default.)
Reference dict of one layer (kvserve_quantizer.py:224-231, quantizer_func.py:67-73):
  {"high_key_meta", "high_value_meta", "low_key_meta", "low_value_meta": {
       "min_val": bf16 keepdim tensor -- [1,1,Hg,D] (channel), [B,S,1,1] (token),
                  [1,1,1,1] (tensor) -- or None, "quant_scale": same,
       "original_dtype": "bfloat16", "quant_dtype": "uint8"},
   "original_dtype": "bfloat16"}
The "low" section is the first n_low output positions and group 0 when it exists.
"""

from __future__ import annotations

from collections.abc import Sequence as _SequenceABC
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import torch

from ..engine import DEFAULT_AXES, meta_shape
from ..profiles import LayerProfile

_SECTIONS = ("high_key_meta", "high_value_meta", "low_key_meta", "low_value_meta")
_PARTS = (("low_key_meta", "high_key_meta"), ("low_value_meta", "high_value_meta"))


def _empty(dtype: str = "bfloat16") -> Dict:
    return {"min_val": None, "quant_scale": None, "original_dtype": dtype, "quant_dtype": "uint8"}


def _sec(mn: torch.Tensor, sc: torch.Tensor) -> Dict:
    return {"min_val": mn, "quant_scale": sc, "original_dtype": "bfloat16", "quant_dtype": "uint8"}


def _keepdim(axis: str, rows: int, D: int, B: int, S: int) -> Tuple[int, ...]:
    """Reference shape of a section's min / scale (quantizer_func.py:52-53, keepdim)."""
    return {"channel": (1, 1, rows, D), "token": (B, S, 1, 1), "tensor": (1, 1, 1, 1)}[axis]


def _sections(prof: LayerProfile, H: int) -> List[Tuple[str, int, int, int]]:
    """(name, first position, last position + 1, group) of the layer's sections."""
    n_low = prof.n_low if prof.n_low is not None else 0
    out = []
    if n_low > 0:
        out.append(("low", 0, n_low, 0))
    if n_low < H:
        out.append(("high", n_low, H, 1 if n_low > 0 else 0))
    return out


def layer_dict(kmeta_l: torch.Tensor, vmeta_l: torch.Tensor, prof: LayerProfile, B: int, S: int,
               axes: Tuple[str, str] = DEFAULT_AXES) -> Dict:
    """Reference-format metadata of one layer (views into the engine tables; a
    table of one layer is [2, rows, cols] as laid out by its part's axis)."""
    H = len(prof.k_order)
    D = kmeta_l.shape[2] if axes[0] == "channel" else vmeta_l.shape[2] if axes[1] == "channel" else None
    n_low = prof.n_low if prof.n_low is not None else 0
    if prof.num_v_groups() > (2 if 0 < n_low < H else 1) or prof.k_order != prof.v_order:
        raise ValueError("this profile has no reference-format metadata (more than two sections)")
    out = {k: _empty() for k in _SECTIONS}
    out["original_dtype"] = "bfloat16"
    for (low_name, high_name), table, axis in zip(_PARTS, (kmeta_l, vmeta_l), axes):
        for sec, lo, hi, g in _sections(prof, H):
            name = low_name if sec == "low" else high_name
            shape = _keepdim(axis, hi - lo, D, B, S)
            rows = slice(lo, hi) if axis == "channel" else g
            out[name] = _sec(table[0, rows].reshape(shape), table[1, rows].reshape(shape))
    return out


def tables_from_dicts(dicts: Sequence[Dict], H: int, D: int, B: int, S: int, device,
                      axes: Tuple[str, str] = DEFAULT_AXES) -> Tuple[torch.Tensor, torch.Tensor]:
    """Inverse of layer_dict for a list of layers: (kmeta, vmeta), each
    [L, 2, rows, cols] as laid out by its part's axis."""
    L = len(dicts)
    G = 1
    for d in dicts:
        for names in _PARTS:
            G = max(G, sum(1 for s in names if d[s]["min_val"] is not None))
    views = _table_views(dicts, H, D, B * S, G, axes, device)
    if views is not None:
        return views
    tables = []
    for names, axis in zip(_PARTS, axes):
        rows, cols = meta_shape(axis, H, D, G, B * S)
        t = torch.zeros((L, 2, rows, cols), dtype=torch.bfloat16, device=device)
        for l, d in enumerate(dicts):
            secs = [d[s] for s in names if d[s]["min_val"] is not None]
            if not secs:
                raise ValueError("Missing quantization params")
            for which, key in ((0, "min_val"), (1, "quant_scale")):
                if axis == "channel":
                    t[l, which] = torch.cat([p[key].reshape(-1, D) for p in secs]).to(device, torch.bfloat16)
                else:
                    for g, p in enumerate(secs):
                        t[l, which, g] = p[key].reshape(-1).to(device, torch.bfloat16)
        tables.append(t)
    return tables[0], tables[1]


def _table_views(dicts: Sequence[Dict], H: int, D: int, BS: int, G: int, axes: Tuple[str, str],
                 device) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """kmeta / vmeta as views when every section tensor already sits where the
    engine's one-allocation layout puts it (the K table followed by the V table, bf16)
    -- the case of a packet made by this engine, also after a wire round trip that
    shipped the allocation whole.  Pointer arithmetic only; None when any tensor is
    elsewhere (the caller then copies)."""
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
    shapes = [meta_shape(a, H, D, G, BS) for a in axes]
    sizes = [L * 2 * r * c for r, c in shapes]
    if (base - sp) % 2 or base - sp + 2 * sum(sizes) > st.nbytes():
        return None
    bases = (base, base + 2 * sizes[0])

    def at(t, addr, numel) -> bool:
        return (t is not None and t.dtype == torch.bfloat16 and t.is_contiguous() and t.numel() == numel
                and t.data_ptr() == addr and t.untyped_storage().data_ptr() == sp)

    for l, d in enumerate(dicts):
        for names, axis, (rows, cols), pbase in zip(_PARTS, axes, shapes, bases):
            r = 0  # next table row: a position (channel axis) or a group
            for s in names:
                mn = d[s]["min_val"]
                if mn is None:
                    continue
                n = mn.numel() // cols if axis == "channel" else 1
                if not (at(mn, pbase + 2 * ((2 * l) * rows + r) * cols, n * cols)
                        and at(d[s]["quant_scale"], pbase + 2 * ((2 * l + 1) * rows + r) * cols, n * cols)):
                    return None
                r += n
            if axis == "channel" and r != H:
                return None
    off = (base - sp) // 2
    kmeta = torch.empty(0, dtype=torch.bfloat16, device=device).set_(st, off, (L, 2) + shapes[0])
    vmeta = torch.empty(0, dtype=torch.bfloat16, device=device).set_(st, off + sizes[0], (L, 2) + shapes[1])
    return kmeta, vmeta


class QuantParams(_SequenceABC):
    """A layer range's "quantization_params" list in the reference's format, each dict
    built on first access (a dict per layer of four sections is most of the host time
    of a request otherwise).  `tables` = (kmeta, vmeta, start, stop): the engine tables
    of the whole request the range belongs to, when known -- the decoder and the wire
    then use them directly and never build the dicts."""

    def __init__(self, n: int, make: Callable[[int], Dict],
                 tables: Optional[Tuple[torch.Tensor, torch.Tensor, int, int]] = None, template=None):
        self._n, self._make, self._dicts = n, make, [None] * n
        self.tables, self.template = tables, template

    def __len__(self) -> int:
        return self._n

    def __getitem__(self, i):
        if isinstance(i, slice):
            return [self[j] for j in range(*i.indices(self._n))]
        if i < 0:
            i += self._n
        if not 0 <= i < self._n:
            raise IndexError("quantization_params index out of range")
        if self._dicts[i] is None:
            self._dicts[i] = self._make(i)
        return self._dicts[i]

    def __eq__(self, other) -> bool:
        return isinstance(other, (list, tuple, QuantParams)) and list(self) == list(other)

    def __repr__(self) -> str:
        return f"QuantParams({self._n} layers)"


def packet_params(kmeta: torch.Tensor, vmeta: torch.Tensor, profiles: Sequence[LayerProfile], B: int, S: int,
                  axes: Tuple[str, str], start: int, stop: int) -> QuantParams:
    """Layers [start, stop) of a packet's tables as a QuantParams."""
    return QuantParams(stop - start,
                       lambda i: layer_dict(kmeta[start + i], vmeta[start + i], profiles[start + i], B, S, axes),
                       (kmeta, vmeta, start, stop), (profiles, B, S, axes))


def joined_tables(params: Sequence) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """(kmeta, vmeta) of a request whose chunks' QuantParams cover the layers of one
    pair of tables in order; None otherwise (the caller converts dicts)."""
    pos, base = 0, None
    for qp in params:
        t = getattr(qp, "tables", None)
        if t is None:
            return None
        kmeta, vmeta, start, stop = t
        if base is None:
            base = (kmeta, vmeta)
        elif kmeta is not base[0] or vmeta is not base[1]:
            return None
        if start != pos:
            return None
        pos = stop
    if base is None or pos != base[0].shape[0]:
        return None
    return base


def section_entries(profiles: Sequence[LayerProfile], start: int, stop: int, B: int, S: int, axes: Tuple[str, str],
                    kshape: Tuple[int, ...], vshape: Tuple[int, ...]) -> Tuple[List, List]:
    """The wire image of layers [start, stop): for each layer the dict of placeholders
    (index relative to the first section) and, per section tensor in placeholder
    order, (byte offset in the metadata allocation, nbytes, keepdim shape) -- the K
    table [L,2,r,c] at offset 0 followed by the V table.  Sections of layer_dict."""
    H = len(profiles[0].k_order)
    D = kshape[3] if axes[0] == "channel" else vshape[3]
    tree, entries = [], []
    vbase = 2 * kshape[0] * kshape[1] * kshape[2] * kshape[3]
    for l in range(start, stop):
        prof = profiles[l]
        where = {}  # section name -> ((offset, nbytes, shape) of min, of scale)
        for (low_name, high_name), (base, shape), axis in zip(_PARTS, ((0, kshape), (vbase, vshape)), axes):
            _, _, rows, cols = shape
            for sec, lo, hi, g in _sections(prof, H):
                r0, n = (lo, hi - lo) if axis == "channel" else (g, 1)
                where[low_name if sec == "low" else high_name] = tuple(
                    (base + 2 * (((l * 2 + which) * rows + r0) * cols), 2 * n * cols,
                     list(_keepdim(axis, hi - lo, D, B, S))) for which in (0, 1))
        # placeholders are numbered in the order a walk of layer_dict's dict meets them
        out = {}
        for name in _SECTIONS:
            if name not in where:
                out[name] = _empty()
                continue
            idx = []
            for e in where[name]:
                entries.append(e)
                idx.append(len(entries) - 1)
            out[name] = {"min_val": idx[0], "quant_scale": idx[1], "original_dtype": "bfloat16", "quant_dtype": "uint8"}
        out["original_dtype"] = "bfloat16"
        tree.append(out)
    return tree, entries
