"""Wire bundle of a compressed KV payload (kvserve_v1/compression/wire.py:19-289).

A `CompressedKVData` is split into
  meta         msgpack-safe dict (no tensors): sizes, ids, body layout, and the
               metadata dicts with every tensor replaced by a placeholder
               ``["__kvserve_aux_tensor__", index]`` (wire.py:16, :176-202);
  body_chunks  the packed stream(s): the manager's layer chunks as they are
               ("manager_chunks"), one stream ("single"), or one stream cut into
               pieces of at most `max_chunk_bytes` ("byte_chunks") (wire.py:35-90);
  aux_tensors  the metadata tensors; more than one are carried as a single byte
               tensor plus ``meta["aux_layout"] = {"mode": "coalesced_bytes",
               "tensors": [{storage, offset, nbytes, shape, dtype}, ...]}``
               (wire.py:205-254).

The meta layout, the placeholder and the layout table are the reference's wire
format, so a bundle built here is read by the reference's `restore_from_wire` and
the other way round.  Where every metadata tensor is a contiguous slice of one
allocation -- the fused engine keeps K and V metadata in one buffer -- the aux
tensor is a view of that allocation and nothing is copied (an allocation used from
its start is shipped to its end when the unused tail is shorter than the used
span, so the receiver can view the engine's tables whole); otherwise the tensors
are copied into one byte tensor, each at an offset aligned to its element size.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple

import torch

from ._meta import QuantParams, section_entries
from .compression_manager import CompressedKVData

AUX_PLACEHOLDER = "__kvserve_aux_tensor__"
# Extra key of a bundle whose aux blob holds the engine's metadata tables whole: where
# the K and V tables sit in it, so a receiver of this engine views them directly; a
# reference receiver ignores the key and reads the placeholders as usual.
TABLES_KEY = "kvserve_tables"


class _Aux:
    """Aux tensors in placeholder order: real tensors, or groups of sections of one
    metadata allocation described by (byte offset, nbytes, shape) entries."""

    def __init__(self):
        self.parts: List[Any] = []
        self.n = 0
        self.tables: Optional[Tuple[torch.Tensor, torch.Tensor]] = None  # of the groups, when any
        self.layout_rows: List[List[Dict[str, Any]]] = []  # aux_layout rows of each group

    def add(self, t: torch.Tensor) -> int:
        self.parts.append(t)
        self.n += 1
        return self.n - 1

    def add_group(self, alloc: torch.Tensor, entries: List[Tuple[int, int, list]]) -> int:
        self.parts.append((alloc, entries))
        self.n += len(entries)
        return self.n - len(entries)

    def tensors(self) -> List[torch.Tensor]:
        out = []
        for p in self.parts:
            if isinstance(p, torch.Tensor):
                out.append(p)
            else:
                alloc, entries = p
                b = _bytes_of(alloc)
                out += [b[o:o + n].view(torch.bfloat16).view(sh) for o, n, sh in entries]
        return out


def _bytes_of(alloc: torch.Tensor) -> torch.Tensor:
    """The whole storage of `alloc` as a 1-D uint8 tensor."""
    st = alloc.untyped_storage()
    return torch.empty(0, dtype=torch.uint8, device=alloc.device).set_(st, 0, (st.nbytes(),))


# wire images of QuantParams ranges: (profiles, range, shapes, axes, first index) -> (tree, entries, layout rows)
_TEMPLATES: Dict[tuple, tuple] = {}


@dataclass
class CompressedWire:
    """A compressed payload as msgpack metadata plus device tensors (wire.py:19-30)."""

    meta: Dict[str, Any]
    body_chunks: List[torch.Tensor]
    aux_tensors: List[torch.Tensor]

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.body_chunks + self.aux_tensors)


# ---------------------------------------------------------------------- build
def build_wire(compressed: CompressedKVData, max_chunk_bytes: int) -> CompressedWire:
    """Bundle `compressed` for transport (wire.py:33-90)."""
    aux = _Aux()
    meta: Dict[str, Any] = {
        "is_chunked": bool(compressed.is_chunked),
        "layer_id": compressed.layer_id,
        "original_size": compressed.original_size,
        "compressed_size": compressed.compressed_size,
        "metadata": _pack_meta(compressed.metadata, aux),
    }
    if compressed.is_chunked:
        if not compressed.chunks or not compressed.chunk_metadata:
            raise ValueError("Chunked CompressedKVData is missing chunks or metadata")
        meta["chunk_metadata"] = [_pack_meta(m, aux) for m in compressed.chunk_metadata]
        meta["body_mode"] = "manager_chunks"
        body = [c.contiguous() for c in compressed.chunks]
    else:
        if compressed.compressed_tensor is None:
            raise ValueError("Non-chunked CompressedKVData is missing compressed_tensor")
        t = compressed.compressed_tensor.contiguous()
        nbytes = t.numel() * t.element_size()
        if nbytes > max_chunk_bytes:
            body = _byte_pieces(t, max_chunk_bytes)
            meta["body_mode"] = "byte_chunks"
        else:
            body = [t]
            meta["body_mode"] = "single"
        meta["body_spec"] = _spec(t)
    aux_out = _coalesce(meta, aux)
    return CompressedWire(meta=meta, body_chunks=body, aux_tensors=aux_out)


def _pack_meta(obj: Any, aux: _Aux) -> Any:
    """Only "quantization_params" may carry tensors (wire.py:140-147); they become
    placeholders, and a tensor anywhere else is an error."""
    if not isinstance(obj, dict):
        _no_tensors(obj)
        return obj
    out = dict(obj)
    for k, v in out.items():
        if k == "quantization_params":
            packed = _pack_params(v, aux) if isinstance(v, QuantParams) else None
            out[k] = packed if packed is not None else _pack_tree(v, aux)
        else:
            _no_tensors(v)
    return out


def _pack_tree(obj: Any, aux: _Aux) -> Any:
    if isinstance(obj, torch.Tensor):
        return [AUX_PLACEHOLDER, aux.add(obj.contiguous())]
    if isinstance(obj, QuantParams):
        obj = list(obj)
    if isinstance(obj, dict):
        return {k: _pack_tree(v, aux) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return [_pack_tree(v, aux) for v in obj]
    return obj


def _one_allocation(kmeta: torch.Tensor, vmeta: torch.Tensor) -> bool:
    """The engine's layout: the K table at the start of one allocation, the V table
    right after it, both contiguous."""
    return (kmeta.is_contiguous() and vmeta.is_contiguous() and kmeta.storage_offset() == 0
            and kmeta.untyped_storage().data_ptr() == vmeta.untyped_storage().data_ptr()
            and vmeta.storage_offset() == kmeta.numel() and kmeta.dtype == vmeta.dtype == torch.bfloat16)


def _pack_params(qp: QuantParams, aux: _Aux) -> Optional[list]:
    """The placeholder tree of a QuantParams range straight from its tables (no dicts,
    no per-section tensors), from a cache of wire images keyed by the profile list
    and shapes; None when the range is not laid out as the engine lays it out."""
    if qp.tables is None or qp.template is None:
        return None
    kmeta, vmeta, start, stop = qp.tables
    profiles, B, S, axes = qp.template
    if not _one_allocation(kmeta, vmeta):
        return None
    first = aux.n
    key = (id(profiles), start, stop, B, S, tuple(axes), tuple(kmeta.shape), tuple(vmeta.shape), first)
    hit = _TEMPLATES.get(key)
    if hit is None or hit[0] is not profiles:
        rel_tree, entries = section_entries(profiles, start, stop, B, S, tuple(axes), tuple(kmeta.shape),
                                            tuple(vmeta.shape))
        tree = [{k: ({f: ([AUX_PLACEHOLDER, first + x] if f in ("min_val", "quant_scale") and x is not None else x)
                      for f, x in v.items()} if isinstance(v, dict) else v) for k, v in layer.items()}
                for layer in rel_tree]
        rows = [{"storage": 0, "offset": int(o), "nbytes": int(n), "shape": sh, "dtype": "bfloat16"}
                for o, n, sh in entries]
        if len(_TEMPLATES) > 256:
            _TEMPLATES.clear()
        hit = (profiles, tree, entries, rows)
        _TEMPLATES[key] = hit
    aux.add_group(kmeta, hit[2])
    aux.tables = (kmeta, vmeta)
    aux.layout_rows.append(hit[3])
    return hit[1]


def _spec(t: torch.Tensor) -> Dict[str, Any]:
    return {"shape": list(t.shape), "dtype": str(t.dtype).replace("torch.", "")}


def _byte_pieces(t: torch.Tensor, max_chunk_bytes: int) -> List[torch.Tensor]:
    """Consecutive pieces of at most max_chunk_bytes of t's bytes (views, wire.py:257-264)."""
    if max_chunk_bytes <= 0:
        raise ValueError("max_chunk_bytes must be positive")
    b = t.reshape(-1).view(torch.uint8)
    return [b[i:i + max_chunk_bytes] for i in range(0, b.numel(), max_chunk_bytes)]


def _coalesce(meta: Dict[str, Any], aux_in: _Aux) -> List[torch.Tensor]:
    """One byte tensor plus a layout table for more than one aux tensor (wire.py:205-237)."""
    groups = [p for p in aux_in.parts if not isinstance(p, torch.Tensor)]
    if groups and len(groups) == len(aux_in.parts) and aux_in.n > 1 and \
            all(g[0].untyped_storage().data_ptr() == groups[0][0].untyped_storage().data_ptr() for g in groups):
        # every section is part of the engine's one metadata allocation: ship it whole
        kmeta, vmeta = aux_in.tables
        meta["aux_layout"] = {"mode": "coalesced_bytes",
                              "tensors": [r for rows in aux_in.layout_rows for r in rows]}
        meta[TABLES_KEY] = {"k_offset": 0, "k_shape": list(kmeta.shape), "v_offset": 2 * kmeta.numel(),
                            "v_shape": list(vmeta.shape)}
        return [_bytes_of(kmeta)]
    aux = aux_in.tensors()
    if len(aux) <= 1:
        return aux
    dev = aux[0].device
    shared = _shared_storage_range(aux)
    if shared is not None:
        storage, lo, hi = shared
        blob = torch.empty(0, dtype=torch.uint8, device=dev).set_(storage, lo, (hi - lo,))
        offsets = [t.data_ptr() - storage.data_ptr() - lo for t in aux]
    else:
        offsets, pos = [], 0
        for t in aux:
            pos += (-pos) % t.element_size()
            offsets.append(pos)
            pos += t.numel() * t.element_size()
        blob = torch.zeros(pos, dtype=torch.uint8, device=dev)
        for t, off in zip(aux, offsets):
            n = t.numel() * t.element_size()
            if n:
                blob[off:off + n].copy_(t.reshape(-1).view(torch.uint8))
    meta["aux_layout"] = {
        "mode": "coalesced_bytes",
        "tensors": [{"storage": 0, "offset": int(off), "nbytes": t.numel() * t.element_size(),
                     "shape": list(t.shape), "dtype": str(t.dtype).replace("torch.", "")}
                    for t, off in zip(aux, offsets)],
    }
    return [blob]


def _shared_storage_range(aux: List[torch.Tensor]):
    """(storage, lo, hi) when every tensor is a contiguous slice of one storage at an
    offset that is a multiple of its element size relative to lo; else None."""
    st = aux[0].untyped_storage()
    base = st.data_ptr()
    spans = []
    for t in aux:
        if t.device != aux[0].device or not t.is_contiguous() or t.untyped_storage().data_ptr() != base:
            return None
        off = t.data_ptr() - base
        spans.append((off, off + t.numel() * t.element_size(), t.element_size()))
    lo = min(s[0] for s in spans)
    hi = max(s[1] for s in spans)
    if any((s[0] - lo) % s[2] for s in spans):
        return None
    # an allocation used from its start ships to its end when the unused tail is
    # shorter than the used span (the engine's metadata tables: the receiver can
    # then view them whole instead of copying section by section)
    if lo == 0 and st.nbytes() - hi < hi:
        hi = st.nbytes()
    return st, lo, hi


def _no_tensors(obj: Any) -> None:
    if isinstance(obj, torch.Tensor):
        raise TypeError("CompressedWire metadata still contains a tensor; extend wire packing for this metadata field.")
    if isinstance(obj, dict):
        for v in obj.values():
            _no_tensors(v)
    elif isinstance(obj, (list, tuple)):
        for v in obj:
            _no_tensors(v)


# ---------------------------------------------------------------------- restore
def restore_from_wire(wire: CompressedWire) -> CompressedKVData:
    """Rebuild the payload from a received bundle (wire.py:93-136).  The request id
    comes from the inner metadata.  A bundle of this engine (TABLES_KEY) is restored
    without expanding its sections: each chunk's quantization_params is a QuantParams
    over the received tables whose dicts are built only if someone reads them."""
    meta = wire.meta
    lazy = _LazyAux.of(wire.aux_tensors, meta)
    aux = lazy if lazy is not None else _expand(wire.aux_tensors, meta.get("aux_layout"))
    pos = [0]

    def unpack(m):
        if lazy is None:
            return _unpack_meta(m, aux)
        return lazy.unpack_meta(m, pos)

    inner = unpack(meta.get("metadata"))
    rid = str(inner.get("request_id", "unknown")) if isinstance(inner, dict) else "unknown"
    common = dict(request_id=rid, layer_id=int(meta.get("layer_id", -1)), metadata=inner,
                  original_size=int(meta.get("original_size", 0)),
                  compressed_size=int(meta.get("compressed_size", 0)))
    if bool(meta["is_chunked"]):
        return CompressedKVData(compressed_tensor=None, is_chunked=True, chunks=wire.body_chunks,
                                chunk_metadata=[unpack(m) for m in meta.get("chunk_metadata", [])],
                                **common)
    if meta.get("body_mode") == "byte_chunks":
        spec = meta["body_spec"]
        b = torch.cat([c.contiguous().view(torch.uint8).reshape(-1) for c in wire.body_chunks])
        tensor = b.view(getattr(torch, spec["dtype"])).reshape(spec["shape"])
    else:
        tensor = wire.body_chunks[0]
    return CompressedKVData(compressed_tensor=tensor, is_chunked=False, **common)


def _expand(aux: List[torch.Tensor], layout: Optional[Dict[str, Any]]) -> List[torch.Tensor]:
    if not layout:
        return aux
    if layout.get("mode") != "coalesced_bytes":
        raise ValueError(f"Unknown aux_layout mode: {layout.get('mode')}")
    if not aux:
        return []
    blob = aux[0].contiguous().view(torch.uint8).reshape(-1)
    out = []
    for e in layout.get("tensors", []):
        if int(e.get("storage", 0)) != 0:
            raise ValueError("Only single-storage aux_layout is supported")
        a, n = int(e["offset"]), int(e["nbytes"])
        out.append(blob[a:a + n].view(getattr(torch, e["dtype"])).reshape(e["shape"]))
    return out


def _unpack_meta(obj: Any, aux: List[torch.Tensor]) -> Any:
    if isinstance(obj, dict) and "quantization_params" in obj:
        obj = dict(obj)
        obj["quantization_params"] = _unpack_tree(obj["quantization_params"], aux)
    return obj


def _unpack_tree(obj: Any, aux: List[torch.Tensor]) -> Any:
    if isinstance(obj, list) and len(obj) == 2 and isinstance(obj[0], str) and obj[0] == AUX_PLACEHOLDER:
        return aux[int(obj[1])]
    if isinstance(obj, dict):
        return {k: _unpack_tree(v, aux) for k, v in obj.items()}
    if isinstance(obj, list):
        return [_unpack_tree(v, aux) for v in obj]
    return obj


class _LazyAux:
    """Aux tensors of a bundle that carries the engine's tables whole: section views
    are made on demand, and the K / V tables are viewed directly."""

    def __init__(self, blob: torch.Tensor, rows: List[Dict[str, Any]], kmeta: torch.Tensor, vmeta: torch.Tensor):
        self.blob, self.rows, self.kmeta, self.vmeta = blob, rows, kmeta, vmeta

    @classmethod
    def of(cls, aux: List[torch.Tensor], meta: Dict[str, Any]) -> Optional["_LazyAux"]:
        t = meta.get(TABLES_KEY)
        layout = meta.get("aux_layout") or {}
        if not t or layout.get("mode") != "coalesced_bytes" or len(aux) != 1:
            return None
        blob = aux[0].contiguous().view(torch.uint8).reshape(-1)
        views = []
        for off, shape in ((t["k_offset"], t["k_shape"]), (t["v_offset"], t["v_shape"])):
            n = 2 * int(torch.Size(shape).numel())
            if off % 2 or off + n > blob.numel():
                return None
            views.append(blob[off:off + n].view(torch.bfloat16).view(shape))
        return cls(blob, layout.get("tensors", []), views[0], views[1])

    def __getitem__(self, i: int) -> torch.Tensor:
        e = self.rows[int(i)]
        a, n = int(e["offset"]), int(e["nbytes"])
        return self.blob[a:a + n].view(getattr(torch, e["dtype"])).reshape(e["shape"])

    def unpack_meta(self, obj: Any, pos: List[int]) -> Any:
        """A chunk's metadata with its quantization_params as a QuantParams over the
        tables (layers [pos, pos + len)), each dict unpacked from the tree on access."""
        if not (isinstance(obj, dict) and isinstance(obj.get("quantization_params"), list)):
            return obj
        tree = obj["quantization_params"]
        obj = dict(obj)
        start = pos[0]
        pos[0] += len(tree)
        obj["quantization_params"] = QuantParams(len(tree), lambda i: _unpack_tree(tree[i], self),
                                                 (self.kmeta, self.vmeta, start, pos[0]))
        return obj
