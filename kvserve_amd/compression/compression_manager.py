"""CompressionManager for the MI355X engine.

Mirrors kvserve_v1/compression/compression_manager.py (CompressionConfig :51-65,
CompressedKVData :68-82, compress_all_layers :200-537, decompress_all_layers
:539-757): the same input [L, 2, B, S, H, D], the 500 MiB / 8-layer chunk rule, the
permuted / native codec layouts (KVSERVE_CODEC_LAYOUT), the same metadata keys, and
None on failure.

Two implementations share that surface:
  CompressionManager       runs the configured operators one layer at a time
                           (Transformer -> Quantizer -> Codec), as the reference does;
  FusedCompressionManager  runs the whole Hadamard + min-max + bitpack pipeline of all
                           layers in two gfx950 launches (one to decompress) and falls
                           back to the operator loop for configurations it does not fuse.
"""

from __future__ import annotations

import copy
import logging
import os
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Sequence

import torch

from ..engine import DEFAULT_SEED, FusedKVCodec, Packet, check_packet, chunk_ranges, supported_geometry
from ._meta import joined_tables, packet_params, tables_from_dicts
from .codec import is_entropy_codec
from .codec.rans_codec import unpack_target
from .. import ops

log = logging.getLogger("kvserve_amd")

_CODEC_LAYOUT_ENV = "KVSERVE_CODEC_LAYOUT"

# The reference default (compression_manager.py:23-43); its nvCOMP ANS codec stage is
# served by this engine's rANS codec (same role, this engine's stream format).
DEFAULT_COMPRESSION_CONFIG: Dict[str, Any] = {
    "enabled": True,
    "pipeline": ["quantizer", "codec"],
    "quantizer_config": {
        "model_name": "Llama-3.1-8B-Instruct",
        "hybrid_ratio": 0.8,
        "high_key_max_value": 12,
        "high_value_max_value": 8,
        "low_key_max_value": 6,
        "low_value_max_value": 4,
        "axis_key": "channel",
        "axis_value": "token",
        "split_type": "head",
    },
    "codec_config": {"codec_type": "nvcomp", "nvcomp_algorithm": "ANS", "data_type": "|u1"},
    "min_compress_size": 1024,
}


def get_default_compression_config() -> Dict[str, Any]:
    return copy.deepcopy(DEFAULT_COMPRESSION_CONFIG)


@dataclass
class CompressionConfig:
    enabled: bool = False
    transformer_config: Optional[Dict[str, Any]] = None
    quantizer_config: Optional[Dict[str, Any]] = None
    codec_config: Optional[Dict[str, Any]] = None
    pipeline: Optional[List[str]] = None
    min_compress_size: int = 0


@dataclass
class CompressedKVData:
    request_id: str
    layer_id: int
    compressed_tensor: Optional[torch.Tensor] = None
    metadata: Dict[str, Any] = None
    original_size: int = 0
    compressed_size: int = 0
    is_chunked: bool = False
    chunks: Optional[List[torch.Tensor]] = None
    chunk_metadata: Optional[List[Dict[str, Any]]] = None


def symbol_bits(config: "CompressionConfig") -> int:
    """Width of the values the codec stage codes: `bitpack_bits` for the bitpack
    codec; for an entropy codec, bit_length of the largest level count when a
    quantizer runs (the quantizer clamps to L inclusive, quantizer_func.py:65), else
    8 (bytes)."""
    cc = config.codec_config or {}
    if not is_entropy_codec(cc):
        return int(cc.get("bitpack_bits", 8))
    qc = config.quantizer_config or {}
    if "quantizer" not in (config.pipeline or []):
        return 8
    top = max(int(qc.get(k, d)) for k, d in (("high_key_max_value", 16), ("high_value_max_value", 16),
                                             ("low_key_max_value", 12), ("low_value_max_value", 12)))
    return max(1, min(8, top.bit_length()))


def codec_layout() -> str:
    layout = os.environ.get(_CODEC_LAYOUT_ENV, "permuted").strip().lower()
    return layout if layout in ("native", "permuted") else "permuted"


class CompressionManager:
    """Operator-by-operator pipeline (compression_manager.py:84-841)."""

    def __init__(self, config: CompressionConfig, transformer=None, quantizer=None, codec=None):
        self.config = config
        self.transformer = transformer(**(config.transformer_config or {})) if transformer else None
        self.quantizer = quantizer(**(config.quantizer_config or {})) if quantizer else None
        self.codec = codec(**(config.codec_config or {})) if codec else None
        self.original_size = 0
        self.compressed_size = 0
        if config.enabled and config.pipeline:
            for name in config.pipeline:
                if name == "transformer" and self.transformer is None:
                    raise ValueError("Transformer component required but not provided")
                if name == "quantizer" and self.quantizer is None:
                    raise ValueError("Quantizer component required but not provided")
                if name == "codec" and self.codec is None:
                    raise ValueError("Codec compression component required but not provided")

    def update_config(self, config: CompressionConfig) -> None:
        self.config = config
        if self.transformer is not None:
            self.transformer.update_params(**(config.transformer_config or {}))
        if self.quantizer is not None:
            self.quantizer.update_params(**(config.quantizer_config or {}))
        if self.codec is not None:
            self.codec.update_params(**(config.codec_config or {}))

    # ---------------------------------------------------------------- compress
    def compress_all_layers(self, all_layers_data, request_id: str, config: CompressionConfig,
                            metadata: Dict[str, Any]) -> Optional[CompressedKVData]:
        self.update_config(config)
        if not self.config.enabled or not self.config.pipeline:
            return None
        if not isinstance(all_layers_data, torch.Tensor) or all_layers_data.dim() != 6:
            log.error("[CompressionManager] all_layers_data must be a 6D tensor")
            return None
        try:
            L = all_layers_data.shape[0]
            original_size = all_layers_data.numel() * all_layers_data.element_size()
            if original_size < self.config.min_compress_size:
                return None
            chunks = chunk_ranges(L, original_size)
            if len(chunks) == 1:
                tensor, meta = self._compress_range(all_layers_data, 0, L, request_id, metadata)
                meta["original_size"] = original_size
                return CompressedKVData(request_id, L - 1, tensor, meta, original_size,
                                        tensor.numel() * tensor.element_size())
            tensors, metas = [], []
            for ci, (s, e) in enumerate(chunks):
                t, m = self._compress_range(all_layers_data, s, e, request_id, metadata)
                m.update({"chunk_index": ci, "total_chunks": len(chunks)})
                tensors.append(t)
                metas.append(m)
            total = sum(t.numel() * t.element_size() for t in tensors)
            return CompressedKVData(request_id, L - 1, None,
                                    {"request_id": request_id, "original_size": original_size, "num_layers": L,
                                     "is_chunked": True, "num_chunks": len(chunks), **metadata},
                                    original_size, total, True, tensors, metas)
        except Exception as e:  # the reference returns None and the connector sends raw KV
            log.error("[CompressionManager] compression failed for %s: %s", request_id, e)
            return None

    def _base_meta(self, x: torch.Tensor, start: int, stop: int, request_id: str, metadata: Dict) -> Dict:
        return {"request_id": request_id, "original_dtype": str(x.dtype).replace("torch.", ""),
                "device": str(x.device), "start_layer_id": start, "num_layers": stop - start,
                "codec_layout": codec_layout(), **metadata}

    def _compress_range(self, x: torch.Tensor, start: int, stop: int, request_id: str, metadata: Dict):
        meta = self._base_meta(x, start, stop, request_id, metadata)
        layout = meta["codec_layout"]
        pipe = self.config.pipeline
        bufs, qparams = [], []
        for l in range(start, stop):
            cur = x[l]
            if "transformer" in pipe:
                cur = self.transformer.transform(l, cur, **(self.config.transformer_config or {}))
                meta["transformer_applied"] = True
            if "quantizer" in pipe:
                cur, qp = self.quantizer.quantize(l, cur, **(self.config.quantizer_config or {}))
                qparams.append(qp)
                meta["quantization_applied"] = True
            bufs.append(cur.permute(0, 3, 1, 2, 4) if layout == "permuted" else cur)
        buf = torch.stack(bufs).contiguous()
        if "quantizer" in pipe:
            meta["quantization_params"] = qparams
        meta["codec_shape"] = list(buf.shape)
        meta["codec_dtype"] = str(buf.dtype).replace("torch.", "")
        if "codec" in pipe:
            try:
                out = self.codec.encode(stop - 1, buf, **self._codec_kwargs())
                meta["codec_applied"] = True
                if is_entropy_codec(self.config.codec_config):
                    meta["codec_symbol_bits"] = symbol_bits(self.config)
            except Exception as e:  # compression_manager.py:781-793
                log.error("[CompressionManager] codec failed: %s", e)
                out = buf.reshape(-1).view(torch.uint8).contiguous()
                meta["codec_skipped"] = True
                meta["codec_error"] = f"{type(e).__name__}: {e}"
        else:
            out = buf.reshape(-1).view(torch.uint8).contiguous()
        meta["compressed_size"] = out.numel() * out.element_size()
        return out, meta

    # ---------------------------------------------------------------- decompress
    def decompress_all_layers(self, compressed_data: CompressedKVData, config: CompressionConfig):
        self.update_config(config)
        if not self.config.enabled or not self.config.pipeline:
            return None
        try:
            if compressed_data.is_chunked:
                if not compressed_data.chunks or not compressed_data.chunk_metadata:
                    log.error("[CompressionManager] chunked data missing chunks or metadata")
                    return None
                return [self._decompress_range(t, m) for t, m in
                        zip(compressed_data.chunks, compressed_data.chunk_metadata)]
            if compressed_data.metadata.get("num_layers") is None:
                log.error("[CompressionManager] Missing num_layers in metadata.")
                return None
            return self._decompress_range(compressed_data.compressed_tensor, compressed_data.metadata)
        except Exception as e:
            log.error("[CompressionManager] decompression failed for %s: %s", compressed_data.request_id, e)
            return None

    def _codec_kwargs(self) -> Dict[str, Any]:
        kw = dict(self.config.codec_config or {})
        if is_entropy_codec(kw):
            kw["symbol_bits"] = symbol_bits(self.config)
        return kw

    def _decode_codec(self, tensor: torch.Tensor, meta: Dict) -> torch.Tensor:
        shape, dtype = meta.get("codec_shape"), meta.get("codec_dtype")
        if "codec" in self.config.pipeline and meta.get("codec_applied", False):
            return self.codec.decode(meta.get("start_layer_id", 0), tensor, dtype, shape, meta.get("device"),
                                     **self._codec_kwargs())
        return tensor.view(getattr(torch, dtype)).reshape(shape)

    def _decompress_range(self, tensor: torch.Tensor, meta: Dict) -> torch.Tensor:
        cur = self._decode_codec(tensor, meta)
        if meta.get("codec_layout", "permuted") == "permuted":
            cur = cur.permute(0, 1, 3, 4, 2, 5).contiguous()
        start, n = meta.get("start_layer_id", 0), meta["num_layers"]
        target = getattr(torch, meta.get("original_dtype", "bfloat16"), torch.bfloat16)
        out = torch.empty(tuple(cur.shape), dtype=target, device=cur.device)
        for i in range(n):
            layer = cur[i]
            if "quantizer" in self.config.pipeline:
                qp = meta.get("quantization_params", [])
                if i >= len(qp) or qp[i] is None:
                    raise ValueError("Missing quantization params")
                layer = self.quantizer.dequantize(start + i, layer, qp[i], **(self.config.quantizer_config or {}))
            if "transformer" in self.config.pipeline:
                layer = self.transformer.inverse(start + i, layer, **(self.config.transformer_config or {}))
            out[i].copy_(layer.to(target))
        return out


class FusedCompressionManager(CompressionManager):
    """All layers of a request in fused gfx950 launches (same surface and metadata)."""

    def __init__(self, config: CompressionConfig, transformer=None, quantizer=None, codec=None):
        super().__init__(config, transformer, quantizer, codec)
        self._codecs: Dict[tuple, FusedKVCodec] = {}

    # ---------------------------------------------------------------- fusability
    def _settings(self):
        pipe = self.config.pipeline or []
        tc = self.config.transformer_config or {}
        cc = self.config.codec_config or {}
        transform = "transformer" in pipe
        seed = int(tc.get("seed", DEFAULT_SEED)) if transform else DEFAULT_SEED
        has_codec = "codec" in pipe
        bits = symbol_bits(self.config) if has_codec else 8
        return transform, seed, has_codec, bits

    def _entropy(self) -> bool:
        return "codec" in (self.config.pipeline or []) and is_entropy_codec(self.config.codec_config)

    def fusable(self, H: int, D: int, dtype) -> bool:
        pipe = self.config.pipeline or []
        if "quantizer" not in pipe or self.quantizer is None or not hasattr(self.quantizer, "layer_profile"):
            return False
        if "transformer" in pipe and (self.config.transformer_config or {}).get("transform_type",
                                                                                 "hadamard") != "hadamard":
            return False
        if "codec" in pipe and (self.config.codec_config or {}).get("codec_type", "nvcomp") not in (
                "bitpack", "rans", "nvcomp", "lc"):
            return False
        return dtype == torch.bfloat16 and supported_geometry(H, D, self._settings()[3])

    def _axes(self):
        return (self.quantizer.axis_key, self.quantizer.axis_value)

    def _codec(self, H, D, S) -> FusedKVCodec:
        transform, seed, has_codec, bits = self._settings()
        key = (H, D, S, transform, seed, has_codec, bits, codec_layout(), self._axes())
        if key not in self._codecs:
            self._codecs[key] = FusedKVCodec(H, D, S, bits, seed, transform=transform, layout=codec_layout(),
                                             header=has_codec, axes=self._axes())
        return self._codecs[key]

    def profiles(self, layer_ids: Sequence[int], H: int):
        """Layer profiles, cached per (layers, heads, quantizer settings): the same list
        object for every request of one shape (the wire caches its image by it)."""
        q = self.quantizer
        state = tuple(getattr(q, k, None) for k in (
            "split_type", "hybrid_ratio", "high_key_max_value", "high_value_max_value", "low_key_max_value",
            "low_value_max_value", "tensor_parallel_size", "tp_rank", "model_name"))
        key = (tuple(layer_ids), H, state, id(getattr(q, "head_scores_mask", None)),
               id(getattr(q, "layer_scores_mask", None)))
        cache = self.__dict__.setdefault("_profile_cache", {})
        hit = cache.get(key)
        if hit is None:
            if len(cache) > 64:
                cache.clear()
            hit = [q.layer_profile(l, H) for l in layer_ids]
            cache[key] = hit
        return hit

    # ---------------------------------------------------------------- compress
    def compress_all_layers(self, all_layers_data, request_id, config, metadata):
        self.update_config(config)
        if (not self.config.enabled or not self.config.pipeline or not isinstance(all_layers_data, torch.Tensor)
                or all_layers_data.dim() != 6):
            return super().compress_all_layers(all_layers_data, request_id, config, metadata)
        L, _, B, S, H, D = all_layers_data.shape
        if not self.fusable(H, D, all_layers_data.dtype) or not all_layers_data.is_cuda:
            return super().compress_all_layers(all_layers_data, request_id, config, metadata)
        try:
            x = all_layers_data.contiguous()
            original_size = x.numel() * x.element_size()
            if original_size < self.config.min_compress_size:
                return None
            ids = torch.arange(B, dtype=torch.int32, device=x.device)
            return self.compress_pools([x[l] for l in range(L)], ids, request_id, metadata)
        except Exception as e:
            log.error("[FusedCompressionManager] compression failed for %s: %s", request_id, e)
            return None

    def compress_pools(self, pools: Sequence[torch.Tensor], block_ids, request_id: str, metadata: Dict,
                       layer_ids: Optional[Sequence[int]] = None) -> CompressedKVData:
        """Fused gather + compress of blocks `block_ids` of per-layer caches
        [2, P, S, H, D]; layer i is the reference's layer index layer_ids[i]."""
        L = len(pools)
        _, _, S, H, D = pools[0].shape
        layer_ids = list(range(L)) if layer_ids is None else list(layer_ids)
        profs = self.profiles(layer_ids, H)
        codec = self._codec(H, D, S)
        packet = codec.compress(pools, block_ids, profs, layer_ids=layer_ids)
        # the metadata dicts are built while the kernels run; the error check (a
        # synchronization) comes last
        B = packet.num_blocks
        original_size = L * 2 * B * S * H * D * 2
        transform, seed, has_codec, bits = self._settings()
        layout = codec.layout
        metas = []
        for s, e in packet.chunks:
            m = {"request_id": request_id, "original_dtype": "bfloat16", "device": str(pools[0].device),
                 "start_layer_id": layer_ids[s], "num_layers": e - s, "codec_layout": layout, **metadata}
            if transform:
                m["transformer_applied"] = True
            m["quantization_applied"] = True
            m["quantization_params"] = packet_params(packet.kmeta, packet.vmeta, profs, B, S, packet.axes, s, e)
            m["codec_shape"] = [e - s, 2, H, B, S, D] if layout == "permuted" else [e - s, 2, B, S, H, D]
            m["codec_dtype"] = "uint8"
            if has_codec:
                m["codec_applied"] = True
            metas.append(m)
        streams = packet.streams  # without a codec: raw uint8 codec buffers (8 bits, no header)
        if self._entropy():
            # the codec stage: rANS over each chunk's packed symbols (the bitpack body)
            per = 2 * H * B * S * D
            streams = ops.rans_encode_batch([(st[16:], (e - s) * per) for (s, e), st in zip(packet.chunks, streams)],
                                            bits)
            for m in metas:
                m["codec_symbol_bits"] = bits
        for m, st in zip(metas, streams):
            m["compressed_size"] = st.numel()
        if len(streams) == 1:
            metas[0]["original_size"] = original_size
            check_packet(packet)
            return CompressedKVData(request_id, L - 1, streams[0], metas[0], original_size, streams[0].numel())
        for ci, m in enumerate(metas):
            m.update({"chunk_index": ci, "total_chunks": len(metas)})
        check_packet(packet)
        total = sum(st.numel() for st in streams)
        return CompressedKVData(request_id, L - 1, None,
                                {"request_id": request_id, "original_size": original_size, "num_layers": L,
                                 "is_chunked": True, "num_chunks": len(metas), **metadata},
                                original_size, total, True, list(streams), metas)

    # ---------------------------------------------------------------- decompress
    def _packet(self, streams, metas, device) -> Packet:
        m0 = metas[0]
        shape = m0["codec_shape"]
        layout = m0.get("codec_layout", "permuted")
        if layout == "permuted":
            _, _, H, B, S, D = shape
        else:
            _, _, B, S, H, D = shape
        chunks, start = [], m0.get("start_layer_id", 0)
        off = 0
        for m in metas:
            n = m["num_layers"]
            chunks.append((off, off + n))
            off += n
        params = [m.get("quantization_params") or [] for m in metas]
        if sum(len(p) for p in params) != off:
            raise ValueError("Missing quantization params")
        layer_ids = list(range(start, start + off))
        tables = joined_tables(params)  # tables of this engine's packet or bundle, as they are
        if tables is not None and tables[0].device == torch.device(device):
            kmeta, vmeta = tables
        else:
            kmeta, vmeta = tables_from_dicts([d for p in params for d in p], H, D, B, S, device, self._axes())
        transform, seed, has_codec, bits = self._settings()
        if not all(m.get("codec_applied", False) == has_codec for m in metas):
            raise ValueError("packet codec does not match the pipeline")
        if self._entropy():
            # undo the codec stage: each chunk back to its bitpack stream
            items, packed = [], []
            for (s, e), st in zip(chunks, streams):
                n = (e - s) * 2 * H * B * S * D
                packed.append(unpack_target(n, bits, device))
                items.append((st.to(device), n, packed[-1][16:]))
            ops.rans_decode_batch(items, bits)
            streams = packed
        return Packet(list(streams), chunks, kmeta, vmeta, self.profiles(layer_ids, H), B, S, H, D, bits, seed,
                      transform, layout, layer_ids, self._axes())

    def _fused_decodable(self, metas) -> bool:
        m = metas[0]
        shape = m.get("codec_shape")
        if not m.get("quantization_applied") or shape is None or len(shape) != 6:
            return False
        if m.get("original_dtype", "bfloat16") != "bfloat16" or m.get("codec_skipped"):
            return False
        D = shape[-1]
        H = shape[2] if m.get("codec_layout", "permuted") == "permuted" else shape[4]
        return self.fusable(H, D, torch.bfloat16) and bool(m.get("transformer_applied", False)) == (
            "transformer" in (self.config.pipeline or []))

    def decompress_all_layers(self, compressed_data: CompressedKVData, config: CompressionConfig):
        self.update_config(config)
        if not self.config.enabled or not self.config.pipeline:
            return None
        if compressed_data.is_chunked:
            streams, metas = compressed_data.chunks, compressed_data.chunk_metadata
        else:
            streams, metas = [compressed_data.compressed_tensor], [compressed_data.metadata]
        if not streams or not metas or streams[0] is None or not self._fused_decodable(metas):
            return super().decompress_all_layers(compressed_data, config)
        try:
            packet = self._packet(streams, metas, streams[0].device)
            L, B, S, H, D = packet.num_layers, packet.num_blocks, packet.block_size, packet.num_heads, packet.head_dim
            out = torch.empty((L, 2, B, S, H, D), dtype=torch.bfloat16, device=streams[0].device)
            self.decompress_into(packet, [out[l] for l in range(L)],
                                 torch.arange(B, dtype=torch.int32, device=out.device))
            if compressed_data.is_chunked:
                return [out[s:e] for s, e in packet.chunks]
            return out
        except Exception as e:
            log.error("[FusedCompressionManager] decompression failed for %s: %s", compressed_data.request_id, e)
            return None

    def decompress_into(self, packet: Packet, pools: Sequence[torch.Tensor], block_ids) -> None:
        codec = self._codec(packet.num_heads, packet.head_dim, packet.block_size)
        codec.decompress(packet, pools, block_ids)
        check_packet(packet)

    def decompress_pools(self, compressed_data: CompressedKVData, pools: Sequence[torch.Tensor], block_ids) -> None:
        """Fused decompress + scatter of a packet into per-layer caches [2, P, S, H, D]."""
        if compressed_data.is_chunked:
            streams, metas = compressed_data.chunks, compressed_data.chunk_metadata
        else:
            streams, metas = [compressed_data.compressed_tensor], [compressed_data.metadata]
        packet = self._packet(streams, metas, pools[0].device)
        self.decompress_into(packet, pools, block_ids)
