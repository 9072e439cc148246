"""KVCompressionAdapter -- the operator registry and connector-facing API.

Mirrors kvserve_v1/compression/manager.py:54-281: the same constructor
(compression_spec, num_kv_heads, head_size, model_name, tp_rank, tp_size), the
"default" and custom-dict modes, config normalisation, manager caching, and
compress(stacked_kv[L,2,B,S,H,D] or [L,2,T,H*D], request_id) /
decompress(CompressedKVData).  Paged variants compress straight from the per-layer
KV caches and decompress straight into them (the gather of kv_utils.py:59-80 and
the scatter of :83-119 fused into the kernels).

Registry (_build_manager, manager.py:187-216):
  pipeline stages          "transformer" -> KVServeTransformer (hadamard),
                           "quantizer"   -> KVServeQuantizer,
                           "codec"       -> KVServeCodec (codec_type "bitpack", or "rans" /
                                            "nvcomp" (ANS) / "lc" served by the GPU rANS codec)
  quantizer_config.impl    absent / "kvserve" / "hip_fused" -> the fused gfx950 manager
                           (same numerics as the modular torch operators);
                           "tilelang_fused" (also as top-level "impl" / "quantizer_impl")
                           -> FusedHadamardQuantizer (the compress_v3 numerics) in the
                           operator pipeline, with the normalisation of manager.py:151-185
                           (the transformer stage is folded into the quantizer);
                           "centered_codebook" is a CUDA-only implementation and is
                           rejected.
  The controller mode (online bandit profile selection) is outside this engine.
"""

from __future__ import annotations

import json
import logging
from typing import Any, Dict, Optional, Sequence, Tuple

import torch

from .codec import KVServeCodec
from .compression_manager import (CompressedKVData, CompressionConfig, CompressionManager,
                                  FusedCompressionManager, get_default_compression_config)
from .quantizer import FusedHadamardQuantizer, KVServeQuantizer
from .transformer import KVServeTransformer

log = logging.getLogger("kvserve_amd")

_COMPRESSED_SENTINEL = "__compressed__"
FUSED_IMPLS = (None, "kvserve", "hip_fused")
_CUDA_ONLY = ("centered_codebook",)
TILELANG_IMPL = "tilelang_fused"


def is_compressed_layer_names(layer_names: list) -> bool:
    return bool(layer_names) and layer_names[0] == _COMPRESSED_SENTINEL


def strip_sentinel(layer_names: list) -> list:
    return layer_names[1:] if is_compressed_layer_names(layer_names) else layer_names


def add_sentinel(layer_names: list) -> list:
    return [_COMPRESSED_SENTINEL] + layer_names


def _cfg_cache_key(cfg: dict) -> str:
    return json.dumps(cfg, sort_keys=True, default=str)


class KVCompressionAdapter:
    def __init__(self, compression_spec: Any, num_kv_heads: int, head_size: int, model_name: Optional[str] = None,
                 tp_rank: int = 0, tp_size: int = 1):
        self._num_kv_heads = num_kv_heads
        self._head_size = head_size
        self._model_name = model_name
        self._tp_rank = tp_rank
        self._tp_size = tp_size
        self._manager_cache: Dict[str, Tuple[CompressionManager, CompressionConfig]] = {}
        if isinstance(compression_spec, dict) and compression_spec.get("mode") == "controller":
            raise NotImplementedError("the online controller mode is not part of the ROCm compression engine")
        if compression_spec == "default":
            cfg = get_default_compression_config()
            if model_name and "quantizer_config" in cfg:
                cfg["quantizer_config"]["model_name"] = model_name
        else:
            cfg = compression_spec
        self._manager = self._build_manager(cfg)
        self._config = self._make_config(cfg)

    # ---------------------------------------------------------------- config
    @staticmethod
    def _impl(cfg: dict) -> Optional[str]:
        if cfg.get("impl") is not None:
            return cfg.get("impl")
        if cfg.get("quantizer_impl") is not None:
            return cfg.get("quantizer_impl")
        return (cfg.get("quantizer_config") or {}).get("impl")

    @staticmethod
    def _is_tilelang_fused(cfg: dict) -> bool:
        """manager.py:151-158."""
        if cfg.get("impl") == TILELANG_IMPL or cfg.get("quantizer_impl") == TILELANG_IMPL:
            return True
        return (cfg.get("quantizer_config") or {}).get("impl") == TILELANG_IMPL

    @classmethod
    def _normalize_tilelang(cls, cfg: dict) -> dict:
        """manager.py:160-185: one fused configuration at construction and per request
        -- the quantizer carries the Hadamard seed and the transformer stage goes."""
        if (cfg.get("quantizer_config") or {}).get("impl") == "centered_codebook":
            raise ValueError("centered_codebook cannot use the tilelang_fused implementation")
        pipeline = list(cfg.get("pipeline", []))
        if "quantizer" not in pipeline:
            raise ValueError("tilelang_fused requires a quantizer pipeline stage")
        qc = dict(cfg.get("quantizer_config") or {})
        qc["impl"] = TILELANG_IMPL
        if "transformer" in pipeline:
            tc = dict(cfg.get("transformer_config") or {})
            if tc.get("transform_type", "hadamard") != "hadamard":
                raise ValueError("tilelang_fused only fuses the Hadamard transformer")
            seed = tc.get("seed", 0x3333)
            explicit = qc.get("base_seed", qc.get("seed"))
            if "seed" in tc and explicit is not None and int(explicit) != int(seed):
                raise ValueError("Conflicting transformer seed and fused quantizer seed")
            qc.setdefault("base_seed", explicit if explicit is not None else seed)
            pipeline = [p for p in pipeline if p != "transformer"]
        cfg["quantizer_config"] = qc
        cfg["pipeline"] = pipeline
        for stage in pipeline:
            if stage not in ("quantizer", "codec"):
                raise ValueError(f"unknown pipeline stage '{stage}'")
        return cfg

    @classmethod
    def _normalize_config(cls, cfg: dict) -> dict:
        """Validate the implementation choice and the pipeline stages."""
        cfg = dict(cfg)
        if cls._is_tilelang_fused(cfg):
            return cls._normalize_tilelang(cfg)
        impl = cls._impl(cfg)
        if impl in _CUDA_ONLY:
            raise ValueError(f"quantizer impl '{impl}' is a CUDA-only implementation; use 'hip_fused'")
        if impl not in FUSED_IMPLS:
            raise ValueError(f"unknown quantizer impl '{impl}'")
        pipeline = list(cfg.get("pipeline", []))
        if impl == "hip_fused" and "quantizer" not in pipeline:
            raise ValueError("hip_fused requires a quantizer pipeline stage")
        for stage in pipeline:
            if stage not in ("transformer", "quantizer", "codec"):
                raise ValueError(f"unknown pipeline stage '{stage}'")
        return cfg

    def _make_config(self, cfg: dict) -> CompressionConfig:
        cfg = self._normalize_config(cfg)
        qc = cfg.get("quantizer_config")
        if qc is not None:
            qc = {k: v for k, v in qc.items() if k != "impl" or v == TILELANG_IMPL}
            qc["tp_rank"] = self._tp_rank
            qc["tensor_parallel_size"] = self._tp_size
        return CompressionConfig(enabled=cfg.get("enabled", True), pipeline=cfg.get("pipeline", []),
                                 transformer_config=cfg.get("transformer_config"), quantizer_config=qc,
                                 codec_config=cfg.get("codec_config"),
                                 min_compress_size=cfg.get("min_compress_size", 0))

    def _build_manager(self, cfg: dict) -> CompressionManager:
        cfg = self._normalize_config(cfg)
        pipeline = list(cfg.get("pipeline", []))
        config = self._make_config(cfg)
        transformer = KVServeTransformer if "transformer" in pipeline else None
        codec = KVServeCodec if "codec" in pipeline else None
        if self._is_tilelang_fused(cfg):
            return CompressionManager(config=config, transformer=transformer, quantizer=FusedHadamardQuantizer,
                                      codec=codec)
        quantizer = KVServeQuantizer if "quantizer" in pipeline else None
        cls = FusedCompressionManager if "quantizer" in pipeline else CompressionManager
        return cls(config=config, transformer=transformer, quantizer=quantizer, codec=codec)

    def _get_cached_manager(self, cfg: dict):
        key = _cfg_cache_key(cfg)
        if key not in self._manager_cache:
            self._manager_cache[key] = (self._build_manager(cfg), self._make_config(cfg))
        return self._manager_cache[key]

    # ---------------------------------------------------------------- public API
    def compress(self, stacked_kv: torch.Tensor, request_id: str) -> Optional[CompressedKVData]:
        meta = {"original_dtype": str(stacked_kv.dtype).replace("torch.", ""),
                "original_shape": list(stacked_kv.shape)}
        if stacked_kv.ndim == 6:
            x = stacked_kv.contiguous()
        elif stacked_kv.ndim == 4:
            L, _, T, _ = stacked_kv.shape
            x = stacked_kv.contiguous().view(L, 2, 1, T, self._num_kv_heads, self._head_size)
        else:
            raise ValueError(f"Unsupported KV tensor rank for compression: {stacked_kv.ndim}, "
                             f"shape={tuple(stacked_kv.shape)}")
        return self._manager.compress_all_layers(all_layers_data=x, request_id=request_id, config=self._config,
                                                 metadata=meta)

    def decompress(self, compressed: CompressedKVData) -> Optional[torch.Tensor]:
        result = self._manager.decompress_all_layers(compressed, config=self._config)
        if result is None:
            return None
        if isinstance(result, list):
            result = torch.cat(result, dim=0)
        shape = compressed.metadata.get("original_shape")
        if shape is not None:
            return result.contiguous().view(*[int(s) for s in shape])
        L = result.shape[0]
        return result.contiguous().view(L, 2, -1, self._num_kv_heads * self._head_size)

    def compress_paged(self, kv_caches: Sequence[torch.Tensor], block_ids, request_id: str,
                       layer_ids: Optional[Sequence[int]] = None) -> Optional[CompressedKVData]:
        """Compress blocks `block_ids` of every layer straight from vLLM's paged caches
        ([2, num_blocks, block_size, H, D] each, in the connector's sorted layer order)."""
        mgr = self._manager
        if not isinstance(mgr, FusedCompressionManager):
            raise ValueError("paged compression needs a quantizer stage")
        mgr.update_config(self._config)
        n = len(block_ids) if not isinstance(block_ids, torch.Tensor) else block_ids.numel()
        _, _, S, H, D = kv_caches[0].shape
        shape = [len(kv_caches), 2, n, S, H, D]
        raw = len(kv_caches) * 2 * n * S * H * D * kv_caches[0].element_size()
        if not self._config.enabled or not self._config.pipeline or raw < self._config.min_compress_size:
            return None
        try:
            return mgr.compress_pools(list(kv_caches), block_ids, request_id,
                                      {"original_dtype": "bfloat16", "original_shape": shape}, layer_ids)
        except Exception as e:
            log.error("[KVCompressionAdapter] paged compression failed for %s: %s", request_id, e)
            return None

    def update_controller(self, request_id: str, observed_latency_ms: float) -> None:
        """Latency feedback for the online controller (manager.py:283-290); without
        the controller mode there is nothing to update."""
        return None

    def get_controller_stats(self) -> Optional[dict]:
        """manager.py:292-296: None outside the controller mode."""
        return None

    def decompress_paged(self, compressed: CompressedKVData, kv_caches: Sequence[torch.Tensor], block_ids) -> None:
        """Decompress into the paged caches at `block_ids` (the first num_blocks ids)."""
        mgr = self._manager
        if not isinstance(mgr, FusedCompressionManager):
            raise ValueError("paged decompression needs a quantizer stage")
        mgr.update_config(self._config)
        mgr.decompress_pools(compressed, list(kv_caches), block_ids)
