"""Fixed-profile runtime configuration (kvserve_v1/compression/runtime/config.py:14-221).

Same fields, defaults, JSON keys (``enable-compression-pipeline``, ``raw_aggregate`` /
``raw_agg``) and validation messages as the reference.  ``codec = "ans"`` selects this
engine's GPU rANS codec (nvCOMP ANS is closed NVIDIA code).
"""

from __future__ import annotations

import logging
from dataclasses import dataclass
from typing import Any, Dict, Literal, Optional, Tuple

logger = logging.getLogger("kvserve_amd.runtime")

QuantAxis = Literal["channel", "token", "tensor"]
SplitType = Literal["head", "layer"]
Transport = Literal["raw", "compression", "raw_aggregate"]

RAW_AGGREGATE_KEY = "raw_aggregate"
RAW_AGGREGATE_ALIAS = "raw_agg"
RAW_AGGREGATE_SLOT_COUNT = 2
RAW_AGGREGATE_LOGICAL_BLOCKS_PER_CHUNK = 160

_raw_aggregate_warned = False


def _parse_raw_aggregate(extra_config: Dict[str, Any]) -> Optional[Tuple[int, int]]:
    """(slot_count, logical_blocks_per_chunk), or None when the key is absent or
    disabled; ``raw_aggregate`` wins over ``raw_agg`` (config.py:28-62)."""
    if RAW_AGGREGATE_KEY in extra_config:
        raw = extra_config[RAW_AGGREGATE_KEY]
    elif RAW_AGGREGATE_ALIAS in extra_config:
        raw = extra_config[RAW_AGGREGATE_ALIAS]
    else:
        return None
    if raw is None or raw is False:
        return None
    if raw is True:
        raw = {}
    if not isinstance(raw, dict):
        raise ValueError(f"{RAW_AGGREGATE_KEY} must be true or an object with "
                         f"{RAW_AGGREGATE_SLOT_COUNT}/{RAW_AGGREGATE_LOGICAL_BLOCKS_PER_CHUNK}")
    unknown = set(raw) - {"slot_count", "logical_blocks_per_chunk"}
    if unknown:
        raise ValueError(f"Unknown {RAW_AGGREGATE_KEY} parameters: {sorted(unknown)}; "
                         "supported: slot_count, logical_blocks_per_chunk")
    slot_count = int(raw.get("slot_count", RAW_AGGREGATE_SLOT_COUNT))
    blocks = int(raw.get("logical_blocks_per_chunk", RAW_AGGREGATE_LOGICAL_BLOCKS_PER_CHUNK))
    if slot_count < 1:
        raise ValueError(f"{RAW_AGGREGATE_KEY}.slot_count must be >= 1")
    if blocks < 1:
        raise ValueError(f"{RAW_AGGREGATE_KEY}.logical_blocks_per_chunk must be >= 1")
    return slot_count, blocks


@dataclass(frozen=True)
class CompressionConfig:
    enabled: bool = False
    transport: Transport = "compression"
    transformer: Literal["hadamard"] = "hadamard"
    seed: int = 3237919422
    split_type: SplitType = "layer"
    score_path: Optional[str] = None
    hybrid_ratio: float = 0.8
    axis_key: QuantAxis = "channel"
    axis_value: QuantAxis = "token"
    high_key_num_levels: int = 12
    high_value_num_levels: int = 8
    low_key_num_levels: int = 6
    low_value_num_levels: int = 4
    codec: Literal["ans"] = "ans"
    slot_count: int = 2
    logical_blocks_per_chunk: int = 1
    pipeline: Tuple[str, ...] = ("transformer", "quantizer", "codec")

    @property
    def available(self) -> bool:
        return self.enabled

    @property
    def is_raw_aggregate(self) -> bool:
        return self.transport == "raw_aggregate"

    @property
    def uses_aggregate(self) -> bool:
        return "aggregate" in self.pipeline

    @property
    def uses_transformer(self) -> bool:
        return not self.uses_aggregate and "transformer" in self.pipeline

    @property
    def uses_quantizer(self) -> bool:
        return not self.uses_aggregate and "quantizer" in self.pipeline

    @property
    def uses_codec(self) -> bool:
        return not self.uses_aggregate and "codec" in self.pipeline

    @classmethod
    def from_extra_config(cls, extra_config: Dict[str, Any]) -> "CompressionConfig":
        """Parse ``kv_connector_extra_config`` (config.py:110-221)."""
        global _raw_aggregate_warned
        extra_config = extra_config or {}
        agg = _parse_raw_aggregate(extra_config)
        if agg is not None:
            compression = extra_config.get("compression") or {}
            if compression.get("enable-compression-pipeline", False) and not _raw_aggregate_warned:
                _raw_aggregate_warned = True
                logger.warning("raw_aggregate transport selected; ignoring compression parameters: %s",
                               ", ".join(sorted(str(k) for k in compression)))
            return cls(enabled=True, transport="raw_aggregate", pipeline=("aggregate",), slot_count=agg[0],
                       logical_blocks_per_chunk=agg[1])
        raw = extra_config.get("compression", {}) or {}
        if not raw.get("enable-compression-pipeline", False):
            return cls(enabled=False, transport="raw")
        normalized = dict(raw)
        normalized.pop("enable-compression-pipeline")
        if "pipeline" in normalized:
            normalized["pipeline"] = tuple(normalized["pipeline"])
        config = cls(enabled=True, transport="compression", **normalized)
        if config.transformer != "hadamard":
            raise ValueError("Mooncake compression only supports transformer='hadamard'.")
        if config.codec != "ans":
            raise ValueError("Mooncake compression only supports codec='ans'.")
        if type(config.slot_count) is not int or config.slot_count < 1:
            raise ValueError("Mooncake compression slot_count must be >= 1.")
        if type(config.logical_blocks_per_chunk) is not int or config.logical_blocks_per_chunk < 1:
            raise ValueError("Mooncake compression logical_blocks_per_chunk must be >= 1.")
        supported = {"aggregate", "transformer", "quantizer", "codec"}
        unknown = set(config.pipeline) - supported
        if unknown:
            raise ValueError(f"Unknown Mooncake compression stages: {sorted(unknown)}; "
                             f"supported stages: {sorted(supported)}")
        if len(set(config.pipeline)) != len(config.pipeline):
            raise ValueError("Mooncake compression stages must be unique.")
        if "aggregate" not in config.pipeline:
            ordered = tuple(s for s in ("transformer", "quantizer", "codec") if s in config.pipeline)
            if config.pipeline != ordered:
                raise ValueError("Mooncake compression stages must follow transformer, quantizer, codec order.")
        if "aggregate" in config.pipeline and len(config.pipeline) > 1:
            logger.warning("The aggregate stage takes precedence over other compression stages; "
                           "configure raw_aggregate for the preferred spelling.")
        if not 0.0 <= config.hybrid_ratio <= 1.0:
            raise ValueError("Mooncake compression hybrid_ratio must be in [0, 1].")
        for name in ("high_key_num_levels", "high_value_num_levels", "low_key_num_levels", "low_value_num_levels"):
            levels = getattr(config, name)
            if type(levels) is not int or not 2 <= levels <= 256:
                raise ValueError(f"Mooncake compression {name} must be an integer in [2, 256].")
        if config.split_type not in ("head", "layer"):
            raise ValueError(f"Unsupported Mooncake compression split_type: {config.split_type}")
        if config.axis_key not in ("channel", "token", "tensor"):
            raise ValueError(f"Unsupported Mooncake key quantization axis: {config.axis_key}")
        if config.axis_value not in ("channel", "token", "tensor"):
            raise ValueError(f"Unsupported Mooncake value quantization axis: {config.axis_value}")
        return config
