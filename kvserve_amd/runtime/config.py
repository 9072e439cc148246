"""Fixed-profile runtime configuration: the ``kv_connector_extra_config`` contract of
kvserve_v1/compression/runtime/config.py:14-221.

What peers depend on is kept as the reference has it: the dataclass fields and their
defaults, the JSON keys (``compression`` / ``enable-compression-pipeline``,
``raw_aggregate`` and its alias ``raw_agg``), the stage names and the error texts'
substance.  The parsing is this module's own: the aggregate request and the compression
object are each checked against a table of rules, and every rule carries the text of its
error.  ``codec = "ans"`` names this engine's GPU rANS codec (nvCOMP's ANS is closed
NVIDIA code).
"""

from __future__ import annotations

import logging
from dataclasses import dataclass, fields
from typing import Any, Callable, Dict, Literal, Optional, Tuple

logger = logging.getLogger("kvserve_amd.runtime")

QuantAxis = Literal["channel", "token", "tensor"]
SplitType = Literal["head", "layer"]
Transport = Literal["raw", "compression", "raw_aggregate"]

RAW_AGGREGATE_KEY = "raw_aggregate"
RAW_AGGREGATE_ALIAS = "raw_agg"
RAW_AGGREGATE_SLOT_COUNT = 2
RAW_AGGREGATE_LOGICAL_BLOCKS_PER_CHUNK = 160

ENABLE_KEY = "enable-compression-pipeline"
CODED_STAGES = ("transformer", "quantizer", "codec")  # the only order they may appear in
STAGES = frozenset(CODED_STAGES + ("aggregate",))
AXES = ("channel", "token", "tensor")
LEVEL_FIELDS = ("high_key_num_levels", "high_value_num_levels", "low_key_num_levels", "low_value_num_levels")

# Several components parse the same extra config (memory plan, connector); each
# warning below is logged once per process.
_warned: set = set()


def _warn_once(key: str, msg: str, *args) -> None:
    if key not in _warned:
        _warned.add(key)
        logger.warning(msg, *args)


def _count(value: Any) -> bool:
    """A positive int that is not a bool."""
    return type(value) is int and value >= 1


def _aggregate_request(extra: Dict[str, Any]) -> Optional[Tuple[int, int]]:
    """(slot_count, logical_blocks_per_chunk) when the lossless aggregate transport is
    requested, else None.  The canonical key shadows its alias; ``false`` / ``null``
    mean "not requested" and ``true`` means "with the defaults"."""
    key = next((k for k in (RAW_AGGREGATE_KEY, RAW_AGGREGATE_ALIAS) if k in extra), None)
    value = extra[key] if key else None
    if value is None or value is False:
        return None
    params = {} if value is True else value
    if not isinstance(params, dict):
        raise ValueError(f"{RAW_AGGREGATE_KEY} must be true or an object with "
                         f"{RAW_AGGREGATE_SLOT_COUNT}/{RAW_AGGREGATE_LOGICAL_BLOCKS_PER_CHUNK}")
    defaults = {"slot_count": RAW_AGGREGATE_SLOT_COUNT,
                "logical_blocks_per_chunk": RAW_AGGREGATE_LOGICAL_BLOCKS_PER_CHUNK}
    extra_keys = sorted(set(params) - set(defaults))
    if extra_keys:
        raise ValueError(f"Unknown {RAW_AGGREGATE_KEY} parameters: {extra_keys}; "
                         "supported: slot_count, logical_blocks_per_chunk")
    got = {name: int(params.get(name, default)) for name, default in defaults.items()}
    for name, value in got.items():
        if value < 1:
            raise ValueError(f"{RAW_AGGREGATE_KEY}.{name} must be >= 1")
    return got["slot_count"], got["logical_blocks_per_chunk"]


def _stage_order_ok(pipeline: Tuple[str, ...]) -> bool:
    """Without the aggregate stage the coded stages keep transformer < quantizer < codec."""
    if "aggregate" in pipeline:
        return True
    ranks = [CODED_STAGES.index(s) for s in pipeline]
    return ranks == sorted(ranks)


# (field, accepts(value), error text).  Checked in this order on an enabled
# configuration; an error text may use {value}.
_RULES: Tuple[Tuple[str, Callable[[Any], bool], str], ...] = (
    ("transformer", lambda v: v == "hadamard", "KVServe compression only supports transformer='hadamard'."),
    ("codec", lambda v: v == "ans", "KVServe compression only supports codec='ans'."),
    ("slot_count", _count, "KVServe compression slot_count must be >= 1."),
    ("logical_blocks_per_chunk", _count, "KVServe compression logical_blocks_per_chunk must be >= 1."),
    ("pipeline", lambda v: set(v) <= STAGES,
     "Unknown KVServe compression stages: {unknown}; supported stages: " + str(sorted(STAGES))),
    ("pipeline", lambda v: len(set(v)) == len(v), "KVServe compression stages must be unique."),
    ("pipeline", _stage_order_ok, "KVServe compression stages must follow transformer, quantizer, codec order."),
    ("hybrid_ratio", lambda v: 0.0 <= v <= 1.0, "KVServe compression hybrid_ratio must be in [0, 1]."),
    *((name, lambda v: type(v) is int and 2 <= v <= 256, f"KVServe compression {name} must be an integer in [2, 256].")
      for name in LEVEL_FIELDS),
    ("split_type", lambda v: v in ("head", "layer"), "Unsupported KVServe compression split_type: {value}"),
    ("axis_key", lambda v: v in AXES, "Unsupported KVServe key quantization axis: {value}"),
    ("axis_value", lambda v: v in AXES, "Unsupported KVServe value quantization axis: {value}"),
)


@dataclass(frozen=True)
class CompressionConfig:
    enabled: bool = False  # JSON key: enable-compression-pipeline
    transport: Transport = "compression"  # "raw" only for a disabled configuration
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
    pipeline: Tuple[str, ...] = CODED_STAGES

    @property
    def available(self) -> bool:
        return self.enabled

    @property
    def is_raw_aggregate(self) -> bool:
        return self.transport == "raw_aggregate"

    @property
    def uses_aggregate(self) -> bool:
        return "aggregate" in self.pipeline

    def _uses(self, stage: str) -> bool:
        # the aggregate stage replaces every coded stage
        return stage in self.pipeline and not self.uses_aggregate

    @property
    def uses_transformer(self) -> bool:
        return self._uses("transformer")

    @property
    def uses_quantizer(self) -> bool:
        return self._uses("quantizer")

    @property
    def uses_codec(self) -> bool:
        return self._uses("codec")

    def _validate(self) -> None:
        for name, accepts, text in _RULES:
            value = getattr(self, name)
            if not accepts(value):
                unknown = sorted(set(value) - STAGES) if name == "pipeline" else None
                raise ValueError(text.format(value=value, unknown=unknown))
        if self.uses_aggregate and len(self.pipeline) > 1:
            _warn_once("aggregate-stage", "The aggregate stage takes precedence over other compression "
                       "stages; configure raw_aggregate for the preferred spelling.")

    @classmethod
    def from_extra_config(cls, extra_config: Optional[Dict[str, Any]]) -> "CompressionConfig":
        """Parse ``kv_connector_extra_config``: the aggregate transport when requested
        (any compression object is then ignored, with a warning), else the compression
        object when enabled, else the raw transport."""
        extra = extra_config or {}
        compression = extra.get("compression") or {}
        aggregate = _aggregate_request(extra)
        if aggregate is not None:
            if compression.get(ENABLE_KEY, False):
                _warn_once("aggregate-shadows", "raw_aggregate transport selected; ignoring compression "
                           "parameters: %s", ", ".join(sorted(map(str, compression))))
            return cls(enabled=True, transport="raw_aggregate", pipeline=("aggregate",),
                       slot_count=aggregate[0], logical_blocks_per_chunk=aggregate[1])
        if not compression.get(ENABLE_KEY, False):
            return cls(enabled=False, transport="raw")  # the rest of the object is ignored
        params = {k: v for k, v in compression.items() if k != ENABLE_KEY}
        known = {f.name for f in fields(cls)}
        stray = sorted(set(params) - known)
        if stray:
            raise TypeError(f"unknown compression parameters: {stray}")
        if "pipeline" in params:
            params["pipeline"] = tuple(params["pipeline"])
        config = cls(enabled=True, transport="compression", **params)
        config._validate()
        return config
