"""Versioned fixed-profile KV compression API for transfer / storage adapters
(kvserve_v1/compression/runtime/__init__.py:1-30).

The caller owns cache registration and slot scheduling.  The runtime owns bounded
codec buffers and returns events; callers fence them before reading a slot or
reusing it.  Nothing here imports vLLM or touches the network.
"""

from .config import CompressionConfig
from .manager import CompressionRuntime, build_signs, create_runtime
from .memory import build_memory_plan
from .spec import CacheSpec

API_VERSION = 1

__all__ = ["API_VERSION", "CacheSpec", "CompressionConfig", "CompressionRuntime", "build_memory_plan",
           "build_signs", "create_runtime"]
