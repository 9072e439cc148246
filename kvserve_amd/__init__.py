"""kvserve_amd -- MI355X (gfx950) engine for KVServe's KV-cache compression hot path.

  engine    FusedKVCodec: paged gather + FWHT + min-max quant + bitpack (and inverse)
  ops       unit operators: bitpack codec, paged gather / scatter, Hadamard
  profiles  signs recipe, head / layer masks, per-layer quantization profiles
  compression  drop-in mirror of kvserve_v1.compression (adapter, manager, operators)

The HIP library (``libkvserve_amd.so``, built by ``python -m kvserve_amd.build``) is
required: nothing here computes on the CPU.
"""

from ._lib import LIB_PATH, KvmiError, load  # noqa: F401

__all__ = ["LIB_PATH", "KvmiError", "load"]
