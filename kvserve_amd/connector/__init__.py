"""vLLM v1 connector for compressed KV transfer (kvserve_v1/connector, kvserve_v1/utils/kv_utils.py).

  CompressedKVConnector            the connector; compresses and decompresses on the paged caches
  CompressedKVConnectorMetadata    per-step requests (ReqMeta) handed from scheduler to workers
  LoopbackTransport                in-process hand-off with the NcclTransport method surface
  extract / inject_kv_*_by_blocks  block-level copies between paged caches and stacked tensors
"""

from .compressed_kv_connector import (HAS_VLLM, CompressedKVConnector, CompressedKVConnectorMetadata,
                                      KVConnectorRole, ReqMeta)
from .kv_utils import extract_kv_from_layer_by_blocks, inject_kv_into_layer_by_blocks, make_slot_mapping
from .transport import LoopbackTransport

__all__ = ["HAS_VLLM", "CompressedKVConnector", "CompressedKVConnectorMetadata", "KVConnectorRole", "ReqMeta",
           "LoopbackTransport", "extract_kv_from_layer_by_blocks", "inject_kv_into_layer_by_blocks",
           "make_slot_mapping"]
