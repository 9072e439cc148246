"""Fused Hadamard quantizer with fp32 statistics (quantizer_config.impl "tilelang_fused").

Mirrors TileLangFusedQuantizer (kvserve_v1/compression/quantizer/tilelang_quantizer.py:
56-181) over KVHadamardQuantOp.compress_v3 / decompress_v3
(kvserve_v1/tilelang_ops/kv_hadamard_quant.py:73-160, :1519-1599, :1645-1750): the
same configuration keys, validation and defaults, the same per-(layer, head) level
table, the same metadata dicts (float16 on the wire, tilelang_quantizer.py:23-53) and
in-place `out=` buffer contract; the arithmetic runs in the kvmi_v3_* HIP kernels
(fp32 FWHT in the reference's butterfly order, fp32 K / V statistics, V grouped over
heads of equal levels, roundf, natural head order).  It replaces the transformer and
quantizer stages of a pipeline (the adapter drops "transformer").
"""

from __future__ import annotations

import ctypes
from typing import Any, Dict, Optional, Tuple

import numpy as np
import torch

from ... import _lib
from ...profiles import head_low_mask, layer_low_mask, rademacher_sign_bits, scores_from_csv, tp_head_slice
from ..components import Quantizer

_ROUTING_KEYS = frozenset({"impl", "quantizer_impl", "tp_rank", "tensor_parallel_size"})


def _f16(t: Any) -> Any:
    if isinstance(t, torch.Tensor) and t.dtype == torch.float32:
        return t.to(torch.float16)
    return t


def _group_map(levels) -> list:
    """Heads with equal levels share a group; ids in order of first occurrence
    (kv_hadamard_quant.py:1382-1390)."""
    ids: Dict[float, int] = {}
    return [ids.setdefault(float(v), len(ids)) for v in levels]


def _stream_handle() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class FusedHadamardQuantizer(Quantizer):
    """Quantizer facade with the compress_v3 / decompress_v3 numerics."""

    # the manager may have the symbols written straight into its codec buffer
    supports_out_buffer = True

    def __init__(self, **kwargs: Any) -> None:
        self._cfg = dict(kwargs)
        self._validate_config(self._cfg)
        self._tables: Dict[tuple, tuple] = {}
        self._signs: Dict[tuple, torch.Tensor] = {}

    # ---------------------------------------------------------------- config (tilelang_quantizer.py:82-140)
    def update_params(self, **kwargs: Any) -> None:
        if not kwargs:
            return
        self._validate_config({**self._cfg, **kwargs})
        changed = False
        for key, value in kwargs.items():
            if self._cfg.get(key) != value:
                self._cfg[key] = value
                changed = True
        if changed:
            self._tables.clear()
            self._signs.clear()

    @staticmethod
    def _validate_config(cfg: dict) -> None:
        if cfg.get("axis_key", "channel") != "channel" or cfg.get("axis_value", "token") != "token":
            raise ValueError("tilelang_fused requires axis_key='channel' and axis_value='token'")
        if cfg.get("quant_type", "minmax") != "minmax":
            raise ValueError("tilelang_fused compress_v3 supports quant_type='minmax' only")
        if cfg.get("split_type", "head") not in {"head", "layer"}:
            raise ValueError("tilelang_fused split_type must be 'head' or 'layer'")

    def _settings(self) -> dict:
        cfg = {k: v for k, v in self._cfg.items() if k not in _ROUTING_KEYS}
        seed = cfg.get("base_seed")
        if seed is None:
            seed = cfg.get("seed", 0x3333)
        dtype = cfg.get("dtype", torch.bfloat16)
        if isinstance(dtype, str):
            dtype = getattr(torch, dtype.replace("torch.", ""))
        if dtype != torch.bfloat16:
            raise ValueError("the fused quantizer reconstructs bfloat16 KV")
        return dict(
            seed=int(seed),
            model_name=cfg.get("model_name"),
            hybrid_ratio=float(cfg.get("hybrid_ratio", 0.8)),
            hk=float(cfg.get("high_key_max_value", 12)),
            hv=float(cfg.get("high_value_max_value", 8)),
            lk=float(cfg.get("low_key_max_value", 6)),
            lv=float(cfg.get("low_value_max_value", 4)),
            split_type=cfg.get("split_type", "head"),
            tp_size=int(self._cfg.get("tensor_parallel_size", 1)),
            tp_rank=int(self._cfg.get("tp_rank", 0)),
        )

    def levels(self, layer_id: int, num_heads: int) -> Tuple[np.ndarray, np.ndarray]:
        """K and V levels (max_value) of every head of `layer_id`
        (KVHadamardQuantOp.__init__ and compress_v3, kv_hadamard_quant.py:105-153,
        :1546-1560): from the model's head-score CSV when it loads, else the high
        values for every head."""
        st = self._settings()
        try:
            scores = scores_from_csv(st["model_name"])
        except Exception:
            scores = None
        if scores is None:
            return np.full(num_heads, st["hk"], np.float32), np.full(num_heads, st["hv"], np.float32)
        mask = tp_head_slice(head_low_mask(scores, st["hybrid_ratio"]), num_heads, st["tp_size"], st["tp_rank"])
        if not 0 <= layer_id < mask.shape[0]:
            raise IndexError(f"layer {layer_id} outside the {mask.shape[0]}-layer head-score table")
        if st["split_type"] == "head":
            low = mask[layer_id]
        else:
            low = np.full(num_heads, bool(layer_low_mask(mask.shape[0])[layer_id]))
        k = np.where(low, st["lk"], st["hk"]).astype(np.float32)
        v = np.where(low, st["lv"], st["hv"]).astype(np.float32)
        return k, v

    def _device_tables(self, layer_id: int, H: int, D: int, device) -> tuple:
        key = (layer_id, H, D, str(device))
        if key not in self._tables:
            k, v = self.levels(layer_id, H)
            for lv in np.concatenate([k, v]):
                if not 1.0 < lv <= 255.0:
                    raise ValueError(f"quantization levels must be in (1, 255], got {lv}")
            seed = self._settings()["seed"]
            levels = torch.from_numpy(np.stack([k, v])).to(device)
            group = torch.tensor(_group_map(v), dtype=torch.int32, device=device)
            signs = torch.from_numpy(rademacher_sign_bits(seed, layer_id, H, D).view(np.int32)).to(device)
            self._tables[key] = (levels, group, signs)
        return self._tables[key]

    # ---------------------------------------------------------------- operator API
    def quantize(self, layer_id: int, tensor: torch.Tensor, out: Optional[torch.Tensor] = None,
                 **kwargs: Any) -> Tuple[torch.Tensor, dict]:
        """[2, blocks, block_size, H, D] bf16 -> (uint8 of the same shape, metadata)
        (tilelang_quantizer.py:142-162, kv_hadamard_quant.py:1519-1599)."""
        if kwargs:
            kwargs.pop("out", None)
            self.update_params(**kwargs)
        if tensor.dim() != 5 or tensor.shape[0] != 2:
            raise ValueError(f"expected [2, num_blocks, block_size, num_heads, head_dim], got {tuple(tensor.shape)}")
        if tensor.dtype != torch.bfloat16 or tensor.device.type != "cuda":
            raise ValueError("the fused quantizer takes bfloat16 KV on the GPU")
        x = tensor if tensor.is_contiguous() else tensor.contiguous()
        _, B, S, H, D = x.shape
        dev = x.device
        expected = (2, B, S, H, D)
        if out is None:
            out = torch.empty(expected, dtype=torch.uint8, device=dev)
        else:  # kv_hadamard_quant.py:1562-1578
            if tuple(out.shape) != expected:
                raise ValueError(f"compress_v3 out shape {tuple(out.shape)} != {expected}")
            if out.dtype != torch.uint8:
                raise ValueError(f"compress_v3 out dtype must be uint8, got {out.dtype}")
            if out.device != dev:
                raise ValueError(f"compress_v3 out device {out.device} != input device {dev}")
            if not out.is_contiguous():
                raise ValueError("compress_v3 out must be contiguous")
        rows = B * S
        lib = _lib.load()
        scratch_n = int(lib.kvmi_v3_scratch_bytes(rows, H, D))
        if scratch_n < 0:
            raise ValueError(f"unsupported geometry for the fused quantizer: heads={H}, head_dim={D}")
        levels, group, signs = self._device_tables(layer_id, H, D, dev)
        # no rows: no statistics are computed, and the K metadata is defined as zeros
        kmeta = (torch.zeros if rows == 0 else torch.empty)((2, H, D), dtype=torch.float32, device=dev)
        vmeta = torch.empty((2, rows, H), dtype=torch.float32, device=dev)
        scratch = torch.empty(max(scratch_n, 1), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            _lib.check(lib.kvmi_v3_compress(x.data_ptr(), rows, H, D, signs.data_ptr(), levels.data_ptr(),
                                            group.data_ptr(), out.data_ptr(), kmeta.data_ptr(), vmeta.data_ptr(),
                                            scratch.data_ptr(), _stream_handle()), "kvmi_v3_compress")
        meta = {"key_meta": {"min_val": _f16(kmeta[0]), "quant_scale": _f16(kmeta[1]), "axis": "channel"},
                "value_meta": {"min_val": _f16(vmeta[0]), "quant_scale": _f16(vmeta[1]), "axis": "token_perhead"}}
        return out, meta

    @staticmethod
    def _value_tables(vm: dict, rows: int, H: int, device) -> Tuple[torch.Tensor, torch.Tensor]:
        """Dense float16 [rows, H] (min, scale) from any value-metadata form the
        reference decodes (kv_hadamard_quant.py:1666-1707)."""
        if "per_group_list" in vm or "per_group_meta" in vm:
            groups = vm["per_group_list"] if "per_group_list" in vm else list(vm["per_group_meta"].values())
            mn = torch.empty((rows, H), dtype=torch.float16, device=device)
            sc = torch.empty((rows, H), dtype=torch.float16, device=device)
            for gm in groups:
                idx = torch.as_tensor(gm["head_idx"], device=device).long()
                m = gm["min_val"].to(device=device, dtype=torch.float16).reshape(-1)[:rows]
                s = gm["quant_scale"].to(device=device, dtype=torch.float16).reshape(-1)[:rows]
                mn[:, idx] = m.unsqueeze(1)
                sc[:, idx] = s.unsqueeze(1)
            return mn, sc
        mn = vm["min_val"].to(device=device, dtype=torch.float16)
        sc = vm["quant_scale"].to(device=device, dtype=torch.float16)
        if vm.get("axis", "") == "token_perhead" and mn.dim() == 2:
            return mn.reshape(rows, H), sc.reshape(rows, H)
        if mn.dim() == 3 and mn.shape[0] == rows:
            return mn.reshape(rows, 1).expand(rows, H), sc.reshape(rows, 1).expand(rows, H)
        if mn.dim() == 2 and tuple(mn.shape) == (rows, H):
            return mn, sc
        raise ValueError(f"Unsupported token meta shapes: min={tuple(mn.shape)} axis={vm.get('axis', '')!r}")

    def dequantize(self, layer_id: int, quantized_data: torch.Tensor, quantization_params: dict,
                   **kwargs: Any) -> torch.Tensor:
        """uint8 [2, blocks, block_size, H, D] + metadata -> bf16
        (tilelang_quantizer.py:164-181, kv_hadamard_quant.py:1709-1750)."""
        if kwargs:
            self.update_params(**kwargs)
        q = quantized_data.contiguous()
        if q.dim() != 5 or q.shape[0] != 2 or q.dtype != torch.uint8:
            raise ValueError("expected uint8 symbols [2, num_blocks, block_size, num_heads, head_dim]")
        _, B, S, H, D = q.shape
        dev = q.device
        rows = B * S
        km = quantization_params["key_meta"]
        kmin = km["min_val"].to(device=dev, dtype=torch.float16)
        ksc = km["quant_scale"].to(device=dev, dtype=torch.float16)
        if kmin.dim() != 2 or kmin.shape[-1] != D:
            raise ValueError(f"key metadata must be [heads, head_dim], got {tuple(kmin.shape)}")
        vmin, vsc = self._value_tables(quantization_params["value_meta"], rows, H, dev)
        kmeta16 = torch.stack([kmin.reshape(H, D), ksc.reshape(H, D)]).contiguous()
        vmeta16 = torch.stack([vmin.reshape(rows, H), vsc.reshape(rows, H)]).contiguous()
        _, _, signs = self._device_tables(layer_id, H, D, dev)
        out = torch.empty((2, B, S, H, D), dtype=torch.bfloat16, device=dev)
        lib = _lib.load()
        with torch.cuda.device(dev):
            _lib.check(lib.kvmi_v3_decompress(q.data_ptr(), rows, H, D, signs.data_ptr(), kmeta16.data_ptr(),
                                              vmeta16.data_ptr(), out.data_ptr(), _stream_handle()),
                       "kvmi_v3_decompress")
        return out


# The reference's class name, for configurations and imports that use it.
TileLangFusedQuantizer = FusedHadamardQuantizer
