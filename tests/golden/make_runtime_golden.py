"""Write golden vectors of the reference's fixed-profile runtime (pipeline encode / decode).

Run in the build container only (the reference tree is absent on GPU boxes):

    python tests/golden/make_runtime_golden.py /root/reference

The reference's runtime tests pin the transform (bf16 op-order FWHT, Sylvester) and
the quantizer's symbols and aux, but nothing pins a whole chunk: the layout offsets,
head order, signs, raw tails and the decode side (dequantize, inverse transform,
signs, scatter).  This script imports the reference's pure-torch runtime modules
(config.py, layout.py, scores.py, manager.build_signs, pipeline.CompressionPipeline)
and drives their CPU path -- the codec stage is left out (nvCOMP is absent; the
runtime's codec is lossless and pinned on its own) -- recording inputs and outputs
as a small .npz fixture.  torch's CPU and GPU elementwise bf16 ops both compute in
fp32 and round to bf16 once per op, so these CPU vectors stand for the GPU path.
"""

from __future__ import annotations

import contextlib
import json
import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import torch

OUT = Path(__file__).resolve().parent

LEVELS = ("high_key_num_levels", "low_key_num_levels", "high_value_num_levels", "low_value_num_levels")

# name, compression extra config, layers, heads, head size (K, V), block size,
# blocks per logical, source / target logical blocks, valid tokens, scores
CASES = [
    ("default_tail", {}, 3, 2, (64, 64), 16, 1, [2, 0], [1, 3], 31, None),
    ("head_split", {"split_type": "head", "hybrid_ratio": 0.5}, 2, 4, (32, 32), 16, 2, [1, 2], [3, 0], 32,
     [[0.3, 0.9, 0.1, 0.5], [0.8, 0.2, 0.7, 0.05]]),
    ("tensor_axis", {"axis_key": "tensor", "axis_value": "tensor"}, 1, 2, (128, 128), 16, 1, [0], [2], 16, None),
    ("transform_only", {"pipeline": ["transformer"]}, 2, 2, (16, 16), 16, 1, [3, 1], [0, 2], 20, None),
    ("quant_only_256", {"pipeline": ["quantizer"], "axis_key": "token", **dict.fromkeys(LEVELS, 256)}, 3, 3, (8, 8),
     16, 4, [0, 2, 1], [3, 1, 2], 48, None),
    ("wide_head", {**dict.fromkeys(LEVELS, 16)}, 1, 1, (256, 256), 16, 1, [1], [0], 16, None),
    ("kv_sizes_differ", {}, 2, 2, (64, 32), 8, 1, [0, 1, 2], [3, 4, 5], 21, None),
    ("channel_both", {"axis_value": "channel", "logical_blocks_per_chunk": 3}, 2, 2, (32, 32), 16, 1, [0, 2], [1, 3],
     32, None),
]


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16)


def main(ref_root: str) -> None:
    sys.dont_write_bytecode = True
    sys.path.insert(0, ref_root)
    from kvserve_v1.compression.runtime import pipeline as ref_pipeline
    from kvserve_v1.compression.runtime.config import CompressionConfig
    from kvserve_v1.compression.runtime.layout import build_compression_layout
    from kvserve_v1.compression.runtime.manager import build_signs
    from kvserve_v1.compression.runtime.scores import build_head_selection
    from kvserve_v1.compression.runtime.spec import CacheSpec

    # the CPU path runs under `torch.cuda.stream(...)` and records slot events
    ref_pipeline.torch.cuda.stream = lambda stream: contextlib.nullcontext()
    fake_event = SimpleNamespace(record=lambda *a, **k: None)
    cpu = SimpleNamespace(device=torch.device("cpu"))

    out = {}
    gen = torch.Generator().manual_seed(20261202)
    for name, compression, layers, heads, (dk, dv), block_size, bpl, src, dst, tokens, scores in CASES:
        extra = {"compression": {"enable-compression-pipeline": True, "logical_blocks_per_chunk": len(src),
                                 **compression}}
        config = CompressionConfig.from_extra_config(extra)
        specs = {f"model.layers.{i}.self_attn": CacheSpec(i, block_size, heads, dk, torch.bfloat16, dv)
                 for i in range(layers)}
        planning = config
        if "quantizer" not in config.pipeline:
            from dataclasses import replace
            planning = replace(config, split_type="layer")
        score_array = np.asarray(scores, dtype=np.float32) if scores is not None else None
        selection = build_head_selection(specs, planning, 0, 1, score_array)
        layout = build_compression_layout(specs, planning, selection.low_counts, layers)
        kernel_tokens = block_size // bpl
        total_blocks = (max(src + dst) + 1) * bpl
        sources = {n: (torch.randn(total_blocks, heads, kernel_tokens, dk + dv, generator=gen) * 2).to(torch.bfloat16)
                   for n in specs}
        for n, c in sources.items():  # a few large channels, as KV caches have
            c[..., :2] *= 8
        targets = {n: torch.full_like(c, -9.0) for n, c in sources.items()}

        def make_pipeline(caches):
            orders, signs = {}, {}
            for part in layout.layer_parts:
                order = selection.local_orders[part.layer_index]
                orders[part.layer_name] = torch.tensor(order, dtype=torch.int64)
                if config.uses_transformer:
                    signs[(part.layer_name, part.kv_part)] = build_signs(part, order, config.seed)
            physical = config.logical_blocks_per_chunk * bpl
            slot = ref_pipeline.CompressionSlotBuffers(
                arena_a=torch.zeros(layout.arena_bytes, dtype=torch.uint8),
                arena_b=torch.zeros(layout.arena_bytes, dtype=torch.uint8),
                aux=torch.zeros(layout.aux_arena_bytes, dtype=torch.uint8),
                block_indices=torch.zeros(1, physical, dtype=torch.int64),
                completion_event=fake_event, host_indices=None,
                raw_tail=torch.zeros(layout.raw_tail_capacity, dtype=torch.uint8))
            p = ref_pipeline.CompressionPipeline(layout, "HND", bpl, [slot], None, cpu, signs, orders,
                                                 stages=tuple(s for s in config.pipeline if s != "codec"),
                                                 pipeline_backend="python")
            p.bind_kv_caches(caches, prepare_backend=False)
            p.identity_orders = {n for n, o in orders.items() if o.tolist() == list(range(o.numel()))}
            return p, slot

        producer, pslot = make_pipeline(sources)
        consumer, cslot = make_pipeline(targets)
        meta = {"compression": compression, "layers": layers, "heads": heads, "head_size": dk, "head_size_v": dv,
                "block_size": block_size, "blocks_per_logical": bpl, "src": src, "dst": dst, "tokens": tokens,
                "scores": scores, "total_blocks": total_blocks,
                "orders": {str(k): list(v) for k, v in selection.local_orders.items()},
                "layout": {"raw_bytes_by_part": layout.raw_bytes_by_part, "u8_bytes_by_part": layout.u8_bytes_by_part,
                           "aux_bytes_by_part": layout.aux_bytes_by_part, "arena_bytes": layout.arena_bytes,
                           "scratch_stride": layout.scratch_stride, "u8_base": layout.u8_base,
                           "aux_arena_bytes": layout.aux_arena_bytes, "raw_tail_capacity": layout.raw_tail_capacity,
                           "parts": [[p.layer_name, p.kv_part, p.u8_offset, p.raw_bytes,
                                      [[s.head_start, s.head_count, s.num_levels, s.axis, s.aux_min_offset,
                                        s.aux_scale_offset] for s in p.sections]] for p in layout.layer_parts]}}
        out[f"{name}_meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
        # only the chunk's physical blocks are kept: [len(ids) * blocks_per_logical, ...]
        src_phys = [b * bpl + i for b in src for i in range(bpl)]
        dst_phys = [b * bpl + i for b in dst for i in range(bpl)]
        for i, n in enumerate(specs):
            out[f"{name}_src{i}"] = bits(sources[n][src_phys])
        quantized = "quantizer" in config.pipeline
        for part in (0, 1):
            encoded = producer.encode(0, [src], part, valid_tokens_by_group={0: tokens})
            u8 = encoded.u8_bytes
            aux = layout.aux_bytes_by_part[part] if quantized and layout.has_body({0: tokens}) else 0
            out[f"{name}_p{part}_payload"] = pslot.arena_a[:u8].numpy().copy()
            out[f"{name}_p{part}_aux"] = pslot.aux[:aux].numpy().copy()
            out[f"{name}_p{part}_tail"] = pslot.raw_tail[:encoded.raw_tail_bytes].numpy().copy()
            cslot.arena_a[:u8].copy_(pslot.arena_a[:u8])
            cslot.aux[:aux].copy_(pslot.aux[:aux])
            cslot.raw_tail[:encoded.raw_tail_bytes].copy_(pslot.raw_tail[:encoded.raw_tail_bytes])
            consumer.decode(0, [dst], part, u8, u8, valid_tokens_by_group={0: tokens})
        for i, n in enumerate(specs):
            untouched = sorted(set(range(total_blocks)) - set(dst_phys))
            assert (targets[n][untouched] == -9).all()
            out[f"{name}_dst{i}"] = bits(targets[n][dst_phys])
        if config.uses_transformer:
            for part in layout.layer_parts:
                out[f"{name}_signs{part.layer_index}_{part.kv_part}"] = (
                    producer.signs[(part.layer_name, part.kv_part)].reshape(heads, -1).to(torch.int8).numpy())
    np.savez_compressed(OUT / "runtime.npz", **out)
    print("runtime.npz", (OUT / "runtime.npz").stat().st_size)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
