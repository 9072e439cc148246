"""Write golden vectors of the reference's min-max quantizer and codec layout.

Run in the build container only (the reference tree is absent on GPU boxes):

    python tests/golden/make_golden.py /root/reference

Nothing pins the bf16 op order of KVServe's quantizer (on every quantization axis)
except the reference code itself (no golden data ships with it), so this script
imports the reference's own pure-torch modules -- quantizer_func.py, split_func.py, kvserve_quantizer.py and
compression_manager.py -- and records inputs and outputs as small .npz fixtures.
The transform (hadamard_func.py) is not imported: it needs the absent third-party
fast_hadamard_transform, and the FWHT is pinned by the Sylvester closed form
instead.  The sign fixture is written with torch's CPU generator following the
recipe of hadamard_func.py:137-152, to catch RNG drift between torch versions.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16)


def kv(gen, shape, outliers=True):
    x = torch.randn(shape, generator=gen)
    if outliers and len(shape) >= 2:
        # a few large channels, as KV caches have
        x[..., :3] *= 10
    return x.to(torch.bfloat16)


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from kvserve_v1.compression.quantizer import quantizer_func as qf
    from kvserve_v1.compression.quantizer.kvserve_quantizer import KVServeQuantizer
    from kvserve_v1.compression.compression_manager import CompressionConfig, CompressionManager

    gen = torch.Generator().manual_seed(20261201)

    # (a) quantizer_func.quantize / dequantize: one section
    cases = {}
    for i, (shape, axis, mv) in enumerate([((3, 16, 2, 128), "channel", 16), ((3, 16, 2, 128), "token", 16),
                                            ((2, 16, 3, 64), "channel", 6), ((2, 16, 3, 64), "token", 12),
                                            ((1, 16, 1, 128), "token", 4), ((2, 16, 6, 128), "channel", 200)]):
        x = kv(gen, shape)
        if i == 4:
            x[0, 5] = x[0, 5, 0, 0]  # a constant token: scale falls to the 1e-5 floor
        q, meta = qf.quantize(mv, x, axis)
        d = qf.dequantize(q, meta)
        cases[f"c{i}_x"] = bits(x)
        cases[f"c{i}_q"] = q.numpy()
        cases[f"c{i}_min"] = bits(meta["min_val"])
        cases[f"c{i}_scale"] = bits(meta["quant_scale"])
        cases[f"c{i}_deq"] = bits(d)
        cases[f"c{i}_cfg"] = np.array([mv, {"channel": 0, "token": 1}[axis]])
    np.savez_compressed(OUT / "quantizer_func.npz", **cases)

    # (b) KVServeQuantizer on whole layers: head split (Llama-3.1-8B mask) and layer split
    layers = {}
    cfgs = [dict(model_name="Llama-3.1-8B-Instruct", hybrid_ratio=0.3, high_key_max_value=16,
                 high_value_max_value=16, low_key_max_value=16, low_value_max_value=16, split_type="head"),
            dict(model_name="Llama-3.1-8B-Instruct", hybrid_ratio=0.8, high_key_max_value=12,
                 high_value_max_value=8, low_key_max_value=6, low_value_max_value=4, split_type="head"),
            dict(model_name="Llama-3.1-8B-Instruct", high_key_max_value=12, high_value_max_value=12,
                 low_key_max_value=6, low_value_max_value=6, split_type="layer")]
    for ci, cfg in enumerate(cfgs):
        quant = KVServeQuantizer(**cfg)
        for layer_id in (0, 31):
            x = kv(gen, (2, 1, 16, 8, 128))
            q, meta = quant.quantize(layer_id, x)
            d = quant.dequantize(layer_id, q, meta)
            key = f"q{ci}_l{layer_id}"
            layers[key + "_x"] = bits(x)
            layers[key + "_q"] = q.numpy()
            layers[key + "_deq"] = bits(d)
            for sec in ("high_key_meta", "high_value_meta", "low_key_meta", "low_value_meta"):
                m = meta[sec]
                if m["min_val"] is not None:
                    layers[f"{key}_{sec}_min"] = bits(m["min_val"])
                    layers[f"{key}_{sec}_scale"] = bits(m["quant_scale"])
    np.savez_compressed(OUT / "kvserve_quantizer.npz", **layers)

    # (c) CompressionManager without codec: permuted / native codec-buffer layout
    mgr_out = {}
    for layout in ("permuted", "native"):
        os.environ["KVSERVE_CODEC_LAYOUT"] = layout
        qc = dict(cfgs[1])
        cfg = CompressionConfig(enabled=True, pipeline=["quantizer"], quantizer_config=qc, min_compress_size=0)
        mgr = CompressionManager(cfg, quantizer=KVServeQuantizer)
        x = kv(gen, (2, 2, 1, 16, 8, 128))
        packet = mgr.compress_all_layers(x, "golden", cfg, {})
        mgr_out[f"{layout}_x"] = bits(x)
        mgr_out[f"{layout}_bytes"] = packet.compressed_tensor.numpy()
        mgr_out[f"{layout}_codec_shape"] = np.array(packet.metadata["codec_shape"])
        restored = mgr.decompress_all_layers(packet, cfg)
        mgr_out[f"{layout}_restored"] = bits(restored)
    os.environ.pop("KVSERVE_CODEC_LAYOUT", None)
    np.savez_compressed(OUT / "compression_manager.npz", **mgr_out)

    # (d) Rademacher signs (torch CPU generator recipe)
    sg = {}
    g = torch.Generator(device="cpu")
    for seed, layer, H, D in [(0xC0FEBABE, 0, 8, 128), (0xC0FEBABE, 31, 8, 128), (0x3333, 7, 4, 64),
                              (123, 79, 8, 128)]:
        rows = []
        for h in range(H):
            g.manual_seed(seed ^ (layer << 16) ^ h)
            rows.append(torch.randint(0, 2, (D,), generator=g, dtype=torch.int8).numpy())
        sg[f"s_{seed}_{layer}_{H}_{D}"] = np.stack(rows)
    np.savez_compressed(OUT / "signs.npz", **sg)

    # (e) quantization axes (quantizer_func.py:41-49, kvserve_quantizer.py:202-214): the
    # tensor axis of quantizer_func, and KVServeQuantizer with every non-default
    # (axis_key, axis_value) pair.  A generator of its own, so (a)-(d) stay as they were.
    gen = torch.Generator().manual_seed(20261202)
    ax = {}
    for i, (shape, mv) in enumerate([((3, 16, 2, 128), 16), ((2, 16, 3, 64), 6), ((1, 16, 1, 128), 200)]):
        x = kv(gen, shape)
        if i == 1:
            x[:] = x[0, 0, 0, 0]  # a constant section: the scale falls to the 1e-5 floor
        q, meta = qf.quantize(mv, x, "tensor")
        ax[f"t{i}_x"] = bits(x)
        ax[f"t{i}_q"] = q.numpy()
        ax[f"t{i}_min"] = bits(meta["min_val"])
        ax[f"t{i}_scale"] = bits(meta["quant_scale"])
        ax[f"t{i}_deq"] = bits(qf.dequantize(q, meta))
        ax[f"t{i}_mv"] = np.array([mv])
    pairs = [(a, b) for a in ("channel", "token", "tensor") for b in ("channel", "token", "tensor")
             if (a, b) != ("channel", "token")]
    for pi, (ak, av) in enumerate(pairs):
        # head split (two sections) on layer 0, layer split (the low layer 31)
        for ci, layer_id in ((1, 0), (2, 31)):
            quant = KVServeQuantizer(**cfgs[ci], axis_key=ak, axis_value=av)
            x = kv(gen, (2, 1, 8, 8, 64))
            q, meta = quant.quantize(layer_id, x)
            d = quant.dequantize(layer_id, q, meta)
            key = f"a{pi}_q{ci}_l{layer_id}"
            ax[key + "_x"] = bits(x)
            ax[key + "_q"] = q.numpy()
            ax[key + "_deq"] = bits(d)
            for sec in ("high_key_meta", "high_value_meta", "low_key_meta", "low_value_meta"):
                m = meta[sec]
                if m["min_val"] is not None:
                    ax[f"{key}_{sec}_min"] = bits(m["min_val"])
                    ax[f"{key}_{sec}_scale"] = bits(m["quant_scale"])
        ax[f"a{pi}_axes"] = np.array([["channel", "token", "tensor"].index(a) for a in (ak, av)])
    np.savez_compressed(OUT / "quantizer_axes.npz", **ax)
    for p in sorted(OUT.glob("*.npz")):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
