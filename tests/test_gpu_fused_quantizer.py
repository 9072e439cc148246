"""impl "tilelang_fused" on the GPU (kvmi_v3_* through the C-ABI) against the oracle of
the compress_v3 / decompress_v3 arithmetic (oracle/fused_v3.py).

The transform is the reference's fp32 butterfly in the same order, and the kernels use
the same fp32 operations (correctly rounded division, roundf, no contraction), so the
fp32 statistics (K per channel, V per row and group), the symbols and the dequantized
layer (computed from the same symbols and float16 metadata) are all compared bit for
bit.
"""

import numpy as np
import pytest
import torch

from oracle import fused_v3 as fv
from oracle import kvpipe as kp

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def _layer(seed, B, S, H, D, outliers=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((2, B, S, H, D), generator=g)
    if outliers:
        ch = torch.randint(0, D, (H, 4), generator=g)
        for h in range(H):
            x[0, :, :, h, ch[h]] *= 10.0
    return x.to(torch.bfloat16)


CASES = [
    # B, S, H, D, model (None: uniform levels), layer
    (4, 16, 8, 128, "Llama-3.1-8B-Instruct", 0),
    (3, 16, 4, 64, None, 5),
    (2, 7, 1, 128, None, 2),
    (1, 5, 16, 128, None, 1),
    (256, 16, 8, 128, "Llama-3.1-8B-Instruct", 17),   # 4096 rows: many passes per workgroup
    (9, 16, 2, 64, "Llama-3.1-8B-Instruct", 3),
    (3, 16, 64, 128, None, 0),   # most heads: 64 KiB of LDS keys in the K statistics
    (5, 3, 32, 64, None, 4),     # ragged block size, last pass partly past the layer
]


@pytest.mark.parametrize("B,S,H,D,model,layer", CASES)
def test_fused_quantizer_matches_oracle(cuda, B, S, H, D, model, layer):
    from kvserve_amd.compression.quantizer import FusedHadamardQuantizer
    from kvserve_amd.profiles import rademacher_sign_bits  # noqa: F401  (signs recipe shared with the oracle)

    print(f"case B={B} S={S} H={H} D={D} model={model} layer={layer}", flush=True)
    kw = {"base_seed": 0xC0FEBABE, "hybrid_ratio": 0.8}
    if model:
        kw["model_name"] = model
        if H != 8:
            kw.update(tensor_parallel_size=8 // H, tp_rank=min(1, 8 // H - 1))
    q = FusedHadamardQuantizer(**kw)
    x = _layer(B * 131 + H * 7 + D, B, S, H, D)
    sym, meta = q.quantize(layer, x.to(cuda))
    torch.cuda.synchronize()
    k_lv, v_lv = q.levels(layer, H)
    signs = kp.rademacher_signs(0xC0FEBABE, layer, H, D)
    R = B * S
    xb = _bits(x).reshape(2, R, H, D)
    ref_q, ref_m = fv.compress_layer(xb, signs, k_lv, v_lv)
    # fp16 metadata = the oracle's fp32 statistics rounded once (tilelang_quantizer.py:23-53)
    km, vm = meta["key_meta"], meta["value_meta"]
    assert km["axis"] == "channel" and vm["axis"] == "token_perhead"
    assert np.array_equal(km["min_val"].cpu().numpy(), ref_m["kmin"].astype(np.float16))
    assert np.array_equal(km["quant_scale"].cpu().numpy(), ref_m["kscale"].astype(np.float16))
    assert np.array_equal(vm["min_val"].cpu().numpy(), ref_m["vmin"].astype(np.float16))
    assert np.array_equal(vm["quant_scale"].cpu().numpy(), ref_m["vscale"].astype(np.float16))
    got = sym.cpu().numpy().reshape(2, R, H, D)
    d = np.abs(got.astype(np.int16) - ref_q.astype(np.int16))
    print(f"symbols differing from the oracle: {np.count_nonzero(d)} of {d.size}", flush=True)
    assert np.array_equal(got, ref_q), (int(d.max()), int(np.count_nonzero(d)))
    # dequantize the GPU's own symbols: same inputs, same arithmetic
    out = q.dequantize(layer, sym, meta)
    torch.cuda.synchronize()
    ref_out = fv.decompress_layer(got, km["min_val"].cpu().numpy(), km["quant_scale"].cpu().numpy(),
                                  vm["min_val"].cpu().numpy(), vm["quant_scale"].cpu().numpy(), signs)
    assert np.array_equal(_bits(out).reshape(2, R, H, D), ref_out)


def test_fused_quantizer_out_buffer_contract(cuda):
    from kvserve_amd.compression.quantizer import TileLangFusedQuantizer

    q = TileLangFusedQuantizer()
    x = _layer(3, 2, 16, 8, 128).to(cuda)
    buf = torch.full((2, 2, 16, 8, 128), 255, dtype=torch.uint8, device=cuda)
    sym, meta = q.quantize(0, x, out=buf)
    assert sym.data_ptr() == buf.data_ptr()
    ref, _ = q.quantize(0, x)
    assert torch.equal(buf, ref)
    for bad, msg in ((torch.empty((2, 2, 16, 8, 64), dtype=torch.uint8, device=cuda), "shape"),
                     (torch.empty((2, 2, 16, 8, 128), dtype=torch.int8, device=cuda), "dtype"),
                     (torch.empty((2, 2, 16, 128, 8), dtype=torch.uint8, device=cuda).transpose(3, 4), "contiguous")):
        with pytest.raises(ValueError, match=msg):
            q.quantize(0, x, out=bad)


def test_adapter_tilelang_fused_roundtrip_through_wire(cuda):
    """The reference's configuration with impl "tilelang_fused" through the adapter,
    the bitpack codec and the wire bundle; the result equals the oracle's
    decompression of the same symbols and float16 metadata."""
    from kvserve_amd.compression import KVCompressionAdapter
    from kvserve_amd.compression.wire import build_wire, restore_from_wire

    cfg = {"pipeline": ["transformer", "quantizer", "codec"],
           "transformer_config": {"transform_type": "hadamard", "seed": 0xC0FEBABE},
           "quantizer_config": {"impl": "tilelang_fused", "model_name": "Llama-3.1-8B-Instruct",
                                "hybrid_ratio": 0.3, "high_key_max_value": 15, "high_value_max_value": 15,
                                "low_key_max_value": 12, "low_value_max_value": 12},
           "codec_config": {"codec_type": "bitpack", "bitpack_bits": 4}}
    enc = KVCompressionAdapter(cfg, num_kv_heads=8, head_size=128)
    dec = KVCompressionAdapter(cfg, num_kv_heads=8, head_size=128)
    L, B, S, H, D = 3, 5, 16, 8, 128
    x = torch.stack([_layer(40 + l, B, S, H, D) for l in range(L)]).to(cuda)
    packet = enc.compress(x, "tl-fused")
    assert packet is not None and packet.metadata["codec_applied"]
    restored = dec.decompress(restore_from_wire(build_wire(packet, max_chunk_bytes=1 << 16)))
    assert restored is not None and restored.shape == x.shape
    qz = enc._manager.quantizer
    for l in range(L):
        xl = _bits(x[l].cpu()).reshape(2, B * S, H, D)
        k_lv, v_lv = qz.levels(l, H)
        signs = kp.rademacher_signs(0xC0FEBABE, l, H, D)
        ref_q, ref_m = fv.compress_layer(xl, signs, k_lv, v_lv)
        ref = fv.decompress_layer(ref_q, ref_m["kmin"].astype(np.float16), ref_m["kscale"].astype(np.float16),
                                  ref_m["vmin"].astype(np.float16), ref_m["vscale"].astype(np.float16), signs)
        got, want = kp.bf16_to_f32(_bits(restored[l])).reshape(2, -1), kp.bf16_to_f32(ref).reshape(2, -1)
        for part in range(2):
            rel = np.abs(got[part] - want[part]).max() / np.abs(want[part]).max()
            assert rel <= 1e-2, (l, part, rel)


def test_fused_quantizer_empty_layer(cuda):
    """A layer with no blocks quantizes to empty symbols and metadata and back."""
    from kvserve_amd.compression.quantizer import FusedHadamardQuantizer

    q = FusedHadamardQuantizer(base_seed=0xC0FEBABE)
    x = torch.empty((2, 0, 16, 8, 128), dtype=torch.bfloat16, device=cuda)
    sym, meta = q.quantize(0, x)
    assert sym.shape == x.shape and sym.dtype == torch.uint8
    assert tuple(meta["key_meta"]["min_val"].shape) == (8, 128)
    assert not meta["key_meta"]["min_val"].any() and not meta["key_meta"]["quant_scale"].any()
    assert tuple(meta["value_meta"]["min_val"].shape) == (0, 8)
    out = q.dequantize(0, sym, meta)
    torch.cuda.synchronize()
    assert out.shape == x.shape and out.dtype == torch.bfloat16
