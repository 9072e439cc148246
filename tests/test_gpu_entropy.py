"""Entropy-coded profiles (codec_type "nvcomp" / "lc" / "rans") end to end on the GPU.

The codec stage is lossless, so the bar is exact: a profile with the rANS codec
decompresses to exactly what the same profile with the bitpack codec (at the same
symbol width) decompresses to, which the bitpack tests pin to the oracle; each
chunk stream is byte-equal to the C oracle's rANS of that bitpack body; the fused
path and the operator loop write the same bytes."""

import copy

import numpy as np
import pytest
import torch

from kvserve_amd.compression import (CompressionConfig, CompressionManager, KVCompressionAdapter, KVServeCodec,
                                     KVServeQuantizer, KVServeTransformer)
from oracle import crans

pytestmark = pytest.mark.gpu

# configs/compression/original_top_nvcomp.json (the reference's shipped profile)
NVCOMP = {"enabled": True, "pipeline": ["transformer", "quantizer", "codec"],
          "transformer_config": {"transform_type": "hadamard", "seed": 3237919422},
          "quantizer_config": {"model_name": "Llama-3.1-8B-Instruct", "hybrid_ratio": 0.9,
                               "high_key_max_value": 6, "high_value_max_value": 6,
                               "low_key_max_value": 6, "low_value_max_value": 4,
                               "axis_key": "channel", "axis_value": "token", "split_type": "head"},
          "codec_config": {"codec_type": "nvcomp", "nvcomp_algorithm": "ANS", "data_type": "|u1"},
          "min_compress_size": 1024}


def _with_codec(cfg, cc):
    c = copy.deepcopy(cfg)
    c["codec_config"] = cc
    return c


def _kv(cuda, L, B, seed, H=8, D=128):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((L, 2, B, 16, H, D), generator=g)
    x[:, 0, :, :, :, 5] *= 6.0
    return x.to(torch.bfloat16).to(cuda)


def _streams(packet):
    return packet.chunks if packet.is_chunked else [packet.compressed_tensor]


def _metas(packet):
    return packet.chunk_metadata if packet.is_chunked else [packet.metadata]


def test_nvcomp_profile_is_lossless_over_the_bitpack_symbols(cuda):
    x = _kv(cuda, 6, 24, 1)
    ent = KVCompressionAdapter(NVCOMP, num_kv_heads=8, head_size=128)
    bp = KVCompressionAdapter(_with_codec(NVCOMP, {"codec_type": "bitpack", "bitpack_bits": 3}), 8, 128)
    pe, pb = ent.compress(x, "e"), bp.compress(x, "b")
    (se,), (sb,) = _streams(pe), _streams(pb)
    n = 6 * 2 * 8 * 24 * 16 * 128
    assert _metas(pe)[0]["codec_symbol_bits"] == 3
    ref = crans.encode_packed(sb[16:].cpu().numpy(), n, 3)
    assert np.array_equal(se.cpu().numpy(), ref)
    assert torch.equal(ent.decompress(pe), bp.decompress(pb))
    assert se.numel() < sb.numel() * 0.8                 # entropy coding beats 3-bit packing here
    for k in ("quantization_params", "codec_shape", "codec_layout"):
        assert str(_metas(pe)[0][k]) == str(_metas(pb)[0][k])


def test_lc_and_rans_profiles_write_the_same_stream(cuda):
    x = _kv(cuda, 3, 10, 2)
    streams = []
    for cc in ({"codec_type": "lc", "lc_algorithm": "TUPL8_1 BIT_8 RZE_2"}, {"codec_type": "rans"}, {}):
        ad = KVCompressionAdapter(_with_codec(NVCOMP, cc), 8, 128)
        p = ad.compress(x, "r")
        streams.append(_streams(p)[0])
        assert torch.equal(ad.decompress(p), KVCompressionAdapter(NVCOMP, 8, 128).decompress(p))
    assert torch.equal(streams[0], streams[1]) and torch.equal(streams[1], streams[2])


def test_fused_path_equals_operator_loop(cuda):
    """The operator loop (transformer -> quantizer -> KVServeCodec per the reference's
    manager) and the fused pipeline write the same chunk stream and decode to the
    same KV."""
    x = _kv(cuda, 4, 12, 3)
    fused = KVCompressionAdapter(NVCOMP, 8, 128)
    cfg = fused._config
    loop = CompressionManager(cfg, KVServeTransformer, KVServeQuantizer, KVServeCodec)
    meta = {"original_dtype": "bfloat16", "original_shape": list(x.shape)}
    pl = loop.compress_all_layers(x, "l", cfg, dict(meta))
    pf = fused.compress(x, "f")
    assert torch.equal(_streams(pl)[0], _streams(pf)[0])
    assert _metas(pl)[0]["codec_symbol_bits"] == _metas(pf)[0]["codec_symbol_bits"] == 3
    assert torch.equal(loop.decompress_all_layers(pf, cfg), fused.decompress(pl).view(4, 2, 12, 16, 8, 128))


def test_reference_default_profile(cuda):
    """"default" = the reference default (nvCOMP ANS codec, levels 12/8/6/4, no
    transform): symbols at 4 bits, entropy-coded."""
    x = _kv(cuda, 4, 16, 4)
    d = KVCompressionAdapter("default", 8, 128)
    qc = {k: v for k, v in d._config.quantizer_config.items() if k not in ("tp_rank", "tensor_parallel_size")}
    bp = KVCompressionAdapter({"enabled": True, "pipeline": ["quantizer", "codec"], "quantizer_config": qc,
                               "codec_config": {"codec_type": "bitpack", "bitpack_bits": 4},
                               "min_compress_size": 1024}, 8, 128)
    pd, pb = d.compress(x, "d"), bp.compress(x, "b")
    assert _metas(pd)[0]["codec_symbol_bits"] == 4
    assert torch.equal(d.decompress(pd), bp.decompress(pb))
    assert np.array_equal(_streams(pd)[0].cpu().numpy(),
                          crans.encode_packed(_streams(pb)[0][16:].cpu().numpy(), 4 * 2 * 8 * 16 * 16 * 128, 4))


def test_codec_only_pipeline_is_lossless_on_raw_bf16(cuda):
    x = _kv(cuda, 2, 8, 5)
    ad = KVCompressionAdapter({"enabled": True, "pipeline": ["codec"], "codec_config": {"codec_type": "nvcomp"}},
                              8, 128)
    p = ad.compress(x, "c")
    assert _metas(p)[0]["codec_symbol_bits"] == 8
    assert torch.equal(ad.decompress(p), x)
    # the codec stage sees the codec buffer in the permuted layout [l, 2, H, B, S, D]
    raw = x.permute(0, 1, 4, 2, 3, 5).contiguous().reshape(-1).view(torch.uint8).cpu().numpy()
    assert np.array_equal(_streams(p)[0].cpu().numpy(), crans.encode_packed(raw, raw.size, 8))


def test_paged_and_chunked_requests(cuda):
    """Paged compress / decompress (the connector's path) with the entropy codec,
    and a request over 500 MiB sent as 8-layer chunks, each its own rANS stream."""
    L, P, B = 10, 1100, 1040
    g = torch.Generator().manual_seed(6)
    pools = [torch.randn((2, P, 16, 8, 128), generator=g).to(torch.bfloat16).to(cuda) for _ in range(L)]
    ids = torch.randperm(P, generator=g)[:B].tolist()
    ad = KVCompressionAdapter(NVCOMP, 8, 128)
    pk = ad.compress_paged(pools, ids, "p")
    assert pk.is_chunked and len(pk.chunks) == 2
    stacked = torch.stack([p[:, torch.tensor(ids, device=cuda)] for p in pools])
    ps = ad.compress(stacked, "s")
    for a, b in zip(pk.chunks, ps.chunks):
        assert torch.equal(a, b)
    dst = [torch.zeros_like(p) for p in pools]
    ad.decompress_paged(pk, dst, ids)
    out = ad.decompress(ps)
    idx = torch.tensor(ids, device=cuda)
    for l in range(L):
        assert torch.equal(dst[l][:, idx], out[l])
    del pools, dst, stacked


def test_wire_round_trip_and_damage(cuda):
    from kvserve_amd.compression import build_wire, restore_from_wire

    x = _kv(cuda, 3, 12, 7)
    ad = KVCompressionAdapter(NVCOMP, 8, 128)
    p = ad.compress(x, "w")
    w = build_wire(p, 4096)
    assert torch.equal(ad.decompress(restore_from_wire(w)), ad.decompress(p))
    nblk = -(-3 * 2 * 8 * 12 * 16 * 128 // 65536)
    bad = p.compressed_tensor.clone()
    bad[32 + 8 * nblk + 4 + 2] ^= 0x5A                   # a frequency of block 0
    p.compressed_tensor = bad
    assert ad.decompress(p) is None                      # the manager reports and returns None
