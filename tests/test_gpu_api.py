"""GPU tests of the drop-in surface (kvserve_amd.compression), modelled on the
reference's tests/test_bitpack_codec.py and tests/test_pluggable_operators.py."""

import threading
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import cbitpack
from oracle import kvpipe as kp

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"

PROFILE = {
    "enabled": True,
    "pipeline": ["transformer", "quantizer", "codec"],
    "transformer_config": {"transform_type": "hadamard", "seed": 3237919422},
    "quantizer_config": {"model_name": "Llama-3.1-8B-Instruct", "hybrid_ratio": 0.3, "high_key_max_value": 16,
                         "high_value_max_value": 16, "low_key_max_value": 16, "low_value_max_value": 16,
                         "axis_key": "channel", "axis_value": "token", "split_type": "head"},
    "codec_config": {"codec_type": "bitpack", "bitpack_bits": 4},
    "min_compress_size": 1024,
}


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def kv(gen, shape):
    x = torch.randn(shape, generator=gen)
    x[..., :3] *= 10
    return x.to(torch.bfloat16)


def test_quantizer_operator_matches_reference_golden(cuda):
    """The gfx950 KVServeQuantizer against vectors written by the reference's own
    KVServeQuantizer (tests/golden/make_golden.py)."""
    from kvserve_amd.compression import KVServeQuantizer

    z = np.load(GOLDEN / "kvserve_quantizer.npz")
    cfgs = [dict(hybrid_ratio=0.3, high_key_max_value=16, high_value_max_value=16, low_key_max_value=16,
                 low_value_max_value=16, split_type="head"),
            dict(hybrid_ratio=0.8, high_key_max_value=12, high_value_max_value=8, low_key_max_value=6,
                 low_value_max_value=4, split_type="head"),
            dict(high_key_max_value=12, high_value_max_value=12, low_key_max_value=6, low_value_max_value=6,
                 split_type="layer")]
    for ci, cfg in enumerate(cfgs):
        q = KVServeQuantizer(model_name="Llama-3.1-8B-Instruct", **cfg)
        for layer in (0, 31):
            key = f"q{ci}_l{layer}"
            x = torch.from_numpy(z[key + "_x"].view(np.int16)).view(torch.bfloat16).to(cuda)
            sym, meta = q.quantize(layer, x)
            assert np.array_equal(sym.cpu().numpy(), z[key + "_q"]), key
            for sec in ("high_key_meta", "high_value_meta", "low_key_meta", "low_value_meta"):
                k = f"{key}_{sec}_min"
                if k in z.files:
                    assert np.array_equal(bits(meta[sec]["min_val"]).reshape(-1), z[k].reshape(-1)), (key, sec)
                    assert np.array_equal(bits(meta[sec]["quant_scale"]).reshape(-1),
                                          z[f"{key}_{sec}_scale"].reshape(-1)), (key, sec)
                    assert tuple(meta[sec]["min_val"].shape) == tuple(z[k].shape)
                else:
                    assert meta[sec]["min_val"] is None
            deq = q.dequantize(layer, sym, meta)
            assert np.array_equal(bits(deq), z[key + "_deq"]), key


@pytest.mark.parametrize("layout", ["permuted", "native"])
def test_manager_without_codec_matches_reference_golden(cuda, monkeypatch, layout):
    from kvserve_amd.compression import KVCompressionAdapter

    monkeypatch.setenv("KVSERVE_CODEC_LAYOUT", layout)
    z = np.load(GOLDEN / "compression_manager.npz")
    cfg = {"pipeline": ["quantizer"], "min_compress_size": 0,
           "quantizer_config": {"model_name": "Llama-3.1-8B-Instruct", "hybrid_ratio": 0.8,
                                "high_key_max_value": 12, "high_value_max_value": 8, "low_key_max_value": 6,
                                "low_value_max_value": 4}}
    ad = KVCompressionAdapter(cfg, num_kv_heads=8, head_size=128)
    x = torch.from_numpy(z[f"{layout}_x"].view(np.int16)).view(torch.bfloat16).to(cuda)
    packet = ad.compress(x, "golden")
    assert packet is not None and not packet.is_chunked
    assert packet.metadata["codec_shape"] == list(z[f"{layout}_codec_shape"])
    assert np.array_equal(packet.compressed_tensor.cpu().numpy(), z[f"{layout}_bytes"])
    assert np.array_equal(bits(ad.decompress(packet)), z[f"{layout}_restored"].reshape(bits(x).shape))


def _oracle_profiles(prof):
    return [kp.LayerProfile(kp.PartProfile(p.k_order, p.k_levels, p.k_groups()),
                            kp.PartProfile(p.v_order, p.v_levels, p.v_group)) for p in prof]


def test_adapter_full_profile_matches_oracle_and_paged_equals_stacked(cuda):
    from kvserve_amd.compression import KVCompressionAdapter

    g = torch.Generator().manual_seed(5)
    L, B, S, H, D = 3, 6, 16, 8, 128
    x = kv(g, (L, 2, B, S, H, D)).to(cuda)
    ad = KVCompressionAdapter(PROFILE, num_kv_heads=H, head_size=D)
    packet = ad.compress(x, "req")
    assert packet is not None and packet.metadata["codec_applied"] and packet.metadata["transformer_applied"]
    assert packet.compressed_tensor.numel() == 16 + (L * 2 * B * S * H * D * 4) // 8
    # the stream against the oracle of the same profile
    prof = ad._manager.profiles(range(L), H)
    ref = kp.compress_request([bits(x[l]) for l in range(L)], list(range(B)), _oracle_profiles(prof),
                              3237919422, 4)[0]
    sym = cbitpack.decode(packet.compressed_tensor.cpu().numpy(), ref.symbols.size, 4)
    d = np.abs(sym.astype(np.int16) - ref.symbols.reshape(-1).astype(np.int16))
    assert d.max() <= 1 and np.count_nonzero(d) <= 1e-4 * d.size
    out = ad.decompress(packet)
    assert out.shape == x.shape and out.dtype == x.dtype
    ref_pools = [np.zeros_like(bits(x[l])) for l in range(L)]
    kp.decompress_request([ref], ref_pools, list(range(B)), _oracle_profiles(prof), 3237919422, 4)
    for l in range(L):
        for p in range(2):
            a, r = kp.bf16_to_f32(bits(out[l, p])), kp.bf16_to_f32(ref_pools[l][p])
            assert np.abs(a - r).max() / np.abs(r).max() <= 1e-2
    # paged entry points on scattered blocks give the same stream and restore the same KV
    P = 40
    perm = torch.randperm(P, generator=g)[:B]
    caches = [torch.zeros((2, P, S, H, D), dtype=torch.bfloat16, device=cuda) for _ in range(L)]
    for l in range(L):
        caches[l][:, perm.to(cuda)] = x[l]
    paged = ad.compress_paged(caches, perm.tolist(), "req")
    assert torch.equal(paged.compressed_tensor, packet.compressed_tensor)
    dst = [torch.full_like(c, 3.0) for c in caches]
    ad.decompress_paged(paged, dst, perm.tolist())
    for l in range(L):
        assert torch.equal(dst[l][:, perm.to(cuda)], out[l])
        untouched = torch.ones(P, dtype=torch.bool)
        untouched[perm] = False
        assert bool((dst[l][:, untouched.to(cuda)] == 3.0).all())


def test_operator_loop_equals_fused(cuda):
    """The operator-by-operator CompressionManager and the fused manager agree."""
    from kvserve_amd.compression import (CompressionConfig, CompressionManager, FusedCompressionManager,
                                         KVServeCodec, KVServeQuantizer, KVServeTransformer)

    g = torch.Generator().manual_seed(8)
    x = kv(g, (2, 2, 3, 16, 8, 128)).to(cuda)
    cfg = CompressionConfig(enabled=True, pipeline=PROFILE["pipeline"], transformer_config=PROFILE["transformer_config"],
                            quantizer_config=PROFILE["quantizer_config"], codec_config=PROFILE["codec_config"])
    loop = CompressionManager(cfg, KVServeTransformer, KVServeQuantizer, KVServeCodec)
    fused = FusedCompressionManager(cfg, KVServeTransformer, KVServeQuantizer, KVServeCodec)
    a = loop.compress_all_layers(x, "a", cfg, {})
    b = fused.compress_all_layers(x, "b", cfg, {})
    assert torch.equal(a.compressed_tensor, b.compressed_tensor)
    assert a.metadata["codec_shape"] == b.metadata["codec_shape"]
    for qa, qb in zip(a.metadata["quantization_params"], b.metadata["quantization_params"]):
        for sec in ("high_key_meta", "high_value_meta", "low_key_meta", "low_value_meta"):
            if qa[sec]["min_val"] is None:
                assert qb[sec]["min_val"] is None
            else:
                assert torch.equal(qa[sec]["min_val"], qb[sec]["min_val"])
                assert torch.equal(qa[sec]["quant_scale"], qb[sec]["quant_scale"])
    # each decodes the other's packet
    assert torch.equal(loop.decompress_all_layers(b, cfg), fused.decompress_all_layers(a, cfg))


def test_codec_only_and_quant_only_pipelines(cuda):
    """test_bitpack_codec.py:87-120 analogues: codec-only manager round trip, and
    quantizer+bitpack equals quantizer only."""
    from kvserve_amd.compression import (CompressionConfig, CompressionManager, KVCompressionAdapter,
                                         KVServeCodec)

    cfg = CompressionConfig(enabled=True, pipeline=["codec"], codec_config={"codec_type": "bitpack",
                                                                            "bitpack_bits": 4})
    mgr = CompressionManager(cfg, codec=KVServeCodec)
    xu = torch.randint(16, (2, 2, 3, 16, 2, 128), device=cuda, dtype=torch.uint8)
    packet = mgr.compress_all_layers(xu, "bitpack", cfg, {})
    assert packet is not None and packet.metadata["codec_applied"]
    assert torch.equal(mgr.decompress_all_layers(packet, cfg), xu)

    config = {"pipeline": ["quantizer", "codec"],
              "quantizer_config": {"model_name": "Qwen2.5-7B-Instruct", "high_key_max_value": 12,
                                   "high_value_max_value": 8, "low_key_max_value": 6, "low_value_max_value": 4},
              "codec_config": {"codec_type": "bitpack", "bitpack_bits": 4}}
    packed = KVCompressionAdapter(config, num_kv_heads=4, head_size=128)
    reference = KVCompressionAdapter({**config, "pipeline": ["quantizer"]}, num_kv_heads=4, head_size=128)
    x = torch.randn(2, 2, 3, 16, 4, 128, device=cuda, dtype=torch.bfloat16)
    pk = packed.compress(x, "quant-bitpack")
    assert pk is not None and pk.metadata["codec_applied"]
    assert torch.equal(packed.decompress(pk), reference.decompress(reference.compress(x, "quant-only")))


def test_chunked_request_over_500_mib(cuda):
    """test_pluggable_operators.py:166-193: > 500 MiB splits into 8-layer chunks whose
    layer ids continue across chunks."""
    from kvserve_amd.compression import KVCompressionAdapter

    ad = KVCompressionAdapter({**PROFILE, "quantizer_config": {**PROFILE["quantizer_config"],
                                                                 "model_name": "Qwen2.5-7B-Instruct"}},
                              num_kv_heads=4, head_size=128)
    g = torch.Generator(device=cuda).manual_seed(3)
    x = torch.randn((9, 2, 256, 128, 4, 128), generator=g, device=cuda).to(torch.bfloat16)
    packet = ad.compress(x, "chunked")
    assert packet is not None and packet.is_chunked and len(packet.chunks) == 2
    assert [m["start_layer_id"] for m in packet.chunk_metadata] == [0, 8]
    out = ad.decompress(packet)
    assert out.shape == x.shape
    rel = ((out.float() - x.float()).square().sum() / x.float().square().sum()).item()
    assert rel < 0.06
    # layer 8 of the chunked stream equals layer 8 compressed on its own with layer id 8
    single = ad.compress_paged([x[8]], list(range(256)), "one", layer_ids=[8])
    assert torch.equal(single.compressed_tensor[16:], packet.chunks[1][16:])


def test_streams_threads_and_graph_capture(cuda):
    """test_bitpack_codec.py:30-67 / test_pluggable_operators.py:132-163 analogues:
    side streams, concurrent threads with per-call widths, and HIP-graph replay."""
    from kvserve_amd.compression import BitPackCodec
    from kvserve_amd.engine import FusedKVCodec
    from kvserve_amd.workloads import make_config1

    codec = BitPackCodec()

    def roundtrip(b):
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            x = torch.randint(2 ** b, (127,), device=cuda, dtype=torch.uint8)
            p = codec.encode(x, bitpack_bits=b)
            r = codec.decode(p, "uint8", [127], "cuda", bitpack_bits=b)
        st.synchronize()
        return x, r

    with ThreadPoolExecutor(max_workers=3) as pool:
        assert all(torch.equal(a, b) for a, b in pool.map(roundtrip, [2, 4, 7]))
    assert codec.bitpack_bits == 8

    wl = make_config1(device=cuda)
    req = wl.requests[0]
    fc = FusedKVCodec(8, 128, 16, 4, wl.seed)
    plan = fc.plan_compress(req.pools, req.block_ids, req.profiles)
    plan.run()
    torch.cuda.synchronize()
    eager = [s.clone() for s in plan.packet.streams]
    km = plan.packet.kmeta.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        for s in plan.packet.streams:
            s.zero_()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=st):
            plan.run()
    for _ in range(3):
        for s in plan.packet.streams:
            s.zero_()
        plan.packet.kmeta.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(eager, plan.packet.streams))
        assert torch.equal(km, plan.packet.kmeta)
    plan.check_errors()

    # the decompress plan (the K-table decode at D = 128, 4 bits) replayed into cleared caches
    dplan = fc.plan_decompress(plan.packet, req.pools, req.block_ids)
    dplan.run()
    torch.cuda.synchronize()
    ids = req.block_ids.long()
    want = [p[:, ids].clone() for p in req.pools]
    dgraph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        torch.cuda.synchronize()
        with torch.cuda.graph(dgraph, stream=st):
            dplan.run()
    for _ in range(3):
        for p in req.pools:
            p[:, ids] = 0
        torch.cuda.synchronize()
        dgraph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(p[:, ids].view(torch.int16), w.view(torch.int16)) for p, w in zip(req.pools, want))
    dplan.check_errors()
