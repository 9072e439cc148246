"""Connector on the GPU: producer save -> loopback transport -> consumer load through
the fused paged kernels, against the reference's procedure run with the same
operators (extract each layer, stack in sorted-name order, compress the stack,
decompress, inject; compressed_kv_connector.py:377-497, :235-371).  The stacked path
is itself pinned to the oracle by the adapter tests, so equality here carries the
parity over; bars are bit-exact (same symbols, same metadata, same bytes written)."""

from types import SimpleNamespace

import pytest
import torch

from kvserve_amd.compression import KVCompressionAdapter
from kvserve_amd.compression.wire import build_wire
from kvserve_amd.connector import (CompressedKVConnector, CompressedKVConnectorMetadata, KVConnectorRole,
                                   LoopbackTransport)

pytestmark = pytest.mark.gpu

SENTINEL = -3.0
NAMES = [f"model.layers.{i}.self_attn.attn" for i in (0, 1, 2, 10, 11)]


def profile(min_size=0, hybrid=0.3):
    return {"pipeline": ["transformer", "quantizer", "codec"],
            "transformer_config": {"transform_type": "hadamard", "seed": 3237919422},
            "quantizer_config": {"model_name": "Llama-3.1-8B-Instruct", "hybrid_ratio": hybrid,
                                 "high_key_max_value": 16, "high_value_max_value": 16,
                                 "low_key_max_value": 12, "low_value_max_value": 12},
            "codec_config": {"codec_type": "bitpack", "bitpack_bits": 4}, "min_compress_size": min_size}


CREDIT = "tests._credit_transport:CreditLoopbackTransport"  # msgpack metadata, staging copies, credit


def vllm_config(producer, port, compression, heads=8, head=128, tp=(0, 1), transport="loopback"):
    extra = {"compression": compression, "transport_class": transport, "tp_rank": tp[0], "tp_size": tp[1]}
    return SimpleNamespace(
        kv_transfer_config=SimpleNamespace(is_kv_producer=producer, kv_buffer_size=1 << 34, kv_ip="127.0.0.1",
                                           kv_port=port, kv_connector_extra_config=extra),
        cache_config=SimpleNamespace(block_size=16),
        model_config=SimpleNamespace(get_num_kv_heads=lambda pc: heads, get_head_size=lambda: head,
                                     model="Llama-3.1-8B-Instruct", use_mla=False),
        parallel_config=SimpleNamespace())


class _Layer:
    def __init__(self, cache):
        self.kv_cache = [cache]


@pytest.fixture(autouse=True)
def _fresh_channels():
    LoopbackTransport.reset_channels()
    yield
    LoopbackTransport.reset_channels()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _caches(cuda, names, P, H, D, seed, fill=None):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for n in names:
        if fill is None:
            x = torch.randn((2, P, 16, H, D), generator=g)
            x[0, :, :, :, 3] *= 8.0      # an outlier K channel
            out[n] = x.to(torch.bfloat16).to(cuda)
        else:
            out[n] = torch.full((2, P, 16, H, D), fill, dtype=torch.bfloat16, device=cuda)
    return out


def _run(cuda, compression, prod, cons, p_ids, d_ids, port, heads, skip_layers=(), tp=(0, 1), transport="loopback"):
    names = list(prod)
    H, D = prod[names[0]].shape[3:]
    p = CompressedKVConnector(vllm_config(True, port, compression, heads, D, tp, transport), KVConnectorRole.WORKER)
    d = CompressedKVConnector(vllm_config(False, port, compression, heads, D, tp, transport), KVConnectorRole.WORKER)
    pm, dm = CompressedKVConnectorMetadata(), CompressedKVConnectorMetadata()
    pm.add_request("p-req", "T", list(range(16 * len(p_ids))), p_ids, 16)
    dm.add_request("d-req", "T", list(range(16 * len(d_ids))), d_ids, 16)
    p.bind_connector_metadata(pm)
    for n in names:
        p.save_kv_layer(n, prod[n], None)
    p.wait_for_save()
    d.bind_connector_metadata(dm)
    layers = {n: _Layer(cons[n]) for n in names if n not in skip_layers}
    d.start_load_kv(SimpleNamespace(no_compile_layers=layers, virtual_engine=0))
    torch.cuda.synchronize()
    return p, d


def _reference_procedure(compression, prod, p_ids, heads, tp=(0, 1)):
    """Stack the request's blocks in sorted-name order, compress the stack and
    decompress it: what the reference's connector writes into the decode cache."""
    names = sorted(prod)
    D = prod[names[0]].shape[-1]
    idx = torch.tensor(p_ids, device=prod[names[0]].device)
    stacked = torch.stack([prod[n][:, idx] for n in names])
    ad = KVCompressionAdapter(compression, num_kv_heads=heads, head_size=D, model_name="Llama-3.1-8B-Instruct",
                              tp_rank=tp[0], tp_size=tp[1])
    packet = ad.compress(stacked, "ref")
    return names, stacked, packet, (ad.decompress(packet) if packet is not None else None)


def _assert_written(cons, names, d_ids, expect, skip=()):
    nb = expect.shape[2]
    for i, n in enumerate(names):
        c = cons[n]
        if n in skip:
            assert (c == SENTINEL).all(), n
            continue
        got = c[:, torch.tensor(d_ids[:nb], device=c.device)]
        assert torch.equal(got, expect[i]), n
        mask = torch.ones(c.shape[1], dtype=torch.bool, device=c.device)
        mask[torch.tensor(d_ids[:nb], device=c.device)] = False
        assert (c[:, mask] == SENTINEL).all(), n


@pytest.mark.parametrize("transport", ["loopback", CREDIT])
def test_compressed_transfer_equals_reference_procedure(cuda, transport):
    """5 layers whose names sort out of numeric order, 40 blocks at random producer
    ids, written at the first 40 of 48 consumer ids; the sent stream is byte-equal to
    the stacked path's and the decode cache holds the stacked path's round trip.  Over
    the hand-off, and over the credit transport, whose msgpack hop and staging copies
    stand for a network's (the bundle is restored from msgpack'd metadata)."""
    P, H, D = 96, 8, 128
    g = torch.Generator().manual_seed(11)
    p_ids = torch.randperm(P, generator=g)[:40].tolist()
    d_ids = torch.randperm(P, generator=g)[:48].tolist()
    prod = _caches(cuda, NAMES, P, H, D, 5)
    cons = _caches(cuda, NAMES, P, H, D, 0, fill=SENTINEL)
    p, d = _run(cuda, profile(), prod, cons, p_ids, d_ids, 20, H, transport=transport)
    names, stacked, ref_packet, ref_out = _reference_procedure(profile(), prod, p_ids, H)
    assert names[2:] == ["model.layers.10.self_attn.attn", "model.layers.11.self_attn.attn",
                         "model.layers.2.self_attn.attn"]
    _assert_written(cons, names, d_ids, ref_out)
    sends = [r for r in p._transport.stats if r["direction"] == "send"]
    assert len(sends) == 1 and sends[0]["kind"] == "bundle"
    wire = build_wire(ref_packet, 512 << 20)
    assert sends[0]["payload_bytes"] == wire.nbytes < stacked.numel() * 2 // 3
    loads = [r for r in d._transport.stats if r["direction"] == "load_wait"]
    assert [r["kind"] for r in loads] == ["compressed"] and d._transport._ch.reserved == 0


def test_sent_stream_is_byte_equal_to_stacked_path(cuda):
    P, H, D = 64, 8, 128
    g = torch.Generator().manual_seed(12)
    p_ids = torch.randperm(P, generator=g)[:24].tolist()
    prod = _caches(cuda, NAMES, P, H, D, 6)
    _, _, ref_packet, _ = _reference_procedure(profile(), prod, p_ids, H)
    ad = KVCompressionAdapter(profile(), num_kv_heads=H, head_size=D, model_name="Llama-3.1-8B-Instruct")
    paged = ad.compress_paged([prod[n] for n in sorted(prod)], p_ids, "paged")
    assert torch.equal(paged.compressed_tensor, ref_packet.compressed_tensor)
    q_ref = ref_packet.metadata["quantization_params"]
    q = paged.metadata["quantization_params"]
    for a, b in zip(q, q_ref):
        for sec in ("high_key_meta", "high_value_meta", "low_key_meta", "low_value_meta"):
            for k in ("min_val", "quant_scale"):
                if b[sec][k] is None:
                    assert a[sec][k] is None
                else:
                    assert torch.equal(a[sec][k], b[sec][k]), (sec, k)


@pytest.mark.parametrize("compression", [None, "below_min"])
def test_raw_transfer_is_bit_exact(cuda, compression):
    """No compression, and compression below min_compress_size (falls back to a raw
    send): the decode cache holds the producer's blocks bit for bit."""
    P, H, D = 48, 8, 128
    g = torch.Generator().manual_seed(13)
    p_ids = torch.randperm(P, generator=g)[:9].tolist()
    d_ids = torch.randperm(P, generator=g)[:9].tolist()
    prod = _caches(cuda, NAMES, P, H, D, 7)
    cons = _caches(cuda, NAMES, P, H, D, 0, fill=SENTINEL)
    comp = profile(min_size=1 << 40) if compression == "below_min" else None
    p, d = _run(cuda, comp, prod, cons, p_ids, d_ids, 21, H)
    names = sorted(prod)
    idx = torch.tensor(p_ids, device=cuda)
    _assert_written(cons, names, d_ids, torch.stack([prod[n][:, idx] for n in names]))
    assert [r["kind"] for r in p._transport.stats if r["direction"] == "send"] == ["tensor"]


def test_missing_decode_layer_is_skipped(cuda):
    """A layer absent from the decode forward context is skipped (the fused path
    needs every layer, so the load goes through decompress + inject)."""
    P, H, D = 64, 8, 128
    g = torch.Generator().manual_seed(14)
    p_ids = torch.randperm(P, generator=g)[:12].tolist()
    d_ids = torch.randperm(P, generator=g)[:12].tolist()
    prod = _caches(cuda, NAMES, P, H, D, 8)
    cons = _caches(cuda, NAMES, P, H, D, 0, fill=SENTINEL)
    skip = (NAMES[2],)
    _run(cuda, profile(), prod, cons, p_ids, d_ids, 22, H, skip_layers=skip)
    names, _, _, ref_out = _reference_procedure(profile(), prod, p_ids, H)
    _assert_written(cons, names, d_ids, ref_out, skip=skip)


def test_tensor_parallel_head_slice(cuda):
    """TP rank 1 of 2 (4 of Llama's 8 KV heads per rank): same as the stacked path
    built for that rank."""
    P, H, D = 64, 4, 128
    g = torch.Generator().manual_seed(15)
    p_ids = torch.randperm(P, generator=g)[:20].tolist()
    d_ids = torch.randperm(P, generator=g)[:20].tolist()
    prod = _caches(cuda, NAMES, P, H, D, 9)
    cons = _caches(cuda, NAMES, P, H, D, 0, fill=SENTINEL)
    _run(cuda, profile(), prod, cons, p_ids, d_ids, 23, H, tp=(1, 2))
    names, _, _, ref_out = _reference_procedure(profile(), prod, p_ids, H, tp=(1, 2))
    _assert_written(cons, names, d_ids, ref_out)


def test_large_request_is_sent_in_layer_chunks(cuda):
    """A request above 500 MiB of raw KV travels as manager chunks of 8 layers
    (compression_manager.py:229-235) and decodes to the stacked path's result."""
    P, H, D, B = 1100, 8, 128, 1040
    names = [f"model.layers.{i}.self_attn.attn" for i in range(10)]
    g = torch.Generator().manual_seed(16)
    p_ids = torch.randperm(P, generator=g)[:B].tolist()
    d_ids = torch.randperm(P, generator=g)[:B].tolist()
    prod = _caches(cuda, names, P, H, D, 10)
    cons = _caches(cuda, names, P, H, D, 0, fill=SENTINEL)
    p, _ = _run(cuda, profile(), prod, cons, p_ids, d_ids, 24, H)
    assert 10 * 2 * B * 16 * H * D * 2 > 500 * 2 ** 20
    del p
    names_s, stacked, ref_packet, ref_out = _reference_procedure(profile(), prod, p_ids, H)
    assert ref_packet.is_chunked and len(ref_packet.chunks) == 2
    del stacked, ref_packet
    _assert_written(cons, names_s, d_ids, ref_out)
