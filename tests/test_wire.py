"""Wire bundle (kvserve_amd.compression.wire) against the reference's format rules
(kvserve_v1/compression/wire.py:16-289): known answers derived by hand from those rules,
round trips, msgpack-safety and the error contracts.  CPU tensors; the GPU case goes
through the adapter in test_gpu_api-style at the end (marked gpu)."""

import msgpack
import pytest
import torch

from kvserve_amd.compression.compression_manager import CompressedKVData
from kvserve_amd.compression.wire import AUX_PLACEHOLDER, CompressedWire, build_wire, restore_from_wire


def _payload(qparams, tensor=None, **kw):
    meta = {"request_id": "req-7", "codec_applied": True, "quantization_params": qparams}
    return CompressedKVData("req-7", 3, tensor if tensor is not None else torch.arange(10, dtype=torch.uint8),
                            meta, 1000, 10, **kw)


def test_known_answer_copy_path_aligns_each_tensor():
    a = torch.tensor([1, 2, 3], dtype=torch.uint8)                # 3 bytes at 0
    b = torch.tensor([[1.0, -2.0]], dtype=torch.bfloat16)        # 4 bytes at 4 (pad 1)
    c = torch.tensor(5, dtype=torch.int64)                       # 8 bytes at 8
    qp = [{"high_key_meta": {"min_val": a, "quant_scale": b, "max_value": 16}, "original_dtype": "bfloat16"},
          {"low_value_meta": {"min_val": c, "quant_scale": None, "max_value": 4}}]
    w = build_wire(_payload(qp), max_chunk_bytes=1 << 20)
    assert w.meta == {
        "is_chunked": False, "layer_id": 3, "original_size": 1000, "compressed_size": 10,
        "metadata": {"request_id": "req-7", "codec_applied": True, "quantization_params": [
            {"high_key_meta": {"min_val": [AUX_PLACEHOLDER, 0], "quant_scale": [AUX_PLACEHOLDER, 1],
                               "max_value": 16}, "original_dtype": "bfloat16"},
            {"low_value_meta": {"min_val": [AUX_PLACEHOLDER, 2], "quant_scale": None, "max_value": 4}}]},
        "body_mode": "single", "body_spec": {"shape": [10], "dtype": "uint8"},
        "aux_layout": {"mode": "coalesced_bytes", "tensors": [
            {"storage": 0, "offset": 0, "nbytes": 3, "shape": [3], "dtype": "uint8"},
            {"storage": 0, "offset": 4, "nbytes": 4, "shape": [1, 2], "dtype": "bfloat16"},
            {"storage": 0, "offset": 8, "nbytes": 8, "shape": [], "dtype": "int64"}]},
    }
    assert AUX_PLACEHOLDER == "__kvserve_aux_tensor__"
    assert len(w.aux_tensors) == 1 and w.aux_tensors[0].dtype == torch.uint8 and w.aux_tensors[0].numel() == 16
    blob = w.aux_tensors[0]
    assert blob[:3].tolist() == [1, 2, 3] and blob[3].item() == 0
    assert torch.equal(blob[4:8].view(torch.bfloat16), b.reshape(-1))
    assert blob[8:16].view(torch.int64).item() == 5
    assert w.nbytes == 10 + 16
    r = restore_from_wire(w)
    q = r.metadata["quantization_params"]
    assert torch.equal(q[0]["high_key_meta"]["min_val"], a) and torch.equal(q[0]["high_key_meta"]["quant_scale"], b)
    assert torch.equal(q[1]["low_value_meta"]["min_val"], c) and q[1]["low_value_meta"]["quant_scale"] is None
    assert r.request_id == "req-7" and r.layer_id == 3 and torch.equal(r.compressed_tensor, torch.arange(10, dtype=torch.uint8))


def test_single_aux_tensor_has_no_layout():
    t = torch.tensor([1.5])
    w = build_wire(_payload({"k": t}), 1 << 20)
    assert "aux_layout" not in w.meta and w.aux_tensors[0] is t
    assert torch.equal(restore_from_wire(w).metadata["quantization_params"]["k"], t)


def test_scalar_and_int_metadata_roundtrip():
    # the reference's test_wire_scalar_metadata case
    vals = {"a": torch.tensor(1.5), "b": torch.tensor([1, 2], dtype=torch.int64)}
    r = restore_from_wire(build_wire(_payload(vals), 1 << 20))
    assert all(torch.equal(vals[k], r.metadata["quantization_params"][k]) for k in vals)


def test_slices_of_one_allocation_ship_without_copy():
    buf = torch.arange(64, dtype=torch.bfloat16)
    qp = [{"min_val": buf[8:16].view(1, 1, 2, 4), "quant_scale": buf[16:24].view(1, 1, 2, 4)},
          {"min_val": buf[40:48].view(8, 1, 1, 1)}]
    w = build_wire(_payload(qp), 1 << 20)
    blob = w.aux_tensors[0]
    assert blob.untyped_storage().data_ptr() == buf.untyped_storage().data_ptr()
    assert blob.numel() == (48 - 8) * 2  # from the first to the end of the last slice
    offs = [e["offset"] for e in w.meta["aux_layout"]["tensors"]]
    assert offs == [0, 16, 64]
    buf[9] = 99  # a view: later writes are visible (nothing was copied)
    r = restore_from_wire(w).metadata["quantization_params"]
    assert r[0]["min_val"].reshape(-1)[1].item() == 99
    assert torch.equal(r[0]["quant_scale"], qp[0]["quant_scale"]) and torch.equal(r[1]["min_val"], qp[1]["min_val"])


def test_byte_chunks_are_views_and_restore():
    body = torch.arange(1000, dtype=torch.int16).reshape(10, 100)
    w = build_wire(_payload({}, tensor=body), max_chunk_bytes=300)
    assert w.meta["body_mode"] == "byte_chunks" and w.meta["body_spec"] == {"shape": [10, 100], "dtype": "int16"}
    assert [c.numel() for c in w.body_chunks] == [300] * 6 + [200]
    assert all(c.untyped_storage().data_ptr() == body.untyped_storage().data_ptr() for c in w.body_chunks)
    assert torch.equal(restore_from_wire(w).compressed_tensor, body)
    with pytest.raises(ValueError, match="max_chunk_bytes"):
        build_wire(_payload({}, tensor=body), max_chunk_bytes=0)


def test_manager_chunks_and_msgpack_roundtrip():
    chunks = [torch.arange(5, dtype=torch.uint8), torch.arange(7, dtype=torch.uint8)]
    cm = [{"request_id": "r", "num_layers": 8, "start_layer_id": 0, "quantization_params": [{"m": torch.ones(2)}]},
          {"request_id": "r", "num_layers": 1, "start_layer_id": 8, "quantization_params": [{"m": torch.zeros(3)}]}]
    p = CompressedKVData("r", 8, None, {"request_id": "r", "chunked": True}, 123, 12, True, chunks, cm)
    w = build_wire(p, max_chunk_bytes=1)
    assert w.meta["body_mode"] == "manager_chunks" and w.body_chunks[0] is chunks[0]
    w = CompressedWire(msgpack.unpackb(msgpack.packb(w.meta), raw=False), w.body_chunks, w.aux_tensors)
    r = restore_from_wire(w)
    assert r.is_chunked and r.compressed_tensor is None and r.request_id == "r"
    assert [c.tolist() for c in r.chunks] == [c.tolist() for c in chunks]
    assert torch.equal(r.chunk_metadata[1]["quantization_params"][0]["m"], torch.zeros(3))
    assert r.chunk_metadata[1]["start_layer_id"] == 8


def test_contract_errors():
    with pytest.raises(ValueError, match="missing chunks"):
        build_wire(CompressedKVData("r", 0, None, {}, 0, 0, True, None, None), 10)
    with pytest.raises(ValueError, match="missing compressed_tensor"):
        build_wire(CompressedKVData("r", 0, None, {}, 0, 0, False), 10)
    with pytest.raises(TypeError, match="still contains a tensor"):
        build_wire(CompressedKVData("r", 0, torch.zeros(1), {"x": torch.zeros(1)}, 0, 0), 10)
    w = build_wire(_payload({"a": torch.ones(1), "b": torch.ones(1)}), 10)
    w.meta["aux_layout"]["mode"] = "other"
    with pytest.raises(ValueError, match="Unknown aux_layout"):
        restore_from_wire(w)


@pytest.mark.gpu
def test_adapter_payload_over_the_wire_decodes_identically(cuda):
    """Fused adapter packet -> wire (4 KiB body pieces, msgpack meta) -> restore ->
    decompress equals decompressing the packet itself; the metadata ships as one
    view of the packet's metadata allocation."""
    from kvserve_amd.compression import KVCompressionAdapter

    cfg = {"pipeline": ["transformer", "quantizer", "codec"],
           "transformer_config": {"transform_type": "hadamard", "seed": 3237919422},
           "quantizer_config": {"model_name": "Llama-3.1-8B-Instruct", "hybrid_ratio": 0.3,
                                "high_key_max_value": 16, "high_value_max_value": 16,
                                "low_key_max_value": 12, "low_value_max_value": 12},
           "codec_config": {"codec_type": "bitpack", "bitpack_bits": 4}}
    ad = KVCompressionAdapter(cfg, num_kv_heads=8, head_size=128)
    g = torch.Generator().manual_seed(9)
    x = torch.randn((3, 2, 5, 16, 8, 128), generator=g).to(torch.bfloat16).to(cuda)
    packet = ad.compress(x, "wire")
    w = build_wire(packet, max_chunk_bytes=4096)
    assert len(w.body_chunks) > 1 and len(w.aux_tensors) == 1
    qp0 = packet.metadata["quantization_params"][0]
    some = next(v["min_val"] for v in qp0.values() if isinstance(v, dict) and v.get("min_val") is not None)
    assert w.aux_tensors[0].untyped_storage().data_ptr() == some.untyped_storage().data_ptr()
    w = CompressedWire(msgpack.unpackb(msgpack.packb(w.meta), raw=False), w.body_chunks, w.aux_tensors)
    out = ad.decompress(restore_from_wire(w))
    assert torch.equal(out, ad.decompress(packet))


def _engine_tables(L, H, D, B, S, rows, G, gen):
    """Engine-layout metadata in one bf16 allocation and its reference-format dicts."""
    from kvserve_amd.compression._meta import layer_dict
    from kvserve_amd.profiles import section_profile

    kn, vn = L * 2 * H * D, L * 2 * G * B * S
    buf = torch.randn(kn + vn, generator=gen).to(torch.bfloat16)
    kmeta, vmeta = buf[:kn].view(L, 2, H, D), buf[kn:].view(L, 2, G, B * S)
    profs = [section_profile(row, 16, 16, 12, 12) for row in rows]
    return buf, kmeta, vmeta, [layer_dict(kmeta[l], vmeta[l], profs[l], B, S) for l in range(L)]


def test_engine_tables_come_back_as_views_also_over_the_wire():
    """Dicts made from the engine's one-allocation tables give the tables back as
    views (no copy), directly and after build_wire / restore_from_wire; dicts
    elsewhere take the copy path and give the same values."""
    from kvserve_amd.compression._meta import tables_from_dicts

    L, H, D, B, S = 3, 4, 8, 2, 4
    rows = [[True, False, False, True], [False] * 4, [True] * 4]   # G: 2, 1, 1 -> G = 2
    buf, kmeta, vmeta, dicts = _engine_tables(L, H, D, B, S, rows, 2, torch.Generator().manual_seed(1))
    k2, v2 = tables_from_dicts(dicts, H, D, B, S, "cpu")
    assert k2.data_ptr() == kmeta.data_ptr() and v2.data_ptr() == vmeta.data_ptr()
    assert torch.equal(k2, kmeta) and torch.equal(v2, vmeta)

    # the last layer uses one of two V groups, so the used span ends before the
    # allocation does: the wire ships the allocation to its end
    w = build_wire(_payload(dicts), 1 << 20)
    assert w.aux_tensors[0].numel() == buf.numel() * 2
    received = CompressedWire(msgpack.unpackb(msgpack.packb(w.meta), raw=False), w.body_chunks,
                              [w.aux_tensors[0].clone()])
    q = restore_from_wire(received).metadata["quantization_params"]
    k3, v3 = tables_from_dicts(q, H, D, B, S, "cpu")
    assert k3.untyped_storage().data_ptr() == received.aux_tensors[0].untyped_storage().data_ptr()
    assert torch.equal(k3, kmeta) and torch.equal(v3[0], vmeta[0]) and torch.equal(v3[1:, :, 0], vmeta[1:, :, 0])

    # copies of the sections (no shared allocation): copy path, same values
    copied = [{k: ({kk: (vv.clone() if isinstance(vv, torch.Tensor) else vv) for kk, vv in v.items()}
                   if isinstance(v, dict) else v) for k, v in d.items()} for d in dicts]
    k4, v4 = tables_from_dicts(copied, H, D, B, S, "cpu")
    assert k4.data_ptr() != kmeta.data_ptr()
    assert torch.equal(k4, kmeta) and torch.equal(v4[0], vmeta[0]) and torch.equal(v4[1:, :, 0], vmeta[1:, :, 0])


def _axis_tables(L, H, D, G, BS, axes):
    from kvserve_amd.engine import meta_shape

    ks, vs = meta_shape(axes[0], H, D, G, BS), meta_shape(axes[1], H, D, G, BS)
    kn, vn = L * 2 * ks[0] * ks[1], L * 2 * vs[0] * vs[1]
    buf = torch.randn(kn + vn).to(torch.bfloat16)
    return buf[:kn].view(L, 2, *ks), buf[kn:].view(L, 2, *vs)


@pytest.mark.parametrize("axes", [("channel", "token"), ("token", "tensor"), ("tensor", "channel")])
@pytest.mark.parametrize("chunked", [False, True])
def test_table_backed_params_pack_like_their_dicts(axes, chunked):
    """QuantParams straight from the engine tables go on the wire exactly as their
    materialised dicts would (same placeholder tree, aux layout and blob bytes, plus the
    tables key), and come back as QuantParams over the received tables whose dicts
    equal the sender's."""
    import msgpack

    from kvserve_amd.compression._meta import QuantParams, joined_tables, packet_params
    from kvserve_amd.compression.wire import TABLES_KEY
    from kvserve_amd.profiles import section_profile, whole_layer_profile

    L, H, D, B, S = 6, 4, 32, 3, 16
    kmeta, vmeta = _axis_tables(L, H, D, 2, B * S, axes)
    profs = [section_profile([l % 2 == 0, True, False, l % 3 == 0], 12, 8, 6, 4) for l in range(L - 1)]
    profs.append(whole_layer_profile(H, 6, 4, is_low=True))
    ranges = [(0, 4), (4, 6)] if chunked else [(0, L)]

    def payload(lazy):
        def qp(s, e):
            p = packet_params(kmeta, vmeta, profs, B, S, axes, s, e)
            return p if lazy else list(p)
        if not chunked:
            return _payload(qp(0, L))
        metas = [{"request_id": "req-7", "num_layers": e - s, "quantization_params": qp(s, e)} for s, e in ranges]
        return CompressedKVData("req-7", L - 1, None, {"request_id": "req-7", "is_chunked": True}, 1000, 10, True,
                                [torch.arange(4, dtype=torch.uint8) for _ in ranges], metas)

    fast, slow = build_wire(payload(True), 1 << 20), build_wire(payload(False), 1 << 20)
    fm = dict(fast.meta)
    assert fm.pop(TABLES_KEY) == {"k_offset": 0, "k_shape": list(kmeta.shape), "v_offset": 2 * kmeta.numel(),
                                  "v_shape": list(vmeta.shape)}
    assert fm == slow.meta
    assert torch.equal(fast.aux_tensors[0], slow.aux_tensors[0])
    assert fast.aux_tensors[0].data_ptr() == kmeta.data_ptr()  # shipped without a copy
    wire = CompressedWire(msgpack.unpackb(msgpack.packb(fast.meta)), fast.body_chunks,
                          [fast.aux_tensors[0].clone()])
    back = restore_from_wire(wire)
    metas = back.chunk_metadata if chunked else [back.metadata]
    params = [m["quantization_params"] for m in metas]
    assert all(isinstance(p, QuantParams) for p in params)
    k2, v2 = joined_tables(params)
    assert torch.equal(k2, kmeta) and torch.equal(v2, vmeta)
    want = [d for s, e in ranges for d in packet_params(kmeta, vmeta, profs, B, S, axes, s, e)]
    got = [d for p in params for d in p]
    for a, b in zip(got, want):
        for sec in ("high_key_meta", "high_value_meta", "low_key_meta", "low_value_meta"):
            for f in ("min_val", "quant_scale"):
                x, y = a[sec][f], b[sec][f]
                assert (x is None and y is None) or (x.shape == y.shape and torch.equal(x, y)), (sec, f)
