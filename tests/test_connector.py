"""Connector (kvserve_amd.connector) host logic on the CPU: the reference's receiver
credit tests (tests/test_receiver_credits.py:16-70), the load loop's timeout and
failure paths, the error contracts of compressed payloads, the scheduler-side
bookkeeping (compressed_kv_connector.py:509-630) and a raw producer -> loopback ->
consumer round trip through CPU caches (device indexing path; the HIP paths run in
the gpu tests)."""

import threading
from types import SimpleNamespace

import pytest
import torch

import kvserve_amd.connector.compressed_kv_connector as connector_module
from kvserve_amd.connector import (CompressedKVConnector, CompressedKVConnectorMetadata, KVConnectorRole,
                                   LoopbackTransport, ReqMeta, make_slot_mapping)
from kvserve_amd.connector.transport import payload_nbytes
from tests._credit_transport import CreditLoopbackTransport

PROFILE = {"pipeline": ["transformer", "quantizer", "codec"],
           "transformer_config": {"transform_type": "hadamard", "seed": 3237919422},
           "quantizer_config": {"model_name": "Llama-3.1-8B-Instruct", "hybrid_ratio": 0.3,
                                "high_key_max_value": 16, "high_value_max_value": 16,
                                "low_key_max_value": 12, "low_value_max_value": 12},
           "codec_config": {"codec_type": "bitpack", "bitpack_bits": 4}}


def vllm_config(producer, port=7000, compression=None, transport="loopback", buffer=1 << 30, heads=8, head=128,
                mla=False, block_size=16):
    extra = {"compression": compression, "transport_class": transport}
    return SimpleNamespace(
        kv_transfer_config=SimpleNamespace(is_kv_producer=producer, kv_buffer_size=buffer, kv_ip="127.0.0.1",
                                           kv_port=port, kv_connector_extra_config=extra),
        cache_config=SimpleNamespace(block_size=block_size),
        model_config=SimpleNamespace(get_num_kv_heads=lambda pc: heads, get_head_size=lambda: head,
                                     model="/models/Llama-3.1-8B-Instruct/", use_mla=mla),
        parallel_config=SimpleNamespace())


@pytest.fixture(autouse=True)
def _fresh_channels():
    LoopbackTransport.reset_channels()
    yield
    LoopbackTransport.reset_channels()


def test_slot_mapping_known_answer():
    assert make_slot_mapping(list(range(6)), [3, 7], 4).tolist() == [12, 13, 14, 15, 28, 29]
    assert make_slot_mapping([], [5], 16).numel() == 0
    m = CompressedKVConnectorMetadata()
    m.add_request("r", "t", [1, 2, 3], [9], 2)
    assert m.requests[0].slot_mapping.tolist() == [18, 19]


def test_load_reordered_payloads_releases_credit(monkeypatch):
    """The reference's test: the payload of the second scheduled request arrives
    first and consuming it is what lets the first one arrive."""
    class Transport:
        device = torch.device("cpu")

        def __init__(self):
            self.ready = {"B": [([], torch.ones(1))]}
            self.rows = []

        def drain_received(self):
            ready, self.ready = self.ready, {}
            return ready

        def payload_nbytes(self, payload):
            return payload.numel() * payload.element_size()

        def release_received(self, rid, nbytes):
            if rid == "B":
                self.ready["A"] = [([], torch.ones(1))]

        def record_stat(self, row):
            self.rows.append(row)

        def set_expected_requests(self, rids):
            pass

    obj = CompressedKVConnector.__new__(CompressedKVConnector)
    obj.is_producer = False
    obj._transport = Transport()
    obj._worker_received_kv = connector_module.defaultdict(connector_module.deque)
    meta = CompressedKVConnectorMetadata(requests=[
        ReqMeta(rid, rid, [], [], torch.empty(0, dtype=torch.long)) for rid in ["A", "B"]])
    obj._get_connector_metadata = lambda: meta
    monkeypatch.setattr(connector_module, "_LOAD_TIMEOUT_S", 0.1)
    obj.start_load_kv(SimpleNamespace(no_compile_layers={}, virtual_engine=0))
    assert not any(row["kind"] == "timeout" for row in obj._transport.rows)
    assert {row["request_id"] for row in obj._transport.rows} == {"A", "B"}
    assert not obj._worker_received_kv


def test_one_scheduled_overflow_unblocks_next_decode_step():
    """Credit rule of the reference's test: with the staging held by a future
    request, one scheduled request may pass the budget; the next is admitted once
    that one releases its credit."""
    tx = CreditLoopbackTransport(True, port=1)
    rx = CreditLoopbackTransport(False, port=1, recv_buffer_size=100, device="cpu")
    for rid in ["future", "current-1", "current-2"]:
        tx.send(rid, ["l"], torch.zeros(100, dtype=torch.uint8))
    assert list(rx.drain_received()) == ["future"]
    assert tx.pending_bytes() == 200
    rx.set_expected_requests(["current-1", "current-2"])
    assert list(rx.drain_received()) == ["current-1"]
    assert rx._ch.reserved == 200 and rx._ch.priority == "current-1"
    assert rx.drain_received() == {}
    rx.release_received("current-1", 100)
    assert list(rx.drain_received()) == ["current-2"] and rx._ch.reserved == 200
    rx.release_received("current-2", 100)
    rx.release_received("future", 100)
    assert rx._ch.reserved == 0 and rx._ch.priority is None and tx.pending_bytes() == 0
    kinds = [(r["direction"], r["kind"]) for r in rx.stats]
    assert kinds.count(("recv_credit", "reserve")) == 3 and kinds.count(("recv_credit_release", "release")) == 3


def test_oversize_payload_admitted_into_empty_staging():
    tx = CreditLoopbackTransport(True, port=2)
    rx = CreditLoopbackTransport(False, port=2, recv_buffer_size=10, device="cpu")
    tx.send("big", ["l"], torch.zeros(64, dtype=torch.uint8))
    got = rx.drain_received()
    assert list(got) == ["big"] and [r for r in rx.stats if r.get("oversize")]


def test_wait_for_below_blocks_until_the_consumer_admits():
    tx = CreditLoopbackTransport(True, port=3)
    rx = CreditLoopbackTransport(False, port=3, recv_buffer_size=100, device="cpu")
    tx.send("a", ["l"], torch.zeros(80, dtype=torch.uint8))
    tx.send("b", ["l"], torch.zeros(80, dtype=torch.uint8))
    rx.drain_received()                      # admits a; b waits for credit
    assert tx.pending_bytes() == 80
    t = threading.Timer(0.05, lambda: rx.release_received("a", 80))
    t.start()
    waited = tx.wait_for_below(0, timeout_s=5.0)
    t.join()
    assert tx.pending_bytes() == 0 and 0.03 < waited < 5.0


def test_bundle_hand_off_and_payload_nbytes():
    """The loopback hands over the tensors and the metadata dict themselves; the
    test-only credit transport sends the metadata through msgpack (a tensor in it
    fails there) and stages copies."""
    tx = LoopbackTransport(True, port=4)
    rx = LoopbackTransport(False, port=4, device="cpu")
    body, aux = [torch.arange(10, dtype=torch.uint8)], [torch.ones(3, dtype=torch.bfloat16)]
    meta = {"a": [1, 2], "b": {"c": "x"}}
    tx.send_bundle("r", ["__compressed__", "l0"], meta, body, aux)
    ((names, payload),) = rx.drain_received()["r"]
    assert names == ["__compressed__", "l0"] and payload["__bundle__"] and payload["meta"] is meta
    assert payload_nbytes(payload) == 16 and payload["body_chunks"][0] is body[0]
    ctx, crx = CreditLoopbackTransport(True, port=14), CreditLoopbackTransport(False, port=14, device="cpu")
    ctx.send_bundle("r", ["__compressed__", "l0"], meta, body, aux)
    ((_, staged),) = crx.drain_received()["r"]
    assert staged["meta"] == meta and staged["meta"] is not meta
    assert staged["body_chunks"][0] is not body[0] and torch.equal(staged["body_chunks"][0], body[0])
    with pytest.raises(TypeError):
        ctx.send_bundle("r", [], {"t": torch.zeros(1)}, body, aux)
    assert payload_nbytes(None) == 0


def test_load_times_out_and_records_it(monkeypatch):
    monkeypatch.setattr(connector_module, "_LOAD_TIMEOUT_S", 0.05)
    c = CompressedKVConnector(vllm_config(False, port=5), KVConnectorRole.WORKER)
    meta = CompressedKVConnectorMetadata()
    meta.add_request("req", "tx-1", [1, 2], [0], 16)
    c.bind_connector_metadata(meta)
    with pytest.raises(TimeoutError, match="tx-1"):
        c.start_load_kv(SimpleNamespace(no_compile_layers={}, virtual_engine=0))
    rows = [r for r in c._transport.stats if r["direction"] == "load_wait"]
    assert rows and rows[0]["kind"] == "timeout" and rows[0]["scheduler_request_id"] == "req"
    assert c._transport._ch.expected == set()


def test_failure_marker_raises_and_releases():
    c = CompressedKVConnector(vllm_config(False, port=6), KVConnectorRole.WORKER)
    meta = CompressedKVConnectorMetadata()
    meta.add_request("req", "tx-2", [1], [0], 16)
    c.bind_connector_metadata(meta)
    c._transport.mark_failed("tx-2")
    with pytest.raises(RuntimeError, match="KV transport failed for tx-2"):
        c.start_load_kv(SimpleNamespace(no_compile_layers={}, virtual_engine=0))
    assert [r["kind"] for r in c._transport.stats if r["direction"] == "load_wait"] == ["failed"]


@pytest.mark.parametrize("compression, payload, match", [
    (None, {"__bundle__": True, "meta": {}, "body_chunks": [], "aux_tensors": []},
     "No KV decompressor configured for tx-3"),
    (PROFILE, torch.zeros(4, dtype=torch.uint8), "Invalid compressed KV payload for tx-3"),
])
def test_compressed_payload_contracts(compression, payload, match):
    c = CompressedKVConnector(vllm_config(False, port=7, compression=compression), KVConnectorRole.WORKER)
    meta = CompressedKVConnectorMetadata()
    meta.add_request("req", "tx-3", [1], [0], 16)
    c.bind_connector_metadata(meta)
    c._transport._ch.received["tx-3"].append((["__compressed__", "l0"], payload))
    with pytest.raises(RuntimeError, match=match):
        c.start_load_kv(SimpleNamespace(no_compile_layers={}, virtual_engine=0))


def test_transport_selection_and_layout():
    with pytest.raises(NotImplementedError, match="transport_class"):
        CompressedKVConnector(vllm_config(True, transport=None), KVConnectorRole.WORKER)
    with pytest.raises(ValueError, match="module:Class"):
        CompressedKVConnector(vllm_config(True, transport="nocolon"), KVConnectorRole.WORKER)
    c = CompressedKVConnector(vllm_config(True, transport="kvserve_amd.connector.transport:LoopbackTransport"),
                              KVConnectorRole.WORKER)
    assert isinstance(c._transport, LoopbackTransport) and c._transport.is_sender
    assert CompressedKVConnector(vllm_config(True, transport=None), KVConnectorRole.SCHEDULER).is_producer
    assert CompressedKVConnector.get_required_kvcache_layout(vllm_config(True)) == "NHD"
    assert CompressedKVConnector.get_required_kvcache_layout(vllm_config(True, mla=True)) is None
    assert CompressedKVConnector.get_required_kvcache_layout(SimpleNamespace(model_config=None)) is None
    assert c._model_name == "Llama-3.1-8B-Instruct"


def _sched_out(new=(), cached=None, num_scheduled=None):
    cached = cached or SimpleNamespace(req_ids=[], num_computed_tokens=[], new_block_ids=[], resumed_req_ids=set())
    return SimpleNamespace(scheduled_new_reqs=list(new), scheduled_cached_reqs=cached,
                           num_scheduled_tokens=num_scheduled or {})


def test_scheduler_producer_chunked_prefill_accumulates_blocks():
    c = CompressedKVConnector(vllm_config(True, transport=None, block_size=4), KVConnectorRole.SCHEDULER)
    req = SimpleNamespace(request_id="r1", kv_transfer_params={"transfer_id": "T1"})
    c.update_state_after_alloc(req, None, 0)
    new = SimpleNamespace(req_id="r1", prompt_token_ids=list(range(10)), num_computed_tokens=0, block_ids=([5, 6],))
    m = c.build_connector_meta(_sched_out([new], num_scheduled={"r1": 8}))
    assert m.requests == [] and c.chunked_prefill["r1"] == ([5, 6], list(range(10)))
    cached = SimpleNamespace(req_ids=["r1"], num_computed_tokens=[8], new_block_ids=[([9],)], resumed_req_ids=set())
    m = c.build_connector_meta(_sched_out(cached=cached, num_scheduled={"r1": 2}))
    (rq,) = m.requests
    assert (rq.request_id, rq.transfer_id, rq.block_ids) == ("r1", "T1", [5, 6, 9])
    assert rq.slot_mapping.tolist() == [20, 21, 22, 23, 24, 25, 26, 27, 36, 37]
    assert "r1" not in c.chunked_prefill
    assert c.get_num_new_matched_tokens(SimpleNamespace(prompt_token_ids=[1] * 10), 0) == (0, False)
    assert c.request_finished(req, []) == (False, None) and "r1" not in c._request_transfer_ids


def test_scheduler_consumer_loads_new_and_resumed_requests():
    c = CompressedKVConnector(vllm_config(False, transport=None, block_size=4), KVConnectorRole.SCHEDULER)
    assert c.get_num_new_matched_tokens(SimpleNamespace(prompt_token_ids=[1] * 10), 0) == (9, False)
    assert c.get_num_new_matched_tokens(SimpleNamespace(prompt_token_ids=[1] * 10), 9) == (0, False)
    blocks = SimpleNamespace(get_block_ids=lambda: ([3, 4, 5],))
    r1 = SimpleNamespace(request_id="r1", kv_transfer_params={"transfer_id": "T1"})
    r2 = SimpleNamespace(request_id="r2", kv_transfer_params=None, all_token_ids=list(range(20)))
    c.update_state_after_alloc(r1, blocks, 9)
    c.update_state_after_alloc(r2, blocks, 9)
    c.update_state_after_alloc(SimpleNamespace(request_id="r3", kv_transfer_params=None), blocks, 0)
    assert set(c._requests_need_load) == {"r1", "r2"}
    new = SimpleNamespace(req_id="r1", prompt_token_ids=list(range(10)), num_computed_tokens=0, block_ids=([3, 4, 5],))
    cached = SimpleNamespace(req_ids=["r2"], num_computed_tokens=[11], new_block_ids=[([7, 8, 9],)],
                             resumed_req_ids={"r2"})
    m = c.build_connector_meta(_sched_out([new], cached))
    got = {r.request_id: (r.transfer_id, r.block_ids, len(r.token_ids)) for r in m.requests}
    assert got == {"r1": ("T1", [3, 4, 5], 10), "r2": ("r2", [7, 8, 9], 12)}
    assert c._requests_need_load == {}


class _Layer:
    def __init__(self, cache):
        self.kv_cache = [cache]


def _raw_roundtrip(names, producer_ids, consumer_ids, nb_pool=12, port=8):
    g = torch.Generator().manual_seed(3)
    prod = {n: torch.randn((2, nb_pool, 4, 2, 8), generator=g).to(torch.bfloat16) for n in names}
    cons = {n: torch.full((2, nb_pool, 4, 2, 8), -7.0, dtype=torch.bfloat16) for n in names}
    p = CompressedKVConnector(vllm_config(True, port=port), KVConnectorRole.WORKER)
    d = CompressedKVConnector(vllm_config(False, port=port), KVConnectorRole.WORKER)
    pm, dm = CompressedKVConnectorMetadata(), CompressedKVConnectorMetadata()
    pm.add_request("req-p", "T", list(range(len(producer_ids) * 4)), producer_ids, 4)
    dm.add_request("req-d", "T", list(range(len(consumer_ids) * 4)), consumer_ids, 4)
    p.bind_connector_metadata(pm)
    for n in names:                      # vLLM's order: model order, not sorted
        p.save_kv_layer(n, prod[n], None)
    p.wait_for_save()
    d.bind_connector_metadata(dm)
    d.start_load_kv(SimpleNamespace(no_compile_layers={n: _Layer(cons[n]) for n in names}, virtual_engine=0))
    return prod, cons, p, d


def test_raw_roundtrip_keeps_layer_names_and_blocks():
    names = [f"model.layers.{i}.self_attn.attn" for i in (0, 1, 2, 10, 11)]
    prod, cons, p, d = _raw_roundtrip(names, [4, 9, 2], [1, 3, 5, 7])
    sent = [r for r in p._transport.stats if r["direction"] == "send"]
    assert len(sent) == 1 and sent[0]["kind"] == "tensor"
    for n in names:
        assert torch.equal(cons[n][:, [1, 3, 5]], prod[n][:, [4, 9, 2]])
        assert (cons[n][:, [0, 2, 4, 6, 7, 8, 9, 10, 11]] == -7).all()
    assert d._transport._ch.reserved == 0 and not d._worker_received_kv
    assert [r["kind"] for r in d._transport.stats if r["direction"] == "load_wait"] == ["raw"]


def test_layers_are_stacked_in_sorted_name_order():
    """layer i of the payload is the i-th name in sorted order ("…10…" before "…2…"),
    the order that also fixes each layer's transform seed."""
    names = ["model.layers.2.attn", "model.layers.10.attn", "model.layers.1.attn"]
    tx = LoopbackTransport(False, port=9, device="cpu")
    g = torch.Generator().manual_seed(4)
    caches = {n: torch.randn((2, 6, 4, 2, 8), generator=g).to(torch.bfloat16) for n in names}
    p = CompressedKVConnector(vllm_config(True, port=9), KVConnectorRole.WORKER)
    m = CompressedKVConnectorMetadata()
    m.add_request("r", "T", [0] * 8, [5, 0], 4)
    p.bind_connector_metadata(m)
    for n in names:
        p.save_kv_layer(n, caches[n], None)
    p.wait_for_save()
    ((lnames, stacked),) = tx.drain_received()["T"]
    assert lnames == sorted(names) == ["model.layers.1.attn", "model.layers.10.attn", "model.layers.2.attn"]
    for i, n in enumerate(lnames):
        assert torch.equal(stacked[i], caches[n][:, [5, 0]])


def test_stale_buffers_dropped_and_consumer_side_noops():
    p = CompressedKVConnector(vllm_config(True, port=10), KVConnectorRole.WORKER)
    m1 = CompressedKVConnectorMetadata()
    m1.add_request("old", "T-old", [0], [0], 4)
    p.bind_connector_metadata(m1)
    p.save_kv_layer("l0", torch.zeros((2, 2, 4, 1, 8), dtype=torch.bfloat16), None)
    p.bind_connector_metadata(CompressedKVConnectorMetadata())
    p.wait_for_save()
    assert p._layer_buffers == {} and p._transport.pending_bytes() == 0
    d = CompressedKVConnector(vllm_config(False, port=10), KVConnectorRole.WORKER)
    d.save_kv_layer("l0", torch.zeros(1), None)
    d.wait_for_save()
    assert d._layer_buffers == {}
    assert d.get_finished(set()) == (None, None)


def test_sent_buffers_are_never_written_again():
    """The loopback hands the consumer the producer's tensors themselves, so the producer
    must never write a sent buffer again: a later request's save (after the caches
    changed) leaves the earlier request's received tensor intact, in other storage."""
    names = ["model.layers.0.attn", "model.layers.1.attn"]
    tx = LoopbackTransport(False, port=15, device="cpu")
    g = torch.Generator().manual_seed(5)
    caches = {n: torch.randn((2, 6, 4, 2, 8), generator=g).to(torch.bfloat16) for n in names}
    p = CompressedKVConnector(vllm_config(True, port=15), KVConnectorRole.WORKER)
    got = {}
    for rid, blocks in (("A", [1, 2]), ("B", [1, 2])):
        m = CompressedKVConnectorMetadata()
        m.add_request(rid, "T" + rid, [0] * 8, blocks, 4)
        p.bind_connector_metadata(m)
        for n in names:
            p.save_kv_layer(n, caches[n], None)
        p.wait_for_save()
        ((_, stacked),) = tx.drain_received()["T" + rid]
        got[rid] = (stacked, stacked.clone())
        for n in names:
            caches[n].mul_(-1)  # the producer's caches move on before the next save
    a, a_at_receive = got["A"]
    b, _ = got["B"]
    assert torch.equal(a, a_at_receive)
    assert torch.equal(b, -a)
    assert a.untyped_storage().data_ptr() != b.untyped_storage().data_ptr()
