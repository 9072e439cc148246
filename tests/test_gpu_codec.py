"""GPU parity of the HIP engine against the CPU oracle (calls go through the C-ABI).

Bars:
  bitpack / unpack, gather / scatter: bit-exact
  symbols: |delta| <= 1 everywhere and mismatches <= 1e-4 of the elements
  dequantized KV: max|x - x_ref| / max|x_ref| <= 1e-2 per (layer, part)
"""

import numpy as np
import pytest
import torch

from oracle import cbitpack
from oracle import kvpipe as kp

pytestmark = pytest.mark.gpu

SYM_MISMATCH_FRAC = 1e-4
DEQ_REL_TOL = 1e-2


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def _oracle_profile(p):
    return kp.LayerProfile(kp.PartProfile(list(p.k_order), list(p.k_levels), list(p.k_groups())),
                           kp.PartProfile(list(p.v_order), list(p.v_levels), list(p.v_group)))


def sym_diff(a: np.ndarray, b: np.ndarray):
    d = np.abs(a.astype(np.int16) - b.astype(np.int16))
    return int(d.max(initial=0)), float(np.count_nonzero(d)) / max(1, d.size)


# ------------------------------------------------------------------ bitpack
@pytest.mark.parametrize("bits", range(1, 9))
@pytest.mark.parametrize("shape", [[], [0, 2], [1], [7], [13], [2, 3, 257], [8193]])
def test_bitpack_matches_oracle(cuda, bits, shape):
    from kvserve_amd import ops

    g = torch.Generator().manual_seed(bits * 1000 + len(shape))
    x = torch.randint(2 ** bits, shape, generator=g, dtype=torch.uint8)
    packed = ops.bitpack_encode(x.to(cuda), bits)
    ref = kp.bitpack_encode(x.numpy(), bits)
    assert packed.numel() == 16 + (x.numel() * bits + 7) // 8
    assert np.array_equal(packed.cpu().numpy(), ref)
    back = ops.bitpack_decode(packed, list(shape), bits)
    assert torch.equal(back.cpu(), x)


def test_bitpack_large_and_unaligned(cuda):
    from kvserve_amd import ops

    g = torch.Generator().manual_seed(7)
    x = torch.randint(16, ((1 << 22) + 5,), generator=g, dtype=torch.uint8)
    xd = x.to(cuda)
    for view in (xd, xd[1:], xd[3:-1]):
        p = ops.bitpack_encode(view, 4)
        assert np.array_equal(p.cpu().numpy(), cbitpack.encode(view.cpu().numpy(), 4))
        assert torch.equal(ops.bitpack_decode(p, [view.numel()], 4), view)
        # payload view at an odd offset: decode from a misaligned pointer
        buf = torch.empty(p.numel() + 1, dtype=torch.uint8, device=cuda)
        buf[1:] = p
        assert torch.equal(ops.bitpack_decode(buf[1:], [view.numel()], 4), view)


def test_bitpack_device_errors_are_raised(cuda):
    from kvserve_amd import ops

    with pytest.raises(RuntimeError, match="symbol exceeds bitpack_bits"):
        ops.bitpack_encode(torch.tensor([255], dtype=torch.uint8, device=cuda), 3)
    p = ops.bitpack_encode(torch.tensor([1], dtype=torch.uint8, device=cuda), 3)
    p[0] = 0
    with pytest.raises(RuntimeError, match="invalid bitpack header"):
        ops.bitpack_decode(p, [1], 3)
    with pytest.raises(ValueError, match="length"):
        ops.bitpack_decode(p[:-1], [1], 3)
    with pytest.raises(ValueError, match="nonnegative"):
        ops.bitpack_decode(p, [-1], 3)
    with pytest.raises(TypeError, match="uint8"):
        ops.bitpack_encode(torch.zeros(1, device=cuda), 3)
    with pytest.raises(ValueError, match="CUDA"):
        ops.bitpack_encode(torch.zeros(1, dtype=torch.uint8), 3)


# ------------------------------------------------------------------ gather / scatter / hadamard
def test_gather_scatter_bit_exact(cuda):
    from kvserve_amd import ops

    g = torch.Generator().manual_seed(11)
    pool = torch.randint(-30000, 30000, (2, 40, 16, 8, 128), generator=g, dtype=torch.int16).view(torch.bfloat16)
    ids = [5, 0, 39, 17, 3]
    got = ops.gather_blocks(pool.to(cuda), ids)
    assert torch.equal(got.cpu().view(torch.int16), pool[:, ids].view(torch.int16))
    dst = torch.zeros_like(pool).to(cuda)
    ops.scatter_blocks(dst, got, ids + [7, 8])  # more ids than payload blocks: overlap only
    ref = torch.zeros_like(pool)
    ref[:, ids] = pool[:, ids]
    assert torch.equal(dst.cpu().view(torch.int16), ref.view(torch.int16))
    with pytest.raises(IndexError):
        ops.gather_blocks(pool.to(cuda), [40])


@pytest.mark.parametrize("shape", [(40, 2, 16, 8, 128), (33, 2, 16, 4, 64), (12, 2, 3, 8)])
def test_gather_scatter_kv_adjacent_bit_exact(cuda, shape):
    """The [num_blocks, 2, ...] branch (kv_utils.py:76-79, :108-114) on the HIP kernels:
    kv[ids] and kv[ids[:nb]] = payload, directly and through the connector's helpers."""
    from kvserve_amd import ops
    from kvserve_amd.connector.kv_utils import extract_kv_from_layer_by_blocks, inject_kv_into_layer_by_blocks

    g = torch.Generator().manual_seed(shape[0])
    pool = torch.randint(-30000, 30000, shape, generator=g, dtype=torch.int16).view(torch.bfloat16)
    P = shape[0]
    ids = [5, 0, P - 1, 7, 3]
    print(f"kv-adjacent gather/scatter {shape}", flush=True)
    got = ops.gather_blocks(pool.to(cuda), ids)
    assert got.shape == (len(ids),) + shape[1:]
    assert torch.equal(got.cpu().view(torch.int16), pool[ids].view(torch.int16))
    via = extract_kv_from_layer_by_blocks(pool.to(cuda), ids)
    assert torch.equal(via.cpu().view(torch.int16), pool[ids].view(torch.int16))
    out = torch.empty_like(got)
    assert ops.gather_blocks(pool.to(cuda), torch.tensor(ids, device=cuda), out=out) is out
    assert torch.equal(out.view(torch.int16), got.view(torch.int16))  # bit patterns (NaNs included)
    dst = torch.zeros_like(pool).to(cuda)
    ops.scatter_blocks(dst, got, ids + [1, 2])  # more ids than payload blocks: overlap only
    ref = torch.zeros_like(pool)
    ref[ids] = pool[ids]
    assert torch.equal(dst.cpu().view(torch.int16), ref.view(torch.int16))
    dst2 = torch.zeros_like(pool).to(cuda)
    inject_kv_into_layer_by_blocks(dst2, got, ids)
    assert torch.equal(dst2.cpu().view(torch.int16), ref.view(torch.int16))
    assert extract_kv_from_layer_by_blocks(pool.to(cuda), []).shape == (0,) + shape[1:]
    with pytest.raises(IndexError):
        ops.gather_blocks(pool.to(cuda), [P])
    with pytest.raises(ValueError):
        ops.scatter_blocks(dst, got[:, :1], ids)  # not a [nb, 2, ...] payload


@pytest.mark.parametrize("D,H", [(64, 8), (128, 8), (96, 8), (256, 4), (80, 6), (16, 3), (224, 2), (100, 8), (70, 5),
                                 (6, 3), (108, 2)])
def test_hadamard_unit_matches_oracle(cuda, D, H):
    """Power-of-two D and D split into power-of-two chunks (hadamard_func.py:50-103):
    bit-exact with the oracle, whose chunked transform is pinned to the Sylvester
    matrices (tests/test_oracle.py)."""
    from kvserve_amd import ops

    g = torch.Generator().manual_seed(D)
    x = torch.randn((3, 16, H, D), generator=g).to(torch.bfloat16)
    seed, layer = 0xC0FEBABE, 5
    print(f"hadamard unit D={D} H={H}", flush=True)
    y = ops.hadamard(x.to(cuda), layer, seed)
    sg = kp.rademacher_signs(seed, layer, H, D)
    ref = kp.hadamard_forward(_bits(x), sg)
    assert np.array_equal(_bits(y), ref)
    z = ops.hadamard(y, layer, seed, inverse=True)
    assert np.array_equal(_bits(z), kp.hadamard_inverse(ref, sg))


# ------------------------------------------------------------------ fused paged codec
def _run_parity(wl, layout="permuted", transform=True):
    from kvserve_amd.engine import FusedKVCodec, check_packet

    req = wl.requests[0]
    codec = FusedKVCodec(wl.num_heads, wl.head_dim, wl.block_size, wl.bits, wl.seed, transform=transform,
                         layout=layout)
    packet = codec.compress(req.pools, req.block_ids, req.profiles, req.layer_ids)
    check_packet(packet)
    pools_np = [_bits(p) for p in req.pools]
    ids = req.block_ids.cpu().numpy().tolist()
    oprof = [_oracle_profile(p) for p in req.profiles]
    chunks = kp.compress_request(pools_np, ids, oprof, wl.seed, wl.bits, transform=transform, layout=layout)
    assert len(chunks) == len(packet.streams)
    for ch, st in zip(chunks, packet.streams):
        got = st.cpu().numpy()
        assert np.array_equal(got[:16], ch.stream[:16]), "header"
        sym = cbitpack.decode(got, ch.symbols.size, wl.bits)
        dmax, frac = sym_diff(sym, ch.symbols.reshape(-1))
        assert dmax <= 1 and frac <= SYM_MISMATCH_FRAC, (dmax, frac)
        for i, l in enumerate(range(ch.start, ch.stop)):
            m = ch.metas[i]
            km = packet.kmeta[l].float().cpu().numpy()
            assert np.array_equal(km[0], m.kmin) and np.array_equal(km[1], m.kscale)
            G = m.vmin.shape[0]
            vm = packet.vmeta[l].float().cpu().numpy()
            assert np.array_equal(vm[0, :G], m.vmin) and np.array_equal(vm[1, :G], m.vscale)
    return codec, packet, chunks, pools_np, ids, oprof


def test_fused_config1_compress_matches_oracle(cuda):
    from kvserve_amd.workloads import make_config1

    _run_parity(make_config1(device=cuda))


@pytest.mark.parametrize("layout,transform", [("native", True), ("permuted", False)])
def test_fused_layout_and_no_transform(cuda, layout, transform):
    """Compress against the oracle, then decompress against the oracle's decode of the
    GPU's own streams and metadata: bit-exact without the transform, bf16 neighbours
    (the inverse transform's fp32 summation order) on <= 1e-3 of the elements with it."""
    from kvserve_amd.workloads import make_config1

    wl = make_config1(device=cuda)
    codec, packet, chunks, pools_np, ids, oprof = _run_parity(wl, layout=layout, transform=transform)
    req = wl.requests[0]
    dst = [torch.zeros_like(p) for p in req.pools]
    codec.decompress(packet, dst, req.block_ids)
    torch.cuda.synchronize()
    own = []
    for ch, st in zip(chunks, packet.streams):
        metas = []
        for i, l in enumerate(range(ch.start, ch.stop)):
            km = packet.kmeta[l].float().cpu().numpy()
            vm = packet.vmeta[l].float().cpu().numpy()
            G = ch.metas[i].vmin.shape[0]
            metas.append(kp.LayerMeta(km[0], km[1], vm[0, :G], vm[1, :G]))
        own.append(kp.Chunk(ch.start, ch.stop, ch.symbols, st.cpu().numpy(), metas))
    ref = [np.zeros_like(p) for p in pools_np]
    kp.decompress_request(own, ref, ids, oprof, wl.seed, wl.bits, transform=transform, layout=layout)
    for l, d in enumerate(dst):
        a = _bits(d)[:, ids].view(np.int16).astype(np.int32)
        b = ref[l][:, ids].view(np.int16).astype(np.int32)
        diff = a != b
        n = int(np.count_nonzero(diff))
        if not transform:
            assert n == 0, (l, n)
        elif n:
            assert np.all((a[diff] ^ b[diff]) >= 0) and np.abs(a[diff] - b[diff]).max() <= 1, l
        assert n <= 1e-3 * a.size, (l, n)


def test_fused_config1_roundtrip_matches_oracle(cuda):
    from kvserve_amd.workloads import make_config1

    wl = make_config1(device=cuda)
    codec, packet, chunks, pools_np, ids, oprof = _run_parity(wl)
    # decompress into a pool of sentinels larger than the request: untouched blocks stay
    req = wl.requests[0]
    P = req.pools[0].shape[1] + 8
    dst = torch.full((2, P, 16, 8, 128), 7.0, dtype=torch.bfloat16, device=cuda)
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(3))[: len(ids)]
    codec.decompress(packet, [dst], perm.to(torch.int32))
    torch.cuda.synchronize()
    ref_pool = np.full((2, P, 16, 8, 128), kp.f32_to_bf16(np.float32([7.0]))[0], np.uint16)
    kp.decompress_request(chunks, [ref_pool], perm.tolist(), oprof, wl.seed, wl.bits)
    got = _bits(dst)
    untouched = np.setdiff1d(np.arange(P), perm.numpy())
    assert np.array_equal(got[:, untouched], ref_pool[:, untouched])
    x_ref = kp.bf16_to_f32(ref_pool[:, perm.numpy()])
    x = kp.bf16_to_f32(got[:, perm.numpy()])
    for part in range(2):
        rel = np.abs(x[part] - x_ref[part]).max() / np.abs(x_ref[part]).max()
        assert rel <= DEQ_REL_TOL, rel
    # with symbols identical the decoded KV is identical too
    exact = np.mean(got[:, perm.numpy()] == ref_pool[:, perm.numpy()])
    assert exact > 0.999


def test_fused_multi_chunk_and_many_layers(cuda):
    """Layers split into several streams (chunk_layers=2), each with its own header."""
    from kvserve_amd.engine import FusedKVCodec, check_packet
    from kvserve_amd.workloads import kv_blocks, llama_row_profiles

    g = torch.Generator().manual_seed(21)
    L, B, S, H, D = 5, 9, 16, 8, 128
    pools = [torch.zeros((2, 20, S, H, D), dtype=torch.bfloat16) for _ in range(L)]
    ids = torch.randperm(20, generator=g)[:B]
    for p in pools:
        p[:, ids] = kv_blocks(g, B, S, H, D)
    prof = llama_row_profiles(L, H, levels=(12, 8, 6, 4), ratio=0.8)
    codec = FusedKVCodec(H, D, S, 4, 1234)
    packet = codec.compress([p.to(cuda) for p in pools], ids.to(torch.int32), prof, chunk_layers=2)
    check_packet(packet)
    assert packet.chunks == [(0, 2), (2, 4), (4, 5)]
    # layer ids of later chunks continue the global numbering (sign seeds)
    chunks_ref = kp.compress_request([_bits(p) for p in pools], ids.tolist(), [_oracle_profile(p) for p in prof],
                                     1234, 4, chunks=packet.chunks)
    for st, ch in zip(packet.streams, chunks_ref):
        got = st.cpu().numpy()
        assert np.array_equal(got[:16], ch.stream[:16])
        sym = cbitpack.decode(got, ch.symbols.size, 4)
        dmax, frac = sym_diff(sym, ch.symbols.reshape(-1))
        assert dmax <= 1 and frac <= SYM_MISMATCH_FRAC
    dst = [torch.zeros_like(p).to(cuda) for p in pools]
    codec.decompress(packet, dst, ids.to(torch.int32))
    torch.cuda.synchronize()
    for l in range(L):
        x = dst[l][:, ids.long()].float().cpu()
        x0 = pools[l][:, ids].float()
        cos = torch.nn.functional.cosine_similarity(x.flatten(), x0.flatten(), dim=0)
        assert cos > 0.9


def test_fused_bad_header_leaves_pool_untouched(cuda):
    from kvserve_amd.engine import FusedKVCodec, check_packet
    from kvserve_amd.workloads import make_config1

    wl = make_config1(device=cuda)
    req = wl.requests[0]
    codec = FusedKVCodec(8, 128, 16, 4, wl.seed)
    packet = codec.compress(req.pools, req.block_ids, req.profiles)
    check_packet(packet)
    packet.streams[0][4] = 5  # wrong bit width in the header
    dst = torch.zeros_like(req.pools[0])
    codec.decompress(packet, [dst], req.block_ids)
    with pytest.raises(RuntimeError, match="invalid bitpack header"):
        check_packet(packet)
    assert int(torch.count_nonzero(dst.view(torch.int16))) == 0


def test_device_block_ids_checked_on_the_device(cuda):
    """A device block table is checked by the plan's first launch instead of a host
    synchronization: an id outside the cache (or negative) is reported as the
    IndexError a host table raises, no kernel touches the caches, and a decompress
    with such a table leaves them as they were; batches report it for all requests."""
    from kvserve_amd.engine import FusedKVCodec, check_packet
    from kvserve_amd.workloads import make_config1

    wl = make_config1(device=cuda)
    req = wl.requests[0]
    fc = FusedKVCodec(wl.num_heads, wl.head_dim, wl.block_size, wl.bits, wl.seed)
    P = req.pools[0].shape[1]
    good = fc.plan_compress(req.pools, req.block_ids, req.profiles)
    assert good.launches() == ["kvmi_check_block_ids", "kvmi_kstats_paged", "kvmi_encode_paged"]
    good.run()
    good.check_errors()
    assert good.launches() == ["kvmi_kstats_paged", "kvmi_encode_paged"]  # checked once per plan
    for bad_id in (P, -1):
        bad = req.block_ids.clone()
        bad[1] = bad_id
        print(f"device block table with id {bad_id}", flush=True)
        plan = fc.plan_compress(req.pools, bad, req.profiles)  # builds without a host check
        plan.run()
        with pytest.raises(IndexError, match="block id outside the KV cache"):
            check_packet(plan.packet)
        before = [p.clone() for p in req.pools]
        d = fc.plan_decompress(good.packet, req.pools, bad)
        d.run()
        with pytest.raises(IndexError):
            d.check_errors()
        assert all(torch.equal(a.view(torch.int16), b.view(torch.int16)) for a, b in zip(before, req.pools))
    # one bad request in a batch: the batch's shared error word reports it
    bad = req.block_ids.clone()
    bad[0] = P + 5
    bp = fc.plan_compress_batch([(req.pools, req.block_ids, req.profiles), (req.pools, bad, req.profiles)])
    bp.run()
    with pytest.raises(IndexError):
        bp.check_errors()
    # a good device table after all this still round-trips
    d = fc.plan_decompress(good.packet, req.pools, req.block_ids)
    d.run()
    d.check_errors()
