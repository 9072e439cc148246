"""One-pass compress (kvmi_compress_paged with a schedule, K read once) against the
two-pass kernels (kvmi_kstats_paged + kvmi_encode_paged) through the C-ABI: packed
streams, K and V metadata must be identical, bit for bit, on every call, with new pool
contents (a smaller K range) before each repeated call, so keys or barrier flags left by
an earlier call would show.  The two-pass path is pinned to the oracle by
test_gpu_codec.py and test_gpu_configs.py; test_one_pass_matches_oracle checks the
one-pass output against the oracle directly, and test_gpu_configs.py runs the
benchmark configurations (full size) through both paths against the oracle."""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _requests(g, lens_blocks, L, H, D, S, P, levels):
    from kvserve_amd.profiles import per_head_profile
    from kvserve_amd.workloads import kv_blocks

    pools = [torch.zeros((2, P, S, H, D), dtype=torch.bfloat16) for _ in range(L)]
    perm = torch.randperm(P, generator=g)
    reqs, off = [], 0
    for B in lens_blocks:
        ids = perm[off:off + B]
        off += B
        for p in pools:
            p[:, ids] = kv_blocks(g, B, S, H, D)
        kl = [[levels[int(i)] for i in torch.randint(0, len(levels), (H,), generator=g)] for _ in range(L)]
        vl = [[levels[int(i)] for i in torch.randint(0, len(levels), (H,), generator=g)] for _ in range(L)]
        reqs.append((ids.to(torch.int32), [per_head_profile(kl[l], vl[l]) for l in range(L)]))
    return pools, reqs


def _outputs(plan):
    """Streams, K metadata and the V metadata rows each layer uses (a layer with fewer
    V groups than the plan's table leaves the other rows unwritten, on either path)."""
    pks = plan.packets if hasattr(plan, "packets") else [plan.packet]
    out = []
    for pk in pks:
        vm = torch.cat([pk.vmeta[l, :, :p.num_v_groups()].reshape(-1) for l, p in enumerate(pk.profiles)])
        out.append(([s.clone() for s in pk.streams], pk.kmeta.clone(), vm))
    return out


def _assert_same(a, b):
    assert len(a) == len(b)
    for (sa, ka, va), (sb, kb, vb) in zip(a, b):
        for x, y in zip(sa, sb):
            assert torch.equal(x, y)
        assert torch.equal(ka.view(torch.int16), kb.view(torch.int16))
        assert torch.equal(va.view(torch.int16), vb.view(torch.int16))


def _compare(cuda, pools, reqs, H, D, S, bits, layout="permuted", runs=3, expect_one_pass=True):
    from kvserve_amd.engine import FusedKVCodec

    pools = [p.to(cuda) for p in pools]
    args = [(pools, ids.to(cuda), prof) for ids, prof in reqs]
    ref_codec = FusedKVCodec(H, D, S, bits, 0xC0FEBABE, layout=layout, compress_path="two_pass")
    one_codec = FusedKVCodec(H, D, S, bits, 0xC0FEBABE, layout=layout, compress_path="one_pass")
    ref = ref_codec.plan_compress_batch(args)
    one = one_codec.plan_compress_batch(args)
    if expect_one_pass:
        assert one.launches() == ["kvmi_check_block_ids", "kvmi_compress_paged"]
    else:  # the one-pass kernel does not take these jobs: the plan runs the two passes
        assert one.workspace is None
        assert one.launches() == ["kvmi_check_block_ids", "kvmi_kstats_paged", "kvmi_encode_paged"]
    for k in range(runs):
        if k:  # new contents with half the range (exact in bf16): stale keys of call k-1 are larger
            for p in pools:
                p.mul_(-0.5)
        ref.run()
        ref.check_errors()
        want = _outputs(ref)
        for j, pk in enumerate(one.packets):  # poison the outputs: every byte must be written again
            for s in pk.streams:
                s.fill_(0xA5)
            if pk.num_blocks:  # a request without blocks keeps its K metadata (C-ABI contract)
                pk.kmeta.view(torch.int16).fill_(-1)
            else:
                pk.kmeta.copy_(ref.packets[j].kmeta)
        one.run()
        one.check_errors()
        _assert_same(_outputs(one), want)
    if expect_one_pass:  # the device epoch counts the one-pass launches
        assert _epoch(one) == runs
    torch.cuda.synchronize()


def _epoch(plan) -> int:
    """The call counter in a plan's workspace (its offset: the schedule header's int64 at
    byte 64)."""
    off = int(np.frombuffer(plan.schedule[64:72].tobytes(), dtype=np.int64)[0])
    return int(plan.workspace[off:off + 4].view(torch.int32).item())


@pytest.mark.parametrize("H,S,D,bits,layout", [
    (8, 16, 128, 4, "permuted"),
    (8, 16, 128, 4, "native"),
    (8, 16, 64, 3, "permuted"),   # two tiles per wave
    (4, 16, 128, 5, "permuted"),
    (2, 16, 128, 4, "native"),
    (1, 32, 128, 2, "permuted"),
    (8, 32, 64, 6, "permuted"),
])
def test_one_pass_equals_two_pass_on_ragged_batches(cuda, H, S, D, bits, layout):
    g = torch.Generator().manual_seed(H * 131 + S * 7 + D + bits)
    top = 2 ** bits - 1
    pools, reqs = _requests(g, [9, 0, 3, 40, 1], 3, H, D, S, 64, (top, max(2, top - 2)))
    print(f"one-pass H={H} S={S} D={D} bits={bits} {layout}", flush=True)
    _compare(cuda, pools, reqs, H, D, S, bits, layout)


def test_one_pass_with_levels_above_128(cuda):
    g = torch.Generator().manual_seed(5)
    pools, reqs = _requests(g, [7, 12], 2, 8, 128, 16, 32, (200, 255))
    _compare(cuda, pools, reqs, 8, 128, 16, 8)


def test_one_pass_config2_shape_whole_grid(cuda):
    """32 layers x 512 blocks of 16 tokens x 8 heads x 128: each job spans the whole
    grid (one group), as on the benchmark's configuration."""
    from kvserve_amd.workloads import kv_blocks, llama_row_profiles

    g = torch.Generator().manual_seed(2)
    L, B, S, H, D = 32, 512, 16, 8, 128
    pools = []
    for _ in range(L):
        pools.append(kv_blocks(g, B, S, H, D))
    ids = torch.randperm(B, generator=g).to(torch.int32)
    prof = llama_row_profiles(L, H)
    print("one-pass config-2 shape", flush=True)
    _compare(cuda, pools, [(ids, prof)], H, D, S, 4, runs=2)


def test_job_too_large_for_one_pass_falls_back(cuda):
    """A job with more tokens per head than the grid's registers hold (8 head-tiles of 32
    tokens per workgroup: 65,536 on 256 CUs) gets no schedule: the plan runs the two
    passes."""
    g = torch.Generator().manual_seed(9)
    pools, reqs = _requests(g, [4100], 1, 8, 128, 16, 4100, (16, 16))
    _compare(cuda, pools, reqs, 8, 128, 16, 4, runs=1, expect_one_pass=False)


def test_one_pass_largest_job_the_grid_holds(cuda):
    """4096 blocks of 16 tokens: each head's K fills every workgroup of a 256-CU grid."""
    g = torch.Generator().manual_seed(19)
    pools, reqs = _requests(g, [4096], 1, 8, 128, 16, 4096, (16, 12))
    _compare(cuda, pools, reqs, 8, 128, 16, 4, runs=2)


def test_workspace_contract_through_the_c_abi(cuda):
    """Direct C-ABI use: the host schedule, a workspace holding its image and zeros, two
    calls with the same workspace, and the host-side argument checks."""
    from kvserve_amd import _lib
    from kvserve_amd.engine import FusedKVCodec

    g = torch.Generator().manual_seed(3)
    pools, reqs = _requests(g, [6], 2, 8, 128, 16, 16, (16, 12))
    pools = [p.to(cuda) for p in pools]
    codec = FusedKVCodec(8, 128, 16, 4, 0xC0FEBABE, compress_path="two_pass")
    plan = codec.plan_compress(pools, reqs[0][0].to(cuda), reqs[0][1])
    plan.run()
    want = _outputs(plan)
    lib = _lib.load()
    geo = ctypes.byref(plan.geo)
    nb = np.full(plan.num_jobs, plan.max_blocks, dtype=np.int32)
    n = lib.kvmi_compress_schedule(geo, nb.ctypes.data, plan.num_jobs, None, 0)
    assert n > 0
    img = np.zeros(n, dtype=np.uint8)
    assert lib.kvmi_compress_schedule(geo, nb.ctypes.data, plan.num_jobs, img.ctypes.data, n - 1) == _lib.EINVAL
    assert lib.kvmi_compress_schedule(geo, nb.ctypes.data, plan.num_jobs, img.ctypes.data, n) == n
    total = lib.kvmi_compress_workspace_bytes(img.ctypes.data)
    assert total >= n
    ws = torch.zeros(total, dtype=torch.uint8, device=cuda)
    ws[:n].copy_(torch.from_numpy(img))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for k in range(2):
        rc = lib.kvmi_compress_paged(geo, plan.jobs.data_ptr(), plan.num_jobs, plan.max_blocks, img.ctypes.data,
                                     ws.data_ptr(), plan.err.data_ptr(), stream)
        assert rc == 0
        plan.check_errors()
        _assert_same(_outputs(plan), want)
    # misaligned workspace, a schedule of other jobs: rejected on the host
    assert lib.kvmi_compress_paged(geo, plan.jobs.data_ptr(), plan.num_jobs, plan.max_blocks, img.ctypes.data,
                                   ws.data_ptr() + 16, plan.err.data_ptr(), stream) == _lib.EINVAL
    assert lib.kvmi_compress_paged(geo, plan.jobs.data_ptr(), plan.num_jobs - 1, plan.max_blocks, img.ctypes.data,
                                   ws.data_ptr(), plan.err.data_ptr(), stream) == _lib.EINVAL
    torch.cuda.synchronize()
    # a schedule built for fewer blocks than the jobs hold: flagged on the device
    nb_short = nb - 1
    n2 = lib.kvmi_compress_schedule(geo, nb_short.ctypes.data, plan.num_jobs, None, 0)
    img2 = np.zeros(n2, dtype=np.uint8)
    assert lib.kvmi_compress_schedule(geo, nb_short.ctypes.data, plan.num_jobs, img2.ctypes.data, n2) == n2
    ws2 = torch.zeros(lib.kvmi_compress_workspace_bytes(img2.ctypes.data), dtype=torch.uint8, device=cuda)
    ws2[:n2].copy_(torch.from_numpy(img2))
    plan.err.zero_()
    assert lib.kvmi_compress_paged(geo, plan.jobs.data_ptr(), plan.num_jobs, plan.max_blocks, img2.ctypes.data,
                                   ws2.data_ptr(), plan.err.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert int(plan.err.item()) == _lib.ERR_SCHEDULE
    plan.err.zero_()


@pytest.mark.parametrize("H,S,D,bits", [(8, 16, 128, 4), (4, 16, 64, 3)])
def test_one_pass_matches_oracle(cuda, H, S, D, bits):
    """The one-pass output against the CPU oracle directly (symbols within the north-star
    bound, K and V metadata exact, round trip within 1e-2)."""
    from kvserve_amd.engine import FusedKVCodec, check_packet
    from kvserve_amd.profiles import section_profile
    from kvserve_amd.workloads import kv_blocks
    from tests.test_gpu_configs import _bits, _check_layer

    g = torch.Generator().manual_seed(H * 7 + D + bits)
    L, B, P = 3, 11, 32
    pools = [torch.zeros((2, P, S, H, D), dtype=torch.bfloat16) for _ in range(L)]
    ids = torch.randperm(P, generator=g)[:B]
    for p in pools:
        p[:, ids] = kv_blocks(g, B, S, H, D)
    top = 2 ** bits - 1
    prof = [section_profile([bool(v) for v in torch.randint(0, 2, (H,), generator=g)], top, top,
                            max(2, top - 2), max(2, top - 2)) for _ in range(L)]
    pools = [p.to(cuda) for p in pools]
    dev_ids = ids.to(torch.int32).to(cuda)
    codec = FusedKVCodec(H, D, S, bits, 0xC0FEBABE, compress_path="one_pass")
    plan = codec.plan_compress(pools, dev_ids, prof)
    assert plan.launches()[-1] == "kvmi_compress_paged"
    plan.run()
    check_packet(plan.packet)
    assert plan.workspace is not None and _epoch(plan) == 1
    dst = [torch.zeros_like(p) for p in pools]
    codec.decompress(plan.packet, dst, dev_ids)
    torch.cuda.synchronize()
    for l in range(L):
        _check_layer(plan.packet, l, _bits(pools[l][:, dev_ids.long()]), _bits(dst[l][:, dev_ids.long()]))


def test_one_pass_plan_captured_in_graph(cuda):
    """The epoch lives in the workspace and a kernel of the plan advances it, so a graph
    captured from a one-pass plan's run() replays correctly: every replay, with new pool
    contents each time (a smaller range, so stale keys would be larger), equals the two
    passes run eagerly on the same contents."""
    from kvserve_amd.engine import FusedKVCodec

    g = torch.Generator().manual_seed(23)
    pools, reqs = _requests(g, [40, 9], 2, 8, 128, 16, 64, (16, 12))
    pools = [p.to(cuda) for p in pools]
    args = [(pools, ids.to(cuda), prof) for ids, prof in reqs]
    ref = FusedKVCodec(8, 128, 16, 4, 0xC0FEBABE, compress_path="two_pass").plan_compress_batch(args)
    one = FusedKVCodec(8, 128, 16, 4, 0xC0FEBABE, compress_path="one_pass").plan_compress_batch(args)
    one.run()  # the first run checks the block tables (outside the graph)
    one.check_errors()
    assert one.launches() == ["kvmi_compress_paged"]
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(graph, stream=st):
            one.run()
    torch.cuda.synchronize()
    for k in range(3):
        for p in pools:
            p.mul_(-0.5)
        ref.run()
        ref.check_errors()
        want = _outputs(ref)
        for pk in one.packets:
            for s in pk.streams:
                s.fill_(0xA5)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        one.check_errors()
        _assert_same(_outputs(one), want)
    assert _epoch(one) == 4  # the eager run and three replays (capturing runs nothing)
