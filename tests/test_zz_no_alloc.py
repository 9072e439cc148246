"""kvmi_v3_compress_noalloc (the fused quantizer's compress with its K partials in a
fixed device array instead of a caller workspace) against kvmi_v3_compress, both
called through the C-ABI on the same inputs: quantized symbols, K and V metadata must be
identical.  Two calls in a row, the second smaller than the first, so that the second
runs on the scratch contents the first left behind; and two calls on two streams, the
second enqueued right after the first, which the library must order."""

import ctypes

import pytest
import torch

from kvserve_amd import _lib
from kvserve_amd.profiles import rademacher_sign_bits

pytestmark = pytest.mark.gpu


def _inputs(dev, B, S, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((2, B, S, H, D), generator=g)
    x[0, :, :, :, 3] *= 10.0  # an outlier channel in K
    x = x.to(torch.bfloat16).to(dev).contiguous()
    signs = torch.from_numpy(rademacher_sign_bits(0xC0FEBABE, 3, H, D).view("int32")).to(dev)
    levels = torch.tensor([16.0] * H + [12.0] * H, dtype=torch.float32, device=dev)
    vgroup = torch.zeros(H, dtype=torch.int32, device=dev)
    return x, signs, levels, vgroup


def _outputs(dev, rows, H, D):
    q = torch.empty((2, rows, H, D), dtype=torch.uint8, device=dev)
    kmeta = torch.empty((2, H, D), dtype=torch.float32, device=dev)
    vmeta = torch.empty((2, rows, H), dtype=torch.float32, device=dev)
    return q, kmeta, vmeta


def _run_pair(lib, dev, B, S, H, D, seed):
    rows = B * S
    x, signs, levels, vgroup = _inputs(dev, B, S, H, D, seed)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # the workspace entry point, with a fresh workspace
    q0, k0, v0 = _outputs(dev, rows, H, D)
    ws = torch.empty(int(lib.kvmi_v3_scratch_bytes(rows, H, D)), dtype=torch.uint8, device=dev)
    _lib.check(lib.kvmi_v3_compress(x.data_ptr(), rows, H, D, signs.data_ptr(), levels.data_ptr(), vgroup.data_ptr(),
                                    q0.data_ptr(), k0.data_ptr(), v0.data_ptr(), ws.data_ptr(), stream),
               "kvmi_v3_compress")
    # the no-allocation entry point
    q1, k1, v1 = _outputs(dev, rows, H, D)
    _lib.check(lib.kvmi_v3_compress_noalloc(x.data_ptr(), rows, H, D, signs.data_ptr(), levels.data_ptr(),
                                            vgroup.data_ptr(), q1.data_ptr(), k1.data_ptr(), v1.data_ptr(), stream),
               "kvmi_v3_compress_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(q0, q1)
    assert torch.equal(k0.view(torch.int32), k1.view(torch.int32))
    assert torch.equal(v0.view(torch.int32), v1.view(torch.int32))


def test_noalloc_matches_workspace_entry_point_twice(cuda):
    lib = _lib.load()
    print("noalloc call 1: B=512 S=16 H=8 D=128", flush=True)
    _run_pair(lib, cuda, 512, 16, 8, 128, seed=11)   # 256 K partials (2 MiB of the array)
    print("noalloc call 2: B=3 S=16 H=4 D=64", flush=True)
    _run_pair(lib, cuda, 3, 16, 4, 64, seed=12)      # 3 partials, over the first call's leftovers


def test_noalloc_calls_on_two_streams_are_ordered(cuda):
    """Two large calls on two streams with no order between them given by the caller:
    each must equal the workspace entry point's output (without the library's ordering
    the second call's K partials would overwrite the first's while it still reads them)."""
    lib = _lib.load()
    H, D, rows = 8, 128, 512 * 16
    runs = []
    for seed in (21, 22):
        x, signs, levels, vgroup = _inputs(cuda, 512, 16, H, D, seed)
        runs.append((x, signs, levels, vgroup, _outputs(cuda, rows, H, D), _outputs(cuda, rows, H, D)))
    ws = torch.empty(int(lib.kvmi_v3_scratch_bytes(rows, H, D)), dtype=torch.uint8, device=cuda)
    cur = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for x, signs, levels, vgroup, (q0, k0, v0), _ in runs:
        _lib.check(lib.kvmi_v3_compress(x.data_ptr(), rows, H, D, signs.data_ptr(), levels.data_ptr(),
                                        vgroup.data_ptr(), q0.data_ptr(), k0.data_ptr(), v0.data_ptr(), ws.data_ptr(),
                                        cur), "kvmi_v3_compress")
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]  # default priority
    print("noalloc two streams: B=512 S=16 H=8 D=128 x2", flush=True)
    for st, (x, signs, levels, vgroup, _, (q1, k1, v1)) in zip(streams, runs):
        _lib.check(lib.kvmi_v3_compress_noalloc(x.data_ptr(), rows, H, D, signs.data_ptr(), levels.data_ptr(),
                                                vgroup.data_ptr(), q1.data_ptr(), k1.data_ptr(), v1.data_ptr(),
                                                ctypes.c_void_p(st.cuda_stream)), "kvmi_v3_compress_noalloc")
    torch.cuda.synchronize()
    for _, _, _, _, (q0, k0, v0), (q1, k1, v1) in runs:
        assert torch.equal(q0, q1)
        assert torch.equal(k0.view(torch.int32), k1.view(torch.int32))
        assert torch.equal(v0.view(torch.int32), v1.view(torch.int32))
