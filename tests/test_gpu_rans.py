"""rANS codec on the GPU against the CPU oracle (oracle/rans.c), through the C-ABI.

Bar: the GPU stream is byte-equal to the oracle's for the same packed input (same
block tables, states, word order, raw fallbacks, offsets and header), the GPU
decodes both its own and the oracle's streams back to the input bytes, and damaged
streams are reported, not silently decoded."""

import numpy as np
import pytest
import torch

from kvserve_amd import ops
from oracle import crans

pytestmark = pytest.mark.gpu


def _symbols(rng, n, w, kind):
    A = 1 << w
    if kind == "skewed":
        p = rng.dirichlet(np.full(A, 0.4))
        return rng.choice(A, n, p=p).astype(np.uint8)
    if kind == "uniform":
        return rng.integers(0, A, n, dtype=np.uint8)
    if kind == "single":
        return np.full(n, A - 1, np.uint8)
    # mixed: alternate compressible and incompressible blocks, drifting tables
    out = np.empty(n, np.uint8)
    for b, lo in enumerate(range(0, n, 65536)):
        m = min(65536, n - lo)
        if b % 3 == 2:
            out[lo:lo + m] = rng.integers(0, A, m)
        else:
            p = rng.dirichlet(np.full(A, 0.2 + b))
            out[lo:lo + m] = rng.choice(A, m, p=p)
    return out


def _gpu_encode(cuda, s, w):
    body = crans.pack(s, w)
    t = torch.from_numpy(body.copy()).to(cuda) if body.size else torch.empty(0, dtype=torch.uint8, device=cuda)
    return body, ops.rans_encode(t, s.size, w)


CASES = [(w, n, kind) for w in range(1, 9) for n, kind in
         ((1, "skewed"), (2047, "skewed"), (65536, "skewed"), (65537, "mixed"), (5 * 65536 + 333, "mixed"),
          (70000, "uniform"), (131072, "single"))]


@pytest.mark.parametrize("w,n,kind", CASES)
def test_stream_equals_oracle_and_round_trips(cuda, w, n, kind):
    rng = np.random.default_rng(w * 7919 + n)
    s = _symbols(rng, n, w, kind)
    body, st = _gpu_encode(cuda, s, w)
    ref = crans.encode_packed(body, n, w)
    got = st.cpu().numpy()
    assert got.size == ref.size and np.array_equal(got, ref), (w, n, kind)
    back = ops.rans_decode(st, n, w).cpu().numpy()
    assert np.array_equal(back, body)
    back2 = ops.rans_decode(torch.from_numpy(ref).to(cuda), n, w).cpu().numpy()
    assert np.array_equal(back2, body)


def test_empty_input(cuda):
    st = ops.rans_encode(torch.empty(0, dtype=torch.uint8, device=cuda), 0, 4)
    assert np.array_equal(st.cpu().numpy(), crans.encode(np.zeros(0, np.uint8), 4))
    assert ops.rans_decode(st, 0, 4).numel() == 0


def test_large_stream_equals_oracle(cuda):
    """64 Mi symbols at 4 bits with drifting statistics (1024 blocks)."""
    rng = np.random.default_rng(11)
    n, w = 64 << 20, 4
    base = np.clip(np.rint(rng.normal(7.5, 2.2, n)), 0, 15).astype(np.uint8)
    base[rng.random(n) < 0.02] = 15
    body, st = _gpu_encode(cuda, base, w)
    ref = crans.encode_packed(body, n, w)
    assert np.array_equal(st.cpu().numpy(), ref)
    assert np.array_equal(ops.rans_decode(st, n, w).cpu().numpy(), body)
    p = np.bincount(base, minlength=16) / n
    p = p[p > 0]
    entropy_bytes = -(p * np.log2(p)).sum() * n / 8
    # per block: offset, tag, table, 3 counts, 4 x 64 states and word-region padding
    per_block = 8 + 4 + 32 + 12 + 1024 + 4 * 2
    assert entropy_bytes <= st.numel() <= 1.01 * entropy_bytes + 32 + (n // 65536) * per_block


def test_damage_is_reported(cuda):
    rng = np.random.default_rng(12)
    n, w = 3 * 65536, 3
    s = _symbols(rng, n, w, "skewed")
    _, st = _gpu_encode(cuda, s, w)
    nblk = 3
    head = 32 + 8 * nblk
    bad = st.clone()
    bad[head + 4 + 16 + 12 + 1] ^= 0x10             # a state of block 0
    with pytest.raises(RuntimeError, match="corrupt entropy-coded stream"):
        ops.rans_decode(bad, n, w)
    bad = st.clone()
    bad[5] = 4                                       # width byte of the header
    with pytest.raises(RuntimeError, match="invalid bitpack header"):
        ops.rans_decode(bad, n, w)
    with pytest.raises(RuntimeError, match="invalid bitpack header"):
        ops.rans_decode(st, n - 1, w)               # n does not match the header
    bad = st.clone()
    bad[head + 4] ^= 0x01                            # frequency table no longer sums to 4096
    with pytest.raises(RuntimeError, match="corrupt entropy-coded stream"):
        ops.rans_decode(bad, n, w)
    # the stream may sit in a larger buffer (its header states its length); a buffer
    # shorter than the stream is rejected
    roomy = torch.zeros(st.numel() + 4096, dtype=torch.uint8, device=cuda)
    roomy[:st.numel()] = st
    assert torch.equal(ops.rans_decode(roomy, n, w), ops.rans_decode(st, n, w))
    with pytest.raises(RuntimeError, match="invalid bitpack header"):
        ops.rans_decode(st[:-4].clone(), n, w)
    # a stated payload near 2^64 must not wrap the kernel's length check
    bad = st.clone()
    bad[24:32] = torch.from_numpy(np.frombuffer(np.uint64(2**64 - 8).tobytes(), np.uint8).copy()).to(cuda)
    with pytest.raises(RuntimeError, match="invalid bitpack header"):
        ops.rans_decode(bad, n, w)
    with pytest.raises(RuntimeError, match="invalid bitpack header"):
        ops.rans_decode(st[:head - 8].clone(), n, w)   # offset table cut short


@pytest.mark.parametrize("w", [3, 4, 8])
def test_batch_of_streams_equals_oracle(cuda, w):
    """Streams of different lengths and statistics coded by one batched launch (more
    than one launch group of 16) equal the oracle stream by stream and decode back in
    one batched launch."""
    rng = np.random.default_rng(40 + w)
    sizes = [0, 1, 65536, 65537, 3 * 65536 + 5, 2047] + [int(rng.integers(1, 300000)) for _ in range(13)]
    kinds = ["skewed", "mixed", "uniform", "single"]
    syms = [_symbols(rng, n, w, kinds[i % 4]) for i, n in enumerate(sizes)]
    bodies = [crans.pack(s, w) for s in syms]
    items = [(torch.from_numpy(b.copy()).to(cuda) if b.size else torch.empty(0, dtype=torch.uint8, device=cuda), s.size)
             for b, s in zip(bodies, syms)]
    streams = ops.rans_encode_batch(items, w)
    for st, b, s in zip(streams, bodies, syms):
        assert np.array_equal(st.cpu().numpy(), crans.encode_packed(b, s.size, w))
    outs = ops.rans_decode_batch([(st, s.size) for st, s in zip(streams, syms)], w)
    for o, b in zip(outs, bodies):
        assert np.array_equal(o.cpu().numpy(), b)
