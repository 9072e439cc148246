"""CPU pins of the rANS oracle (oracle/rans.c; its header comment is the stream
format).  The codec stage's reference is nvCOMP ANS (kvserve_codec.py:57-64), a
closed library with an unpublished format, so the pins are closed forms and
special cases computed here without the oracle's arithmetic:

  - one symbol: the table is {s: 4096}, states never move, no words;
  - two equiprobable symbols (f = 2048 each): encoding inserts the symbol bit at
    bit 11 of the state and emits the low 16 bits once the state reaches 2^31 --
    a bit-insertion model that fixes the sub-block / lane / step symbol order, the
    word order and the state and count layout;
  - normalised frequencies of a hand-counted block;
  - incompressible bytes: every block stored raw, byte for byte;
  - the coded size against the empirical entropy of each block;
  - round trips at every width and at the block edges; corruption is detected.
"""

import numpy as np
import pytest

from oracle import crans

MAGIC = 0x5352564B


def _u32(a, off):
    return int(np.frombuffer(a[off:off + 4].tobytes(), np.uint32)[0])


def _u64(a, off):
    return int(np.frombuffer(a[off:off + 8].tobytes(), np.uint64)[0])


def _parse(stream):
    nblk = _u32(stream, 12)
    payload = 32 + 8 * nblk
    offs = [_u64(stream, 32 + 8 * b) for b in range(nblk)] + [_u64(stream, 24)]
    return nblk, [stream[payload + offs[b]:payload + offs[b + 1]] for b in range(nblk)]


def _lane_symbols(sym_block, sub, lane):
    """Symbols of `lane` of sub-block `sub` in step order t = 0..255:
    sub*16384 + (t/32)*2048 + lane*32 + t%32."""
    t = np.arange(256)
    return sym_block[sub * 16384 + (t // 32) * 2048 + lane * 32 + t % 32]


def test_header_and_single_symbol_closed_form():
    w, n = 4, 65536
    st = crans.encode(np.full(n, 9, np.uint8), w)
    assert _u32(st, 0) == MAGIC and list(st[4:8]) == [2, w, 12, 8]
    assert _u32(st, 8) == 65536 and _u32(st, 12) == 1 and _u64(st, 16) == n
    nblk, blocks = _parse(st)
    (blk,) = blocks
    assert _u32(blk, 0) == 0                                        # rANS, no words in sub-block 0
    freq = np.frombuffer(blk[4:4 + 32].tobytes(), np.uint16)
    assert freq[9] == 4096 and freq.sum() == 4096
    counts = np.frombuffer(blk[36:48].tobytes(), np.uint32)         # sub-blocks 1..3
    states = np.frombuffer(blk[48:48 + 1024].tobytes(), np.uint32)  # 4 sub-blocks x 64 lanes
    assert not counts.any() and (states == 1 << 16).all() and blk.size == 4 + 32 + 12 + 1024
    assert st.size == 32 + 8 + 1072


def _bit_insert_model(sym_block, sub):
    """f = 2048 for both symbols: x -> (x >> 11) << 12 | s << 11 | (x & 2047), emit
    the low 16 bits when x >= 2^31 (encoding runs t = 255..0, lanes in order)."""
    x = np.full(64, 1 << 16, np.uint64)
    steps = []
    lanes = [_lane_symbols(sym_block, sub, i) for i in range(64)]
    for t in range(255, -1, -1):
        emitted = []
        for i in range(64):
            s = int(lanes[i][t])
            if x[i] >= (1 << 31):
                emitted.append(int(x[i]) & 0xFFFF)
                x[i] >>= np.uint64(16)
            x[i] = ((x[i] >> np.uint64(11)) << np.uint64(12)) | np.uint64(s << 11) | (x[i] & np.uint64(2047))
        steps.append(emitted)
    words = [wd for e in reversed(steps) for wd in e]
    return x.astype(np.uint32), np.array(words, np.uint16)


def test_two_equiprobable_symbols_bit_insertion():
    # symbols 0 and 1 of a 2-bit alphabet: raw costs 2 bits, rANS 1 bit per symbol
    rng = np.random.default_rng(5)
    s = np.zeros(65536, np.uint8)
    s[rng.permutation(65536)[:32768]] = 1
    st = crans.encode(s, 2)
    _, (blk,) = _parse(st)
    tag = _u32(blk, 0)
    assert tag & 1 == 0
    counts = [tag >> 1] + [int(c) for c in np.frombuffer(blk[12:24].tobytes(), np.uint32)]
    freq = np.frombuffer(blk[4:12].tobytes(), np.uint16)
    assert list(freq) == [2048, 2048, 0, 0]
    states = np.frombuffer(blk[24:24 + 1024].tobytes(), np.uint32).reshape(4, 64)
    at = 24 + 1024
    for sub in range(4):
        exp_states, exp_words = _bit_insert_model(s, sub)
        region = (2 * counts[sub] + 3) // 4 * 4
        words = np.frombuffer(blk[at + region - 2 * counts[sub]:at + region].tobytes(), np.uint16)
        assert counts[sub] == exp_words.size
        assert np.array_equal(states[sub], exp_states) and np.array_equal(words, exp_words)
        at += region
    assert at == blk.size
    assert (crans.decode(st, s.size, 2) == s).all()


def test_normalised_frequencies_of_a_hand_counted_block():
    # counts 60000 / 5000 / 536 / 0 of 65536: f = 1 + c * 4093 // 65536 -> 3748, 313, 34,
    # and the remainder 4096 - 4095 = 1 goes to the most frequent symbol
    s = np.concatenate([np.zeros(60000), np.ones(5000), np.full(536, 2)]).astype(np.uint8)
    s = s[np.random.default_rng(1).permutation(s.size)]
    _, (blk,) = _parse(crans.encode(s, 2))
    assert list(np.frombuffer(blk[4:12].tobytes(), np.uint16)) == [3749, 313, 34, 0]


def test_ties_give_the_remainder_to_the_lowest_symbol():
    # 3 symbols of equal count: f = 1 + 21845 * 4093 // 65535 (nb = 65535) each
    s = np.repeat(np.arange(3, dtype=np.uint8), 21845)
    _, (blk,) = _parse(crans.encode(s, 2))
    f = 1 + 21845 * 4093 // 65535
    assert list(np.frombuffer(blk[4:12].tobytes(), np.uint16)) == [f + 4096 - 3 * f, f, f, 0]


def test_incompressible_bytes_are_stored_raw():
    rng = np.random.default_rng(2)
    n = 2 * 65536 + 1000
    s = rng.integers(0, 256, n, dtype=np.uint8)
    st = crans.encode(s, 8)
    nblk, blocks = _parse(st)
    assert nblk == 3
    for b, blk in enumerate(blocks):
        raw = s[b * 65536:(b + 1) * 65536]
        assert _u32(blk, 0) == 1 and np.array_equal(blk[4:4 + raw.size], raw)
        assert blk.size == 4 + (raw.size + 3) // 4 * 4 and not blk[4 + raw.size:].any()
    assert st.size == crans.max_bytes(n, 8)


def test_size_tracks_the_block_entropy():
    rng = np.random.default_rng(3)
    w, blocks = 4, 6
    sym = []
    for b in range(blocks):           # each block its own distribution
        p = rng.dirichlet(np.full(16, 0.3 + b))
        sym.append(rng.choice(16, 65536, p=p).astype(np.uint8))
    s = np.concatenate(sym)
    st = crans.encode(s, w)
    bound = 0.0
    for blk in sym:
        c = np.bincount(blk, minlength=16) / blk.size
        c = c[c > 0]
        bound += -(c * np.log2(c)).sum() * blk.size / 8
    overhead = 32 + blocks * (8 + 4 + 32 + 12 + 1024)
    assert bound <= st.size <= 1.005 * bound + overhead + 2 * 4 * blocks
    assert (crans.decode(st, s.size, w) == s).all()


@pytest.mark.parametrize("w", range(1, 9))
@pytest.mark.parametrize("n", [0, 1, 63, 2047, 65535, 65536, 65537, 3 * 65536 + 17])
def test_round_trip_every_width_and_edge(w, n):
    rng = np.random.default_rng(w * 1000 + n % 997)
    p = rng.dirichlet(np.full(1 << w, 0.5))
    s = rng.choice(1 << w, n, p=p).astype(np.uint8)
    st = crans.encode(s, w)
    assert st.size <= crans.max_bytes(n, w)
    assert (crans.decode(st, n, w) == s).all()


def test_corruption_and_contract_errors():
    rng = np.random.default_rng(4)
    s = rng.choice(8, 70000, p=[0.5, 0.2, 0.1, 0.1, 0.05, 0.03, 0.01, 0.01]).astype(np.uint8)
    st = crans.encode(s, 3)
    nblk = _u32(st, 12)
    bad = st.copy()
    bad[32 + 8 * nblk + 4 + 16 + 12 + 5] ^= 0x40  # a state byte of block 0
    with pytest.raises(ValueError, match="-2"):
        crans.decode(bad, s.size, 3)
    with pytest.raises(ValueError, match="-1"):
        crans.decode(st, s.size, 4)              # width differs from the header
    with pytest.raises(ValueError, match="-1"):
        crans.decode(st[:-4], s.size, 3)         # truncated
    # a receive buffer longer than the stream (its header states the length) decodes
    roomy = np.concatenate([st, np.full(100, 0xAB, np.uint8)])
    assert np.array_equal(crans.decode(roomy, s.size, 3), s)
    # a stated payload near 2^64 must not wrap the length check (head + payload)
    huge = st.copy()
    huge[24:32] = np.frombuffer(np.uint64(2**64 - 8).tobytes(), np.uint8)
    with pytest.raises(ValueError, match="-1"):
        crans.decode(huge, s.size, 3)
    with pytest.raises(ValueError, match="-1"):
        crans.decode(st[:32 + 8 * nblk - 1], s.size, 3)  # offset table cut short
