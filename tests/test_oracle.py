"""Pins of the CPU oracle (no GPU): golden vectors written by the reference's own
quantizer / manager, closed forms, exhaustive identities and planted mistakes."""

from pathlib import Path

import numpy as np
import pytest
import scipy.linalg

from oracle import cbitpack
from oracle import kvpipe as kp

GOLDEN = Path(__file__).resolve().parent / "golden"


def f(bits):
    return kp.bf16_to_f32(bits)


# ------------------------------------------------------------------ quantizer_func golden
def _check_quantizer_func(quantize=kp.quantize, dequantize=kp.dequantize):
    z = np.load(GOLDEN / "quantizer_func.npz")
    n = len([k for k in z.files if k.endswith("_cfg")])
    for i in range(n):
        mv, ax = z[f"c{i}_cfg"]
        axis = ["channel", "token"][ax]
        sym, mn, sc = quantize(int(mv), f(z[f"c{i}_x"]), axis)
        assert np.array_equal(sym, z[f"c{i}_q"]), i
        assert np.array_equal(kp.f32_to_bf16(mn), z[f"c{i}_min"]), i
        assert np.array_equal(kp.f32_to_bf16(sc), z[f"c{i}_scale"]), i
        deq = dequantize(sym, mn, sc)
        assert np.array_equal(kp.f32_to_bf16(deq), z[f"c{i}_deq"]), i


def test_quantizer_func_matches_reference_golden():
    _check_quantizer_func()


def test_planted_mistake_dropped_rounding_is_caught(monkeypatch):
    """Dropping the bf16 rounding of (x - min) must break the golden comparison."""
    orig = kp.quantize

    def no_round_t(max_value, x, axis):
        dims = {"channel": (0, 1), "token": (2, 3)}[axis]
        mx, mn = x.max(axis=dims, keepdims=True), x.min(axis=dims, keepdims=True)
        sc = kp.section_scale(mn, mx, max_value)
        q = kp.rbf((x - mn) / sc)  # t not rounded
        return np.clip(np.rint(q), 0, max_value).astype(np.uint8), mn, sc

    with pytest.raises(AssertionError):
        _check_quantizer_func(quantize=no_round_t)
    assert kp.quantize is orig


def test_planted_mistake_single_rounding_dequant_is_caught():
    """Fusing the dequant into one rounding (fma-like) must break the golden check."""
    def fused(sym, mn, sc):
        return kp.rbf(sym.astype(np.float32) * sc + mn)

    with pytest.raises(AssertionError):
        _check_quantizer_func(dequantize=fused)


# ------------------------------------------------------------------ KVServeQuantizer golden
def _profiles_for(cfg_idx: int, layer: int):
    scores = np.loadtxt(GOLDEN.parents[1] / "kvserve_amd/compression/config/duo_config/Llama-3.1-8B-Instruct_scores.csv",
                        delimiter=",", dtype=np.float32)
    if cfg_idx == 0:
        m = kp.head_mask_from_scores(scores, 0.3)
        return kp.head_split_profile(m[layer], 16, 16, 16, 16)
    if cfg_idx == 1:
        m = kp.head_mask_from_scores(scores, 0.8)
        return kp.head_split_profile(m[layer], 12, 8, 6, 4)
    lm = kp.layer_mask(scores.shape[0])
    return kp.layer_split_profile(bool(lm[layer]), 8, 12, 12, 6, 6)


@pytest.mark.parametrize("cfg_idx", [0, 1, 2])
@pytest.mark.parametrize("layer", [0, 31])
def test_kvserve_quantizer_matches_reference_golden(cfg_idx, layer):
    z = np.load(GOLDEN / "kvserve_quantizer.npz")
    key = f"q{cfg_idx}_l{layer}"
    prof = _profiles_for(cfg_idx, layer)
    x = f(z[key + "_x"])
    sym, meta = kp.quantize_layer(x, prof)
    assert np.array_equal(sym, z[key + "_q"])
    # metadata sections in the reference dict layout
    low_k = f"{key}_low_key_meta_min"
    if 1 in prof.v.group:
        nl = prof.v.group.count(0)
        secs = {"low": (slice(0, nl), 0), "high": (slice(nl, None), 1)}
    elif low_k in z.files:
        secs = {"low": (slice(None), 0)}
    else:
        secs = {"high": (slice(None), 0)}
    for name, (hs, g) in secs.items():
        kmin = z[f"{key}_{name}_key_meta_min"].reshape(-1)
        assert np.array_equal(kp.f32_to_bf16(meta.kmin[hs]).reshape(-1), kmin)
        assert np.array_equal(kp.f32_to_bf16(meta.kscale[hs]).reshape(-1), z[f"{key}_{name}_key_meta_scale"].reshape(-1))
        assert np.array_equal(kp.f32_to_bf16(meta.vmin[g]), z[f"{key}_{name}_value_meta_min"].reshape(-1))
        assert np.array_equal(kp.f32_to_bf16(meta.vscale[g]), z[f"{key}_{name}_value_meta_scale"].reshape(-1))
    deq = kp.dequantize_layer(sym, meta, prof)
    assert np.array_equal(kp.f32_to_bf16(deq), z[key + "_deq"])


# ------------------------------------------------------------------ quantization axes golden
def test_tensor_axis_matches_reference_golden():
    z = np.load(GOLDEN / "quantizer_axes.npz")
    for i in range(3):
        mv = int(z[f"t{i}_mv"][0])
        sym, mn, sc = kp.quantize(mv, f(z[f"t{i}_x"]), "tensor")
        assert mn.shape == (1, 1, 1, 1) and np.array_equal(sym, z[f"t{i}_q"]), i
        assert np.array_equal(kp.f32_to_bf16(mn), z[f"t{i}_min"]), i
        assert np.array_equal(kp.f32_to_bf16(sc), z[f"t{i}_scale"]), i
        assert np.array_equal(kp.f32_to_bf16(kp.dequantize(sym, mn, sc)), z[f"t{i}_deq"]), i


def _axis_cases():
    z = np.load(GOLDEN / "quantizer_axes.npz")
    return sorted({k.rsplit("_x", 1)[0] for k in z.files if k.startswith("a") and k.endswith("_x")})


@pytest.mark.parametrize("key", _axis_cases())
def test_kvserve_quantizer_axes_match_reference_golden(key):
    """KVServeQuantizer with every non-default (axis_key, axis_value): symbols, each
    section's metadata in the reference's keepdim layout, and the dequantized layer."""
    z = np.load(GOLDEN / "quantizer_axes.npz")
    pi, ci, layer = key.split("_")
    axes = tuple(kp.AXES[int(a)] for a in z[f"{pi}_axes"])
    prof = _profiles_for(int(ci[1:]), int(layer[1:]))
    x = f(z[key + "_x"])
    sym, meta = kp.quantize_layer(x, prof, axes)
    assert np.array_equal(sym, z[key + "_q"]), axes
    groups = sorted(set(prof.v.group))
    nl = prof.v.group.count(0) if len(groups) == 2 else None
    names = ["low", "high"] if nl is not None else (["low"] if f"{key}_low_key_meta_min" in z.files else ["high"])
    for si, name in enumerate(names):
        hs = slice(None) if nl is None else (slice(0, nl) if si == 0 else slice(nl, None))
        for part, (mn_t, sc_t), axis in (("key", (meta.kmin, meta.kscale), axes[0]),
                                         ("value", (meta.vmin, meta.vscale), axes[1])):
            sel = hs if axis == "channel" else si  # channel: rows of the section; else: its group
            for t, what in ((mn_t, "min"), (sc_t, "scale")):
                want = z[f"{key}_{name}_{part}_meta_{what}"]
                assert np.array_equal(kp.f32_to_bf16(t[sel]).reshape(-1), want.reshape(-1)), (axes, name, part, what)
    deq = kp.dequantize_layer(sym, meta, prof, axes)
    assert np.array_equal(kp.f32_to_bf16(deq), z[key + "_deq"]), axes


@pytest.mark.parametrize("layout", ["permuted", "native"])
def test_manager_layout_matches_reference_golden(layout):
    """CompressionManager without codec: the byte stream is the uint8 codec buffer."""
    z = np.load(GOLDEN / "compression_manager.npz")
    x = z[f"{layout}_x"]  # [L, 2, B, S, H, D]
    L = x.shape[0]
    pools = [x[l] for l in range(L)]
    B = x.shape[2]
    profs = [_profiles_for(1, l) for l in range(L)]
    chunks = kp.compress_request(pools, list(range(B)), profs, 0, 8, transform=False, layout=layout)
    assert len(chunks) == 1
    assert list(chunks[0].symbols.shape) == list(z[f"{layout}_codec_shape"])
    assert np.array_equal(chunks[0].symbols.reshape(-1), z[f"{layout}_bytes"])
    assert np.array_equal(chunks[0].stream[16:], z[f"{layout}_bytes"])
    dst = [np.zeros_like(p) for p in pools]
    kp.decompress_request(chunks, dst, list(range(B)), profs, 0, 8, transform=False, layout=layout)
    assert np.array_equal(np.stack(dst), z[f"{layout}_restored"])


# ------------------------------------------------------------------ signs
def test_signs_fixture_and_product_recipe():
    from kvserve_amd.profiles import rademacher_sign_bits

    z = np.load(GOLDEN / "signs.npz")
    for k in z.files:
        _, seed, layer, H, D = k.split("_")
        seed, layer, H, D = int(seed), int(layer), int(H), int(D)
        s = kp.rademacher_signs(seed, layer, H, D)
        assert np.array_equal(s, z[k].astype(np.float32) * 2 - 1)
        assert np.array_equal(rademacher_sign_bits(seed, layer, H, D), kp.sign_bits(s))


# ------------------------------------------------------------------ FWHT closed forms
@pytest.mark.parametrize("D", [8, 64, 128])
def test_fwht_is_sylvester_on_exact_inputs(D):
    rng = np.random.default_rng(D)
    x = rng.integers(-1, 2, (33, D)).astype(np.float32)
    H = scipy.linalg.hadamard(D)
    assert np.array_equal(kp.fwht_f32(x), (x.astype(np.int64) @ H).astype(np.float32))
    # H.H = D.I: the transform applied twice is D times the identity
    assert np.array_equal(kp.fwht_f32(kp.fwht_f32(x)), x * D)


def test_hadamard_roundtrip_and_signs_on_exact_inputs():
    rng = np.random.default_rng(3)
    D, H = 128, 4
    x = rng.integers(-1, 2, (5, H, D)).astype(np.float32)
    s = kp.rademacher_signs(7, 2, H, D)
    y = kp.hadamard_forward(kp.f32_to_bf16(x), s)
    ref = ((x * s).astype(np.float64) @ scipy.linalg.hadamard(D)) / np.sqrt(D)
    assert np.array_equal(y, kp.f32_to_bf16(ref.astype(np.float32)))
    z = kp.hadamard_inverse(y, s)
    back = kp.bf16_to_f32(z)
    assert np.max(np.abs(back - x)) <= 2 ** -6  # one bf16 rounding in each direction


def test_pow2_chunks_follow_the_reference_examples():
    # hadamard_func.py:63-64 docstring: 96 -> [64, 32], 100 -> [64, 32, 4]
    assert kp.pow2_chunks(96) == [64, 32] and kp.pow2_chunks(100) == [64, 32, 4]
    assert kp.pow2_chunks(128) == [128] and kp.pow2_chunks(80) == [64, 16]


@pytest.mark.parametrize("D", [96, 80, 224, 256])
def test_chunked_transform_is_sylvester_per_chunk(D):
    """Each unit vector inside chunk [a, a + c) maps to a Walsh row of H_c / sqrt(c) at
    [a, a + c) and zero elsewhere: the chunks are transformed independently, with
    their own scale (Sylvester closed form, scipy.linalg.hadamard)."""
    eye = np.eye(D, dtype=np.float32)
    y = kp.fwht_scaled_f32(eye)
    start = 0
    for c in kp.pow2_chunks(D):
        blk = scipy.linalg.hadamard(c).astype(np.float32) * np.float32(1.0 / np.sqrt(c))
        assert np.array_equal(y[start:start + c, start:start + c], blk)
        assert not y[start:start + c, :start].any() and not y[start:start + c, start + c:].any()
        start += c
    # signs and rounding: forward then inverse restores exact {-1, 0, 1} inputs within
    # one bf16 rounding each way
    rng = np.random.default_rng(D)
    x = rng.integers(-1, 2, (4, 3, D)).astype(np.float32)
    s = kp.rademacher_signs(9, 1, 3, D)
    back = kp.bf16_to_f32(kp.hadamard_inverse(kp.hadamard_forward(kp.f32_to_bf16(x), s), s))
    assert np.max(np.abs(back - x)) <= 2 ** -6
    assert kp.sign_bits(s).shape == (3, (D + 31) // 32)


def test_fwht_random_close_to_float64():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((64, 128)).astype(np.float32)
    ref = x.astype(np.float64) @ scipy.linalg.hadamard(128)
    assert np.max(np.abs(kp.fwht_f32(x) - ref)) < 1e-4


# ------------------------------------------------------------------ bitpack
def test_bitpack_known_answer():
    s = kp.bitpack_encode(np.array([1, 2, 3, 4, 5], np.uint8), 4)
    assert s.tobytes().hex() == "4b425001040000000500000000000000214305"
    s3 = kp.bitpack_encode(np.array([7, 0, 5, 1], np.uint8), 3)
    # 7 | 0<<3 | 5<<6 | 1<<9 -> bits 0..11 = 0b001_101_000_111 -> bytes 0x47, 0x03
    assert s3[16:].tobytes().hex() == "4703"
    assert kp.bitpack_encode(np.zeros(0, np.uint8), 8).tobytes().hex() == "4b425001080000000000000000000000"


@pytest.mark.parametrize("bits", range(1, 9))
def test_bitpack_c_oracle_matches_numpy(bits):
    rng = np.random.default_rng(bits)
    for n in [0, 1, 7, 13, 8193, 100003]:
        x = rng.integers(0, 2 ** bits, n, dtype=np.uint8)
        a = kp.bitpack_encode(x, bits)
        assert a.size == 16 + (n * bits + 7) // 8
        assert np.array_equal(a, cbitpack.encode(x, bits))
        assert np.array_equal(cbitpack.decode(a, n, bits), x)
        assert np.array_equal(kp.bitpack_decode(a, n, bits), x)


def test_bitpack_contract_errors():
    a = kp.bitpack_encode(np.array([1, 2, 3], np.uint8), 2)
    with pytest.raises(ValueError, match="length"):
        kp.bitpack_decode(a[:-1], 3, 2)
    b = a.copy()
    b[0] = 0
    with pytest.raises(ValueError, match="header"):
        cbitpack.decode(b, 3, 2)
    with pytest.raises(ValueError, match="exceeds"):
        kp.bitpack_encode(np.array([4], np.uint8), 2)


# ------------------------------------------------------------------ exhaustive identities
def _all_positive_bf16():
    b = np.arange(0x0080, 0x7F80, dtype=np.uint16)  # normal positive finite bf16
    return kp.bf16_to_f32(b)


def test_scalar_division_equals_reciprocal_multiply_exhaustively():
    """torch divides a bf16 tensor by a Python int on the GPU as x * fp32(1/b); on the
    CPU as x / b.  After the bf16 rounding the two agree for every bf16 x and every
    level count, so CPU golden vectors stand for the GPU reference."""
    d = _all_positive_bf16()
    for L in range(2, 256):
        a = kp.rbf(d / np.float32(L - 1))
        b = kp.rbf(d * (np.float32(1.0) / np.float32(L - 1)))
        assert np.array_equal(a, b), L


def test_bf16_quotient_by_reciprocal_sampled():
    """bf16(t / sc) == bf16(t * (1/sc)) for bf16 t, sc (the GPU quantizer's form)."""
    rng = np.random.default_rng(11)
    allv = _all_positive_bf16()
    for _ in range(10):
        t = rng.choice(allv, 1_000_000)
        sc = rng.choice(allv, 1_000_000)
        with np.errstate(over="ignore", under="ignore"):
            ok = np.isfinite(t / sc) & (t / sc < 3e38) & (t / sc > 1e-37)
        t, sc = t[ok], sc[ok]
        assert np.array_equal(kp.rbf(t / sc), kp.rbf(t * (np.float32(1) / sc)))


def test_quantizer_within_one_level_of_fp32_reference():
    """The reference's own procedural pin (scripts/bench_compression_stages.py:343-356;
    tests/runtime/test_gpu.py:412-467): bf16 min-max within +-1 of an fp32 min-max."""
    rng = np.random.default_rng(9)
    x = kp.rbf(rng.standard_normal((4, 16, 3, 128)).astype(np.float32) * 3)
    for axis, dims in (("channel", (0, 1)), ("token", (2, 3))):
        sym, _, _ = kp.quantize(16, x, axis)
        mn, mx = x.min(axis=dims, keepdims=True), x.max(axis=dims, keepdims=True)
        ref = np.clip(np.rint((x - mn) / ((mx - mn) / 15)), 0, 16)
        assert np.abs(sym.astype(np.int64) - ref).max() <= 1


# ------------------------------------------------------------------ masks
def test_masks_brute_force_from_scores():
    from kvserve_amd.profiles import head_low_mask, layer_low_mask, scores_from_csv

    s = scores_from_csv("Llama-3.1-8B-Instruct")
    assert s.shape == (32, 8) and len(np.unique(s)) == 256
    m3 = head_low_mask(s, 0.3)
    assert m3.sum() == 77 and list(np.nonzero(m3[0])[0]) == [0, 6]
    assert list(np.nonzero(head_low_mask(s, 0.8)[0])[0]) == [0, 1, 2, 3, 4, 5, 6]
    # brute force: a head is low iff fewer than 77 scores are smaller than it
    flat = s.reshape(-1)
    brute = np.array([(flat < v).sum() < 77 for v in flat]).reshape(s.shape)
    assert np.array_equal(brute, m3)
    assert np.array_equal(m3, kp.head_mask_from_scores(s, 0.3))
    assert layer_low_mask(32).sum() == 11 and layer_low_mask(32)[-11:].all()
    assert np.array_equal(layer_low_mask(28), kp.layer_mask(28))
