"""impl "tilelang_fused" on the CPU: the adapter's normalisation and the quantizer's
validation (as the reference's tests pin them: test_compression_regressions.py:14-46,
test_pluggable_operators.py:226-227), the per-(layer, head) level table, and the
numpy oracle of the compress_v3 / decompress_v3 arithmetic (oracle/fused_v3.py)
pinned by an independent float64 derivation on exactly representable inputs."""

import copy
import math

import numpy as np
import pytest

from oracle import fused_v3 as fv
from oracle import kvpipe as kp


# ------------------------------------------------------------------ adapter / facade
def test_fused_normalization_preserves_seed_and_request_pipeline():
    from kvserve_amd.compression.manager import KVCompressionAdapter

    spec = {"pipeline": ["transformer", "quantizer"],
            "transformer_config": {"transform_type": "hadamard", "seed": 1234},
            "quantizer_config": {"impl": "tilelang_fused"}}
    before = copy.deepcopy(spec)
    adapter = KVCompressionAdapter(spec, num_kv_heads=4, head_size=128)
    assert spec == before
    assert adapter._config.pipeline == ["quantizer"]
    assert adapter._manager.config.pipeline == adapter._config.pipeline
    assert adapter._config.quantizer_config["base_seed"] == 1234
    adapter._manager.update_config(adapter._config)
    assert adapter._manager.quantizer._cfg["base_seed"] == 1234
    assert type(adapter._manager.quantizer).__name__ == "FusedHadamardQuantizer"


@pytest.mark.parametrize("patch", [
    {"axis_key": "token"}, {"axis_value": "tensor"},
    {"quant_type": "absmax"}, {"split_type": "invalid"},
])
def test_fused_rejects_unsupported_config(patch):
    from kvserve_amd.compression.quantizer import TileLangFusedQuantizer

    with pytest.raises(ValueError):
        TileLangFusedQuantizer(**patch)
    q = TileLangFusedQuantizer()
    before = dict(q._cfg)
    with pytest.raises(ValueError):
        q.update_params(**patch)
    assert q._cfg == before


def test_fused_rejects_conflicting_seed_and_other_impls():
    from kvserve_amd.compression.manager import KVCompressionAdapter

    with pytest.raises(ValueError, match="Conflicting"):
        KVCompressionAdapter._normalize_config({
            "pipeline": ["transformer", "quantizer"], "impl": "tilelang_fused",
            "transformer_config": {"seed": 1}, "quantizer_config": {"base_seed": 2}})
    cfg = {"pipeline": ["transformer", "quantizer", "codec"], "transformer_config": {"transform_type": "hadamard"},
           "quantizer_config": {"impl": "centered_codebook"}, "codec_config": {"codec_type": "bitpack"}}
    with pytest.raises(ValueError, match="cannot use"):
        KVCompressionAdapter({**cfg, "impl": "tilelang_fused"}, 4, 128)
    with pytest.raises(ValueError, match="requires a quantizer"):
        KVCompressionAdapter._normalize_config({"pipeline": ["transformer"], "quantizer_impl": "tilelang_fused"})
    with pytest.raises(ValueError, match="only fuses the Hadamard"):
        KVCompressionAdapter._normalize_config({
            "pipeline": ["transformer", "quantizer"], "impl": "tilelang_fused",
            "transformer_config": {"transform_type": "dct"}})
    # an explicit quantizer seed without a transformer seed wins; the default seed otherwise
    n = KVCompressionAdapter._normalize_config({"pipeline": ["transformer", "quantizer", "codec"],
                                               "quantizer_config": {"impl": "tilelang_fused", "seed": 7}})
    assert n["pipeline"] == ["quantizer", "codec"] and n["quantizer_config"]["base_seed"] == 7
    n = KVCompressionAdapter._normalize_config({"pipeline": ["transformer", "quantizer"], "impl": "tilelang_fused"})
    assert n["quantizer_config"]["base_seed"] == 0x3333


def test_fused_levels_table():
    """Levels per (layer, head) as KVHadamardQuantOp builds them
    (kv_hadamard_quant.py:105-153): uniform high values without a loadable CSV; with
    the Llama-3.1-8B scores at ratio 0.8 layer 0's low heads are {0..6} (derived from
    the data file); layer split: the last round(0.33 * 32) = 11 layers are low."""
    from kvserve_amd.compression.quantizer import FusedHadamardQuantizer

    k, v = FusedHadamardQuantizer().levels(0, 8)
    assert k.tolist() == [12.0] * 8 and v.tolist() == [8.0] * 8
    q = FusedHadamardQuantizer(model_name="Llama-3.1-8B-Instruct", hybrid_ratio=0.8)
    k, v = q.levels(0, 8)
    assert k.tolist() == [6.0] * 7 + [12.0] and v.tolist() == [4.0] * 7 + [8.0]
    # tensor parallel: the second half of the 8 heads on rank 1 of 2
    k1, _ = FusedHadamardQuantizer(model_name="Llama-3.1-8B-Instruct", hybrid_ratio=0.8,
                                   tensor_parallel_size=2, tp_rank=1).levels(0, 4)
    assert k1.tolist() == [6.0, 6.0, 6.0, 12.0]
    ql = FusedHadamardQuantizer(model_name="Llama-3.1-8B-Instruct", split_type="layer")
    assert ql.levels(20, 8)[0].tolist() == [12.0] * 8
    assert ql.levels(21, 8)[0].tolist() == [6.0] * 8 and ql.levels(31, 8)[1].tolist() == [4.0] * 8
    with pytest.raises(IndexError):
        q.levels(32, 8)


# ------------------------------------------------------------------ oracle pins
def test_round_half_away_known_answers():
    v = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 0.49999997, 2.4999998, 3.0, -0.2], np.float32)
    assert fv.round_half_away(v).tolist() == [1.0, 2.0, 3.0, -1.0, -2.0, 0.0, 2.0, 3.0, -0.0]


def test_group_map_first_occurrence():
    assert fv.group_map([4, 8, 4, 6, 8]).tolist() == [0, 1, 0, 2, 1]
    assert fv.group_map([12.0] * 3).tolist() == [0, 0, 0]


def _f32(x):
    return np.float32(x)


def test_compress_matches_float64_derivation_on_exact_inputs():
    """Inputs in {-3..3}: every butterfly sum is exact in fp32, so y = fl32(sum * s32)
    and each later fp32 op (difference, max with 1e-5, quotient) is the float64 value
    rounded once -- an independent restatement of the op order."""
    rng = np.random.default_rng(5)
    R, H, D = 9, 4, 64
    x = rng.integers(-3, 4, size=(2, R, H, D)).astype(np.float32)
    signs = kp.rademacher_signs(0xC0FEBABE, 3, H, D)
    kl = [12.0, 6.0, 12.0, 6.0]
    vl = [8.0, 4.0, 4.0, 8.0]
    q, m = fv.compress_layer(kp.f32_to_bf16(x), signs, kl, vl)
    Hm = np.array([[(-1) ** bin(i & j).count("1") for j in range(D)] for i in range(D)], np.float64)
    s32 = float(_f32(1.0 / math.sqrt(D)))
    y = ((x * signs).astype(np.float64) @ Hm * s32).astype(np.float32)
    kmn, kmx = y[0].min(0), y[0].max(0)
    ksc = (np.maximum((kmx.astype(np.float64) - kmn).astype(np.float32), _f32(1e-5)).astype(np.float64)
           / (np.array(kl)[:, None] - 1)).astype(np.float32)
    assert np.array_equal(m["kmin"], kmn) and np.array_equal(m["kscale"], ksc)
    had = kp.rbf(y)
    # the difference and the quotient are one fp32 op each, rounded before roundf
    quot = ((had[0].astype(np.float64) - kmn).astype(np.float32).astype(np.float64) / ksc).astype(np.float32)
    qk = np.clip(np.sign(quot) * np.floor(np.abs(quot.astype(np.float64)) + 0.5), 0, np.array(kl)[:, None])
    assert np.array_equal(q[0], qk.astype(np.uint8))
    # V: rows reduced over heads {0, 3} (levels 8) and {1, 2} (levels 4)
    rmn, rmx = y[1].min(-1), y[1].max(-1)
    for heads, L in (([0, 3], 8.0), ([1, 2], 4.0)):
        gmn, gmx = rmn[:, heads].min(1), rmx[:, heads].max(1)
        sc = (np.maximum((gmx.astype(np.float64) - gmn).astype(np.float32), _f32(1e-5)).astype(np.float64)
              / (L - 1)).astype(np.float32)
        for h in heads:
            assert np.array_equal(m["vmin"][:, h], gmn) and np.array_equal(m["vscale"][:, h], sc)
            quot = ((had[1][:, h].astype(np.float64) - gmn[:, None]).astype(np.float32).astype(np.float64)
                    / sc[:, None]).astype(np.float32)
            ref = np.clip(np.sign(quot) * np.floor(np.abs(quot.astype(np.float64)) + 0.5), 0, L)
            assert np.array_equal(q[1][:, h], ref.astype(np.uint8))


def test_planted_mistake_bf16_statistics_is_caught(monkeypatch):
    """Statistics taken on bf16(y) instead of the fp32 y change the K minima."""
    rng = np.random.default_rng(2)
    x = kp.f32_to_bf16(rng.standard_normal((2, 64, 8, 128)).astype(np.float32))
    signs = kp.rademacher_signs(1, 0, 8, 128)
    _, good = fv.compress_layer(x, signs, [12.0] * 8, [8.0] * 8)
    real = fv.transform
    monkeypatch.setattr(fv, "transform", lambda xb, s: kp.rbf(real(xb, s)))
    _, bad = fv.compress_layer(x, signs, [12.0] * 8, [8.0] * 8)
    assert not np.array_equal(good["kmin"], bad["kmin"])


def test_decompress_exact_on_integer_reconstruction():
    """With scale 1 and integer minima the dequantized values are small integers, so
    the fp32 butterflies are exact and the output is bf16(sum * s32) * sign."""
    rng = np.random.default_rng(9)
    R, H, D = 5, 2, 128
    q = rng.integers(0, 16, size=(2, R, H, D)).astype(np.uint8)
    kmin = rng.integers(-8, 1, size=(H, D)).astype(np.float16)
    vmin = rng.integers(-8, 1, size=(R, H)).astype(np.float16)
    one_k, one_v = np.ones((H, D), np.float16), np.ones((R, H), np.float16)
    signs = kp.rademacher_signs(11, 2, H, D)
    out = fv.decompress_layer(q, kmin, one_k, vmin, one_v, signs)
    x = np.stack([q[0].astype(np.float64) + kmin, q[1].astype(np.float64) + vmin[..., None]])
    Hm = np.array([[(-1) ** bin(i & j).count("1") for j in range(D)] for i in range(D)], np.float64)
    s32 = float(_f32(1.0 / math.sqrt(D)))
    ref = kp.f32_to_bf16(((x @ Hm) * s32).astype(np.float32) * signs)
    assert np.array_equal(out, ref)


def test_symbols_within_half_a_step_and_roundtrip_isometry():
    """Every symbol reconstructs its transformed value to within half a quantization
    step, plus the bf16 rounding of y and the float16 rounding of the metadata; the
    inverse transform is an isometry, so each row's error is that of its transform."""
    rng = np.random.default_rng(4)
    R, H, D = 48, 8, 128
    xb = kp.f32_to_bf16(rng.standard_normal((2, R, H, D)).astype(np.float32))
    signs = kp.rademacher_signs(0xC0FEBABE, 1, H, D)
    kl, vl = [16.0, 6.0] * 4, [12.0, 12.0, 4.0, 4.0] * 2
    q, m = fv.compress_layer(xb, signs, kl, vl)
    y = fv.transform(xb, signs).astype(np.float64)
    kmn16, ksc16 = m["kmin"].astype(np.float16), m["kscale"].astype(np.float16)
    vmn16, vsc16 = m["vmin"].astype(np.float16), m["vscale"].astype(np.float16)
    parts = ((q[0], m["kmin"][None], m["kscale"][None], kmn16[None], ksc16[None], np.array(kl)[:, None]),
             (q[1], m["vmin"][..., None], m["vscale"][..., None], vmn16[..., None], vsc16[..., None],
              np.array(vl)[:, None]))
    for part, (sym, mn, sc, mn16, sc16, L) in enumerate(parts):
        assert (sym <= L).all()
        yq = sym.astype(np.float64) * sc16.astype(np.float64) + mn16.astype(np.float64)
        bound = (0.5 * sc + np.abs(y[part]) * 2.0 ** -8 + np.abs(mn - mn16.astype(np.float64))
                 + sym * np.abs(sc - sc16.astype(np.float64)) + 1e-6)
        assert (np.abs(y[part] - yq) <= bound).all(), part
    out = fv.decompress_layer(q, kmn16, ksc16, vmn16, vsc16, signs)
    x, xr = kp.bf16_to_f32(xb).astype(np.float64), kp.bf16_to_f32(out).astype(np.float64)
    yq = np.stack([q[0] * ksc16.astype(np.float64) + kmn16, q[1] * vsc16[..., None].astype(np.float64)
                   + vmn16[..., None]])
    row_err = np.linalg.norm(xr - x, axis=-1)
    t_err = np.linalg.norm(yq - y, axis=-1)
    assert (row_err <= t_err * 1.01 + np.linalg.norm(x, axis=-1) * 2.0 ** -7).all()
