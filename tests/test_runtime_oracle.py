"""Pins of the fixed-profile runtime oracle (oracle/runtime_ref.py) and of the host
side of kvserve_amd.runtime: configuration, head selection, signs, layout.  CPU only.

The oracle is checked against the reference's own CPU runtime (golden chunks), the
Sylvester matrix, Walsh functions of unit vectors and the reference tests'
quantizer formulas (tests/runtime/test_gpu.py:412-535, test_hadamard.py:14-23).
"""

from __future__ import annotations

import json
import numpy as np
import pytest
import torch

from oracle import runtime_ref as R
from tests._runtime_cases import MINUS_NINE, extra_config, full_caches, load_cases, physical

from kvserve_amd.runtime import CacheSpec, CompressionConfig, build_signs
from kvserve_amd.runtime.layout import build_compression_layout
from kvserve_amd.runtime.scores import build_head_selection

CASES = load_cases()


def oracle_parts(case, caches, kv_part):
    meta = case["meta"]
    config = CompressionConfig.from_extra_config(extra_config(meta))
    parts = []
    for name, part, u8_offset, _raw, sections in meta["layout"]["parts"]:
        if part != kv_part:
            continue
        layer = int(name.split(".")[2])
        signs = case.get(f"signs{layer}_{part}")
        parts.append(R.LayerPart(
            cache=caches[layer], channel_offset=0 if part == 0 else meta["head_size"],
            head_size=meta["head_size"] if part == 0 else meta["head_size_v"], order=meta["orders"][str(layer)],
            u8_offset=u8_offset, signs=signs, sections=[R.Section(*s) for s in sections]))
    return parts, config


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_reference_runtime_chunks(name):
    case = CASES[name]
    meta = case["meta"]
    src, dst = full_caches(case, True), full_caches(case, False)
    src_ids, dst_ids = physical(meta, meta["src"]), physical(meta, meta["dst"])
    for part in (0, 1):
        parts, config = oracle_parts(case, src, part)
        transform, quant = config.uses_transformer, config.uses_quantizer
        payload, aux, tail = R.encode_part(parts, src_ids, meta["tokens"], meta["block_size"],
                                           meta["blocks_per_logical"], transform, quant,
                                           case[f"p{part}_payload"].size, case[f"p{part}_aux"].size)
        assert np.array_equal(payload, case[f"p{part}_payload"])
        assert np.array_equal(aux, case[f"p{part}_aux"])
        assert np.array_equal(tail, case[f"p{part}_tail"])
        targets, _ = oracle_parts(case, dst, part)
        R.decode_part(targets, dst_ids, meta["tokens"], meta["block_size"], meta["blocks_per_logical"], transform,
                      quant, payload, aux, tail)
    for i, cache in enumerate(dst):
        assert np.array_equal(cache[dst_ids], case[f"dst{i}"])
        untouched = sorted(set(range(cache.shape[0])) - set(dst_ids))
        assert (cache[untouched] == MINUS_NINE).all()


def test_oracle_catches_a_planted_stage_order_mistake():
    """Butterflies in decreasing bit order give different bf16 roundings on real data."""
    case = CASES["default_tail"]
    meta = case["meta"]
    src = full_caches(case, True)
    parts, _ = oracle_parts(case, src, 0)
    good, _, _ = R.encode_part(parts, physical(meta, meta["src"]), meta["tokens"], meta["block_size"], 1, True, True,
                               case["p0_payload"].size, case["p0_aux"].size)
    original = R.fwht

    def reversed_stages(rows):
        return original(rows[..., ::-1])[..., ::-1]

    R.fwht = reversed_stages
    try:
        bad, _, _ = R.encode_part(parts, physical(meta, meta["src"]), meta["tokens"], meta["block_size"], 1, True,
                                  True, case["p0_payload"].size, case["p0_aux"].size)
    finally:
        R.fwht = original
    assert np.array_equal(good, case["p0_payload"]) and not np.array_equal(bad, case["p0_payload"])


def sylvester(d):
    m = np.ones((1, 1))
    while m.shape[0] < d:
        m = np.block([[m, m], [m, -m]])
    return m


@pytest.mark.parametrize("dim", [1, 2, 4, 8, 16, 32, 64, 128, 256])
def test_fwht_matches_sylvester_on_small_integers(dim):
    """Small integers keep every bf16 intermediate exact (test_hadamard.py:72-86)."""
    rng = np.random.default_rng(dim)
    x = rng.integers(-1, 2, (33, dim)).astype(np.float32)
    expected = R.rn((x.astype(np.float64) @ sylvester(dim) / np.sqrt(dim)).astype(np.float32))
    assert np.array_equal(R.fwht(x), expected)


@pytest.mark.parametrize("dim", [512, 1024, 2048])
def test_fwht_of_unit_vectors_is_a_walsh_row(dim):
    rows = np.eye(dim, dtype=np.float32)[[0, 1, dim // 2 + 3, dim - 1]]
    out = R.fwht(rows)
    k = np.array([0, 1, dim // 2 + 3, dim - 1])[:, None]
    j = np.arange(dim)[None, :]
    sign = 1 - 2 * (np.vectorize(lambda v: bin(v).count("1"))(k & j) % 2)
    assert np.array_equal(out, R.rn(sign.astype(np.float32) * np.float32(1 / np.sqrt(dim))))


def torch_bf16_reference(source):
    """The reference test's bf16 op-order transform (test_hadamard.py:14-23)."""
    result = source.clone()
    dim = result.shape[-1]
    step = 1
    while step < dim:
        pair = result.view(-1, dim // (2 * step), 2, step)
        a, b = pair[:, :, 0, :], pair[:, :, 1, :]
        result = torch.stack((a + b, a - b), dim=2).reshape_as(result)
        step *= 2
    return result.mul_(dim ** -0.5)


@pytest.mark.parametrize("dim", [1, 2, 8, 64, 128, 1024, 2048])
def test_fwht_matches_torch_bf16_op_order(dim):
    torch.manual_seed(42)
    source = torch.randn(7, dim, dtype=torch.bfloat16) * 17
    expected = torch_bf16_reference(source).view(torch.int16).numpy().view(np.uint16)
    got = R.to_bits(R.fwht(R.from_bits(source.view(torch.int16).numpy().view(np.uint16))))
    assert np.array_equal(got, expected)


@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("pattern,levels", [("random", 4), ("random", 6), ("constant", 12), ("tiny", 8),
                                            ("zeros", 16)])
def test_quantizer_matches_reference_test_formula(axis, pattern, levels):
    """test_gpu.py:470-535's bf16-exact symbols and aux."""
    torch.manual_seed(0)
    x = torch.rand(2, 16, 2, 8, dtype=torch.bfloat16) - 0.5
    if pattern == "constant":
        x.fill_(-3.125)
    elif pattern == "tiny":
        x.mul_(1e-6)
    elif pattern == "zeros":
        x.zero_()
    dims = (0, 1) if axis == "channel" else (2, 3)
    minimum = x.amin(dims, keepdim=True)
    maximum = x.amax(dims, keepdim=True)
    scale = ((maximum - minimum).clamp_min(1e-5).float() / (levels - 1)).to(x.dtype)
    inverse = scale.float().reciprocal().to(x.dtype)
    shifted = (x.float() - minimum.float()).to(x.dtype)
    expected = (shifted.float() * inverse.float()).to(x.dtype).float().round().clamp(0, levels - 1).to(torch.uint8)
    xs = R.from_bits(x.view(torch.int16).numpy().view(np.uint16))
    mn, mx = xs.min(axis=dims, keepdims=True), xs.max(axis=dims, keepdims=True)
    s, inv = R.quant_params(mn, mx, levels)
    assert np.array_equal(R.quantize(xs, mn, inv, levels), expected.numpy())
    assert np.array_equal(R.to_bits(s), scale.view(torch.int16).numpy().view(np.uint16))


@pytest.mark.parametrize("axis", ["channel", "token", "tensor"])
def test_quantizer_within_one_level_of_float64(axis):
    """test_gpu.py:412-467: symbols within one level of the float64 formula, and the
    dequantized values within step * 0.65 + 2 % of the range."""
    rng = np.random.default_rng(1)
    x = R.rn(rng.standard_normal((1, 16, 2, 8)).astype(np.float32) * 3 + 1)
    axes = {"channel": (0, 1), "token": (2, 3), "tensor": (0, 1, 2, 3)}[axis]
    lo, hi = x.min(axis=axes, keepdims=True), x.max(axis=axes, keepdims=True)
    step = np.maximum(hi.astype(np.float64) - lo, 1e-5) / 15
    expected = np.clip(np.rint((x - lo.astype(np.float64)) / step), 0, 15)
    s, inv = R.quant_params(lo, hi, 16)
    q = R.quantize(x, lo, inv, 16)
    assert np.abs(q.astype(np.float64) - expected).max() <= 1
    restored = R.dequantize(q, lo, s)
    assert np.all(np.abs(restored - x) <= step * 0.65 + np.maximum(np.abs(lo), np.abs(hi)) * 0.02)


# ---------------------------------------------------------------- host side of the runtime
def specs_of(meta):
    return {f"model.layers.{i}.self_attn": CacheSpec(i, meta["block_size"], meta["heads"], meta["head_size"],
                                                     torch.bfloat16, meta["head_size_v"])
            for i in range(meta["layers"])}


@pytest.mark.parametrize("name", sorted(CASES))
def test_layout_orders_and_signs_match_reference(name):
    from dataclasses import replace

    case = CASES[name]
    meta = case["meta"]
    config = CompressionConfig.from_extra_config(extra_config(meta))
    planning = config if "quantizer" in config.pipeline else replace(config, split_type="layer")
    scores = np.asarray(meta["scores"], dtype=np.float32) if meta["scores"] is not None else None
    specs = specs_of(meta)
    selection = build_head_selection(specs, planning, 0, 1, scores)
    assert {str(k): list(v) for k, v in selection.local_orders.items()} == meta["orders"]
    layout = build_compression_layout(specs, planning, selection.low_counts, meta["layers"])
    want = meta["layout"]
    for key in ("raw_bytes_by_part", "u8_bytes_by_part", "aux_bytes_by_part"):
        assert list(getattr(layout, key)) == want[key], key
    for key in ("arena_bytes", "scratch_stride", "u8_base", "aux_arena_bytes", "raw_tail_capacity"):
        assert getattr(layout, key) == want[key], key
    got_parts = [[p.layer_name, p.kv_part, p.u8_offset, p.raw_bytes,
                  [[s.head_start, s.head_count, s.num_levels, s.axis, s.aux_min_offset, s.aux_scale_offset]
                   for s in p.sections]] for p in layout.layer_parts]
    assert got_parts == want["parts"]
    if config.uses_transformer:
        for p in layout.layer_parts:
            signs = build_signs(p, selection.local_orders[p.layer_index], config.seed)
            assert np.array_equal(signs.reshape(meta["heads"], -1).to(torch.int8).numpy(),
                                  case[f"signs{p.layer_index}_{p.kv_part}"])


def test_signs_follow_the_fixture_generator_recipe():
    """Rows are the Rademacher rows of tests/golden/signs.npz (seed ^ layer << 16 ^ head)."""
    fixture = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "signs.npz")
    key = "s_3237919422_31_8_128"
    part = type("P", (), {"num_heads": 8, "head_size": 128, "dtype": torch.bfloat16, "layer_index": 31})()
    order = (3, 1, 0, 2, 7, 6, 5, 4)
    signs = build_signs(part, order, 3237919422).reshape(8, 128).to(torch.int8).numpy()
    assert np.array_equal(signs, fixture[key][list(order)].astype(np.int8) * 2 - 1)


@pytest.mark.parametrize("bad,message", [
    ({"transformer": "dct"}, "only supports transformer='hadamard'"),
    ({"codec": "zstd"}, "only supports codec='ans'"),
    ({"slot_count": 0}, "slot_count must be >= 1"),
    ({"logical_blocks_per_chunk": 0}, "logical_blocks_per_chunk must be >= 1"),
    ({"pipeline": ["quantizer", "transformer"]}, "must follow transformer, quantizer, codec order"),
    ({"pipeline": ["codec", "codec"]}, "must be unique"),
    ({"pipeline": ["squeeze"]}, "Unknown KVServe compression stages"),
    ({"hybrid_ratio": 1.5}, "hybrid_ratio must be in"),
    ({"high_key_num_levels": 1}, "must be an integer in"),
    ({"split_type": "row"}, "Unsupported KVServe compression split_type"),
    ({"axis_key": "row"}, "Unsupported KVServe key quantization axis"),
])
def test_config_rejects_like_the_reference(bad, message):
    with pytest.raises(ValueError, match=message):
        CompressionConfig.from_extra_config({"compression": {"enable-compression-pipeline": True, **bad}})


def test_config_raw_aggregate_spellings():
    agg = CompressionConfig.from_extra_config({"raw_agg": {"slot_count": 3}})
    assert agg.is_raw_aggregate and agg.slot_count == 3 and agg.logical_blocks_per_chunk == 160
    assert CompressionConfig.from_extra_config({"raw_aggregate": True, "raw_agg": {"slot_count": 5}}).slot_count == 2
    assert not CompressionConfig.from_extra_config({"raw_aggregate": False}).available
    with pytest.raises(ValueError, match="Unknown raw_aggregate parameters"):
        CompressionConfig.from_extra_config({"raw_aggregate": {"slots": 1}})
    assert not CompressionConfig.from_extra_config({}).available


def test_memory_plan_sizes_codec_arenas_without_a_device():
    from kvserve_amd.runtime import build_memory_plan
    from kvserve_amd.runtime.memory import codec_capacity

    config = CompressionConfig.from_extra_config({"compression": {"enable-compression-pipeline": True,
                                                                  "logical_blocks_per_chunk": 4}})
    specs = {f"l.{i}": CacheSpec(i, 16, 4, 128, torch.bfloat16) for i in range(4)}
    plan = build_memory_plan(config, specs, num_layers=4)
    cap, scratch = codec_capacity(plan.layout.packed_bytes_by_part[0])
    assert plan.codec_max_output_bytes[0] == cap > plan.layout.packed_bytes_by_part[0]
    assert plan.layout.arena_bytes >= max(cap, plan.layout.u8_base + max(plan.layout.packed_bytes_by_part))
    assert plan.codec_workspace_bytes >= 2 * scratch
    assert build_memory_plan(CompressionConfig(), specs) is None
    with pytest.raises(ValueError, match="whole kernel blocks"):
        build_memory_plan(config, specs, blocks_per_logical=3)


def test_head_selection_tp_slices_and_replicated_kv_heads():
    config = CompressionConfig(enabled=True, split_type="head", hybrid_ratio=0.5)
    scores = np.array([[4.0, 1.0, 3.0, 2.0]], dtype=np.float32)
    one = {"l.0": CacheSpec(0, 16, 2, 8, torch.bfloat16)}
    # global lowest two of {4,1,3,2} are heads 1 and 3
    assert build_head_selection(one, config, 0, 2, scores).local_orders[0] == (1, 0)
    assert build_head_selection(one, config, 1, 2, scores).local_orders[0] == (1, 0)
    single = {"l.0": CacheSpec(0, 16, 1, 8, torch.bfloat16)}
    wide = np.array([[0.5, 2.0]], dtype=np.float32)
    # 4 ranks share 2 score columns: ranks 0,1 -> column 0 (low), ranks 2,3 -> column 1
    assert [build_head_selection(single, config, r, 4, wide).low_counts[0] for r in range(4)] == [1, 1, 0, 0]
    with pytest.raises(ValueError, match="incompatible"):
        build_head_selection(single, config, 0, 3, np.ones((1, 5), dtype=np.float32))
    with pytest.raises(ValueError, match="finite 2D"):
        build_head_selection(one, config, 0, 1, np.array([[np.nan, 1.0]], dtype=np.float32))



def test_layout_layer_split_and_arena_invariants():
    """Layer split: of 10 layers the last round(3.3) = 3 are low.  Every aux table is
    256-aligned, disjoint from the others and inside its part's aux bytes; the u8 stream
    of each part is gap-free in layer order; K and V alternate per layer."""
    config = CompressionConfig.from_extra_config({"compression": {"enable-compression-pipeline": True,
                                                                  "axis_value": "tensor",
                                                                  "logical_blocks_per_chunk": 2}})
    specs = {f"m.{i}": CacheSpec(i, 16, 4, 64 if i % 2 else 128, torch.bfloat16, head_size_v=64) for i in range(10)}
    layout = build_compression_layout(specs, config, {}, 10)
    assert [p.kv_part for p in layout.layer_parts] == [0, 1] * 10
    for kv in (0, 1):
        parts = layout.parts(kv)
        assert [p.layer_index for p in parts] == list(range(10))
        assert [p.sections[0].num_levels for p in parts] == (
            [config.high_key_num_levels] * 7 + [config.low_key_num_levels] * 3 if kv == 0
            else [config.high_value_num_levels] * 7 + [config.low_value_num_levels] * 3)
        at, tables = 0, []
        for p in parts:
            assert p.u8_offset == at and p.raw_bytes == 2 * 32 * 4 * p.head_size
            at += 32 * 4 * p.head_size
            (s,) = p.sections
            n = 2 * (4 * p.head_size if s.axis == "channel" else 1)
            tables += [(s.aux_min_offset, n), (s.aux_scale_offset, n)]
        assert layout.u8_bytes_by_part[kv] == at
        for (o, n), (o2, _) in zip(tables, tables[1:]):
            assert o % 256 == 0 and o + n <= o2
        assert tables[-1][0] + tables[-1][1] <= layout.aux_bytes_by_part[kv]
    assert layout.aux_arena_bytes == 2 * max(layout.aux_bytes_by_part)
    assert layout.scratch_stride == 2 * 32 * 4 * 128 and layout.u8_base == 2 * layout.scratch_stride
    agg = build_compression_layout(specs, CompressionConfig.from_extra_config({"raw_agg": True}), {}, 10)
    assert agg.aggregate and agg.aux_arena_bytes == 0 and agg.raw_tail_capacity == 0
    assert agg.arena_bytes == max(agg.raw_bytes_by_part)


def test_head_selection_ties_follow_binding_order():
    """Equal scores: the earlier candidate (binding order, then column) is low first."""
    config = CompressionConfig(enabled=True, split_type="head", hybrid_ratio=0.25)
    scores = np.ones((3, 4), dtype=np.float32)
    specs = {"b": CacheSpec(2, 16, 4, 8, torch.bfloat16), "a": CacheSpec(0, 16, 4, 8, torch.bfloat16)}
    sel = build_head_selection(specs, config, 0, 1, scores)
    assert sel.low_counts == {2: 2, 0: 0} and sel.local_orders[2] == (0, 1, 2, 3)
    with pytest.raises(ValueError, match="no row for layer 5"):
        build_head_selection({"x": CacheSpec(5, 16, 4, 8, torch.bfloat16)}, config, 0, 1, scores)


def test_score_loaders_read_every_supported_format(tmp_path):
    from kvserve_amd.runtime.scores import load_scores

    table = np.array([[0.5, 2.0, 1.0], [3.0, 0.25, 4.0]], dtype=np.float32)
    np.save(tmp_path / "s.npy", table)
    torch.save({"head_scores": torch.from_numpy(table)}, tmp_path / "s.pt")
    torch.save(torch.from_numpy(table), tmp_path / "s.pth")
    (tmp_path / "s.json").write_text(json.dumps(table.tolist()))
    (tmp_path / "s.csv").write_text("layer,h0,h1,h2\n" + "\n".join("," + ",".join(map(str, r)) for r in table.tolist()))
    for name in ("s.npy", "s.pt", "s.pth", "s.json", "s.csv"):
        got = load_scores(str(tmp_path / name))
        assert got.dtype == np.float32 and np.array_equal(got, table), name
