"""C-ABI and host-logic checks that need no GPU (no kernel is launched)."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kvserve_amd.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t)\s+(kvmi_\w+)\s*\(", text, flags=re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    from kvserve_amd import _lib

    lib = _lib.load()
    syms = declared_symbols()
    assert syms, "no declarations parsed"
    assert set(syms) == set(_lib.EXPORTS)
    for s in syms:
        assert hasattr(lib, s), s
    assert lib.kvmi_abi_version() == _lib.ABI_VERSION


def test_struct_layouts_match_header():
    from kvserve_amd import _lib

    assert ctypes.sizeof(_lib.Geometry) == 32
    assert _lib.JOB_BYTES == 104


def test_host_contract_errors_return_einval():
    """Argument checks happen on the host before any HIP call."""
    from kvserve_amd import _lib

    lib = _lib.load()
    E = _lib.EINVAL
    assert lib.kvmi_bitpack_encode(None, 4, 0, None, None, None) == E
    assert lib.kvmi_bitpack_encode(None, 4, 9, None, None, None) == E
    assert lib.kvmi_bitpack_decode(None, 16, 1, 4, None, None, None) == E
    buf = ctypes.create_string_buffer(32)
    err = ctypes.create_string_buffer(4)
    # wrong stream length for (n=5, bits=4): 16 + 3 bytes expected
    assert lib.kvmi_bitpack_decode(ctypes.addressof(buf), 18, 5, 4, ctypes.addressof(buf), ctypes.addressof(err),
                                   None) == E
    assert lib.kvmi_hadamard(None, None, 4, 8, 96, None, 0, None) == E
    g = _lib.Geometry()
    g.block_size, g.num_heads, g.head_dim, g.bits, g.max_groups = 16, 8, 128, 4, 2
    # head_dim: a multiple of 16 in [16, 256]; heads: 1..64 with heads * next_pow2(head_dim) <= 8192
    for bad in ({"head_dim": 100}, {"head_dim": 8}, {"head_dim": 272}, {"bits": 0}, {"num_heads": 0},
                {"num_heads": 65}, {"max_groups": 9}, {"num_heads": 64, "head_dim": 256, "max_groups": 2},
                {"num_heads": 48, "head_dim": 160}):
        gg = _lib.Geometry.from_buffer_copy(g)
        for field, value in bad.items():
            setattr(gg, field, value)
        for fn in (lib.kvmi_kstats_paged, lib.kvmi_encode_paged, lib.kvmi_decode_paged):
            assert fn(ctypes.byref(gg), None, 1, 1, None, None) == E, bad
    for good in ({"head_dim": 96}, {"num_heads": 3}, {"num_heads": 64}, {"head_dim": 256, "num_heads": 32}):
        gg = _lib.Geometry.from_buffer_copy(g)
        for field, value in good.items():
            setattr(gg, field, value)
        # a valid geometry with zero jobs returns before touching any pointer
        assert lib.kvmi_encode_paged(ctypes.byref(gg), None, 0, 1, None, None) == 0, good
    gg = _lib.Geometry.from_buffer_copy(g)
    gg.flags = _lib.F_NO_HEADER  # raw symbols need 8 bits
    assert lib.kvmi_encode_paged(ctypes.byref(gg), None, 1, 1, None, None) == E
    # zero jobs / zero blocks: nothing to do
    assert lib.kvmi_encode_paged(ctypes.byref(g), None, 0, 5, None, None) == 0
    # unknown flag bits are refused
    gg = _lib.Geometry.from_buffer_copy(g)
    gg.flags = 2048
    assert lib.kvmi_encode_paged(ctypes.byref(gg), None, 1, 1, None, None) == E
    # the device block-table check: no jobs is a no-op, bad arguments are refused
    assert lib.kvmi_check_block_ids(None, 0, None, None) == 0
    assert lib.kvmi_check_block_ids(None, -1, None, None) == E
    assert lib.kvmi_check_block_ids(None, 2, ctypes.addressof(err), None) == E
    assert lib.kvmi_check_block_ids(ctypes.addressof(buf), 2, None, None) == E


def test_rans_sizes_and_contract_errors():
    """Stream capacity is the raw-block bound of oracle/rans.c; bad arguments are
    rejected on the host."""
    from kvserve_amd import _lib
    from oracle import crans

    lib = _lib.load()
    E = _lib.EINVAL
    for n, w in ((0, 4), (1, 1), (65536, 4), (65537, 3), (3 * 65536 + 17, 8)):
        assert lib.kvmi_rans_max_bytes(n, w) == crans.max_bytes(n, w)
    assert lib.kvmi_rans_max_bytes(65536, 4) == 32 + 8 + 4 + 32768
    # per block: tag, table, 3 counts, 4 x 64 states; 4 word regions of guard + 16384 * 4 / 8
    assert lib.kvmi_rans_scratch_bytes(65536 * 2, 4) == 2 * (4 + 32 + 12 + 1024 + 4 * (4096 + 8192)) + 8
    assert lib.kvmi_rans_max_bytes(-1, 4) == E and lib.kvmi_rans_max_bytes(10, 0) == E
    assert lib.kvmi_rans_max_bytes(10, 9) == E and lib.kvmi_rans_scratch_bytes(10, 9) == E
    buf = ctypes.create_string_buffer(1 << 16)
    a = (ctypes.addressof(buf) + 7) // 8 * 8
    # capacity too small, misaligned pointers, missing pointers
    assert lib.kvmi_rans_encode(a, 100, 4, a, 10, a, 1 << 12, a, None) == E
    assert lib.kvmi_rans_encode(a, 100, 4, a + 1, 1 << 12, a, 1 << 12, a, None) == E
    assert lib.kvmi_rans_encode(None, 100, 4, a, 1 << 12, a, 1 << 12, a, None) == E
    assert lib.kvmi_rans_decode(a, 16, 100, 4, a, a, None) == E
    assert lib.kvmi_rans_decode(a + 4, 64, 100, 4, a, a, None) == E
    assert lib.kvmi_rans_decode(a, 64, 100, 0, a, a, None) == E


def test_profiles_validate_and_serialize():
    from kvserve_amd.profiles import LayerProfile, per_head_profile, section_profile, whole_layer_profile

    p = section_profile([True, False, False, False, False, False, True, False], 16, 16, 12, 12)
    assert p.k_order == [0, 6, 1, 2, 3, 4, 5, 7]
    assert p.v_group == [0, 0, 1, 1, 1, 1, 1, 1]
    p.validate(8)
    a = p.to_array()
    assert a.shape == (2, 3, 8) and a.dtype == np.uint8
    assert list(a[1, 1]) == [12, 12, 16, 16, 16, 16, 16, 16]
    q = per_head_profile([6, 12, 6, 6], [12, 6, 6, 12])
    assert q.v_order == [1, 2, 0, 3] and q.v_group == [0, 0, 1, 1] and q.v_levels == [6, 6, 12, 12]
    assert q.k_levels == [12, 6, 6, 6]
    q.validate(4)
    whole_layer_profile(8, 6, 6).validate(8)
    with pytest.raises(ValueError):
        LayerProfile([0, 0], [4, 4], [0, 1], [4, 4], [0, 0]).validate(2)
    with pytest.raises(ValueError):
        LayerProfile([0, 1], [4, 4], [0, 1], [4, 8], [0, 0]).validate(2)
    with pytest.raises(ValueError):
        LayerProfile([0, 1], [4, 1], [0, 1], [4, 4], [0, 0]).validate(2)


def test_profiles_from_reference_config_match_oracle():
    from oracle import kvpipe as kp
    from kvserve_amd.profiles import profiles_from_quantizer_config, scores_from_csv

    qc = dict(model_name="Llama-3.1-8B-Instruct", hybrid_ratio=0.3, high_key_max_value=16,
              high_value_max_value=16, low_key_max_value=12, low_value_max_value=8)
    prof = profiles_from_quantizer_config(qc, 32, 8)
    m = kp.head_mask_from_scores(scores_from_csv("Llama-3.1-8B-Instruct"), 0.3)
    for l in range(32):
        o = kp.head_split_profile(m[l], 16, 16, 12, 8)
        assert prof[l].k_order == o.k.order and prof[l].k_levels == o.k.levels
        assert prof[l].v_levels == o.v.levels and prof[l].v_group == o.v.group
    lay = profiles_from_quantizer_config({**qc, "split_type": "layer"}, 32, 8)
    assert [p.k_levels[0] for p in lay].count(12) == 11
    # TP: 2 ranks of 4 heads each see their own mask columns
    r1 = profiles_from_quantizer_config({**qc, "tp_rank": 1, "tensor_parallel_size": 2}, 32, 4)
    assert sorted(r1[0].k_order) == [0, 1, 2, 3]
    with pytest.raises(NotImplementedError):
        profiles_from_quantizer_config({**qc, "axis_key": "token"}, 1, 8)
    with pytest.raises(IndexError):
        profiles_from_quantizer_config(qc, 33, 8)


def test_chunk_rule():
    from kvserve_amd.engine import chunk_ranges

    assert chunk_ranges(32, 500 * 2 ** 20) == [(0, 32)]
    assert chunk_ranges(32, 500 * 2 ** 20 + 1) == [(0, 8), (8, 16), (16, 24), (24, 32)]
    assert chunk_ranges(9, 2 ** 30) == [(0, 8), (8, 9)]


def test_codec_constructor_contracts():
    from kvserve_amd.engine import FusedKVCodec

    for bits in (0, 9, True, 3.5, None):
        with pytest.raises(ValueError, match="bitpack_bits"):
            FusedKVCodec(8, 128, 16, bits)
    for H, D, b in ((8, 101, 4), (8, 100, 3), (8, 272, 4), (65, 64, 4), (64, 256, 4), (0, 128, 4)):
        with pytest.raises(ValueError, match="unsupported geometry"):
            FusedKVCodec(H, D, 16, b)  # odd D, 37.5-byte packed rows, too wide, too many heads, none
    FusedKVCodec(6, 96, 16, 4)  # D split into power-of-two chunks, H not dividing 128
    FusedKVCodec(8, 100, 16, 4)  # 64 + 32 + 4: a chunk below 16 channels (hadamard_func.py:63-64)
    with pytest.raises(ValueError):
        FusedKVCodec(8, 128, 16, 4, header=False)


def test_entropy_codec_switch_and_symbol_width():
    """codec_type "rans" / "nvcomp" (ANS) / "lc" take the rANS codec; quantized symbols
    of a profile whose largest level count is L are coded at bit_length(L) bits
    (the quantizer clamps to L inclusive), anything else as bytes."""
    from kvserve_amd.compression import CompressionConfig, KVServeCodec
    from kvserve_amd.compression.codec import BitPackCodec, RANSCodec
    from kvserve_amd.compression.compression_manager import symbol_bits

    for cc in ({"codec_type": "rans"}, {"codec_type": "nvcomp"}, {"codec_type": "nvcomp", "nvcomp_algorithm": "ANS"},
               {"codec_type": "lc", "lc_algorithm": "TUPL8_1 BIT_8 RZE_2"}, {}):
        assert isinstance(KVServeCodec(**cc).codec, RANSCodec), cc
    c = KVServeCodec(codec_type="rans")
    c.update_params(codec_type="bitpack", bitpack_bits=3)
    assert isinstance(c.codec, BitPackCodec) and c.codec.bitpack_bits == 3
    c.update_params(codec_type="lc")
    assert isinstance(c.codec, RANSCodec)
    with pytest.raises(ValueError, match="not available on the ROCm engine"):
        KVServeCodec(codec_type="nvcomp", nvcomp_algorithm="Zstd")
    with pytest.raises(ValueError, match="Invalid nvcomp's algorithm"):
        KVServeCodec(codec_type="nvcomp", nvcomp_algorithm="zip")
    with pytest.raises(ValueError, match="symbol_bits"):
        RANSCodec(symbol_bits=9)

    def cfg(pipe, cc, **levels):
        qc = {"high_key_max_value": 16, "high_value_max_value": 16, "low_key_max_value": 12,
              "low_value_max_value": 12, **levels}
        return CompressionConfig(enabled=True, pipeline=pipe, quantizer_config=qc, codec_config=cc)

    q = ["quantizer", "codec"]
    assert symbol_bits(cfg(q, {"codec_type": "bitpack", "bitpack_bits": 4})) == 4
    assert symbol_bits(cfg(q, {"codec_type": "nvcomp"})) == 5                      # L = 16 -> 0..16
    assert symbol_bits(cfg(q, {"codec_type": "nvcomp"}, high_key_max_value=6, high_value_max_value=6,
                           low_key_max_value=6, low_value_max_value=4)) == 3        # original_top_nvcomp.json
    assert symbol_bits(cfg(q, {"codec_type": "lc"}, high_key_max_value=12, high_value_max_value=8,
                           low_key_max_value=6, low_value_max_value=4)) == 4        # the reference default
    assert symbol_bits(cfg(["codec"], {"codec_type": "nvcomp"})) == 8              # lossless over raw bytes
    assert symbol_bits(cfg(q, {"codec_type": "rans"}, high_key_max_value=200)) == 8


def test_adapter_registry_contracts():
    from kvserve_amd.compression import (CompressionManager, FusedCompressionManager, KVCompressionAdapter,
                                         get_default_compression_config)

    base = {"pipeline": ["transformer", "quantizer", "codec"],
            "transformer_config": {"transform_type": "hadamard", "seed": 7},
            "quantizer_config": {"model_name": "Llama-3.1-8B-Instruct"},
            "codec_config": {"codec_type": "bitpack", "bitpack_bits": 4}}
    ad = KVCompressionAdapter(base, num_kv_heads=8, head_size=128)
    assert isinstance(ad._manager, FusedCompressionManager)
    assert ad._config.quantizer_config["tp_rank"] == 0
    hip = KVCompressionAdapter({**base, "quantizer_config": {"impl": "hip_fused"}}, 8, 128)
    assert isinstance(hip._manager, FusedCompressionManager)
    codec_only = KVCompressionAdapter({"pipeline": ["codec"], "codec_config": {"codec_type": "bitpack"}}, 8, 128)
    assert type(codec_only._manager) is CompressionManager
    # impl "tilelang_fused": the operator pipeline with the fused Hadamard quantizer
    tl = KVCompressionAdapter({**base, "quantizer_config": {"impl": "tilelang_fused"}}, 8, 128)
    assert type(tl._manager) is CompressionManager and tl._config.pipeline == ["quantizer", "codec"]
    assert type(tl._manager.quantizer).__name__ == "FusedHadamardQuantizer"
    for bad, exc in (({**base, "impl": "centered_codebook"}, ValueError),
                     ({**base, "pipeline": ["transformer", "zip"]}, ValueError),
                     ({**base, "codec_config": {"codec_type": "nvcomp", "nvcomp_algorithm": "LZ4"}}, ValueError),
                     ({**base, "codec_config": {"codec_type": "nvcomp", "nvcomp_algorithm": "Brotli"}}, ValueError),
                     ({**base, "codec_config": {"codec_type": "zip"}}, ValueError),
                     ({**base, "transformer_config": {"transform_type": "dct"}}, ValueError),
                     ({"mode": "controller", "library_path": "x"}, NotImplementedError)):
        with pytest.raises(exc):
            KVCompressionAdapter(bad, num_kv_heads=8, head_size=128)
    d = KVCompressionAdapter("default", num_kv_heads=4, head_size=128, model_name="Qwen2.5-7B-Instruct")
    assert d._config.quantizer_config["model_name"] == "Qwen2.5-7B-Instruct"
    assert get_default_compression_config()["codec_config"] == {"codec_type": "nvcomp", "nvcomp_algorithm": "ANS",
                                                                "data_type": "|u1"}
    for cc in ({"codec_type": "nvcomp"}, {"codec_type": "lc", "lc_algorithm": "TUPL8_1 BIT_8 RZE_2"},
               {"codec_type": "rans"}):
        assert isinstance(KVCompressionAdapter({**base, "codec_config": cc}, 8, 128)._manager,
                          FusedCompressionManager)


def test_quantizer_validation_matches_reference_asserts():
    from kvserve_amd.compression import KVServeQuantizer

    for kw in ({"hybrid_ratio": 1.5}, {"low_key_max_value": 0}, {"high_value_max_value": 255},
               {"low_key_max_value": 16, "high_key_max_value": 12}, {"axis_key": "row"}, {"split_type": "x"}):
        with pytest.raises(AssertionError):
            KVServeQuantizer(**kw)
    q = KVServeQuantizer(split_type="layer", low_key_max_value=6, high_key_max_value=12)
    assert q.layer_profile(31, 8).k_levels == [6] * 8 and q.layer_profile(0, 8).k_levels == [12] * 8
    assert q.layer_profile(31, 8).n_low == 8 and q.layer_profile(0, 8).n_low == 0


def test_v3_sizes_and_contract_errors():
    """The fused quantizer's scratch: up to 256 K partials [2][H][D] uint32,
    whatever the row count; unsupported shapes and misaligned buffers are rejected on the host
    (no kernel runs: every pointer below is a small integer)."""
    from kvserve_amd import _lib

    lib = _lib.load()
    E = _lib.EINVAL
    assert lib.kvmi_v3_scratch_bytes(100, 8, 128) == 256 * 2 * 8 * 128 * 4
    assert lib.kvmi_v3_scratch_bytes(3, 4, 64) == 256 * 2 * 4 * 64 * 4
    for bad in ((5, 8, 96), (5, 3, 128), (5, 128, 128), (-1, 8, 128)):
        assert lib.kvmi_v3_scratch_bytes(*bad) == -1
    assert lib.kvmi_v3_compress(None, 4, 8, 96, None, None, None, None, None, None, None, None) == E
    assert lib.kvmi_v3_compress(None, 0, 8, 128, None, None, None, None, None, None, None, None) == 0
    assert lib.kvmi_v3_compress(None, 4, 8, 128, None, None, None, None, None, None, None, None) == E
    assert lib.kvmi_v3_compress(8, 4, 8, 128, 16, 16, 16, 16, 16, 16, 16, None) == E  # x misaligned
    assert lib.kvmi_v3_compress(16, 4, 8, 128, 16, 16, 16, 24, 16, 16, 16, None) == E  # q misaligned
    assert lib.kvmi_v3_compress(16, 4, 8, 128, 16, 16, 16, 16, 8, 16, 16, None) == E  # kmeta misaligned
    assert lib.kvmi_v3_decompress(16, 4, 8, 128, 16, 16, 16, 8, None) == E  # out misaligned
    assert lib.kvmi_v3_decompress(16, 4, 8, 128, 16, 8, 16, 16, None) == E  # kmeta16 misaligned


def test_v3_noalloc_contract_errors():
    """kvmi_v3_compress_noalloc checks shapes, pointers and its fixed scratch capacity on
    the host before any HIP call (every pointer below is a small integer)."""
    from kvserve_amd import _lib

    lib = _lib.load()
    f = lib.kvmi_v3_compress_noalloc
    assert f(16, 4, 8, 96, 16, 16, 16, 16, 16, 16, None) == _lib.EINVAL  # head_dim
    assert f(16, 0, 8, 128, 16, 16, 16, 16, 16, 16, None) == _lib.OK  # nothing to do
    assert f(None, 4, 8, 128, 16, 16, 16, 16, 16, 16, None) == _lib.EINVAL
    assert f(8, 4, 8, 128, 16, 16, 16, 16, 16, 16, None) == _lib.EINVAL  # x misaligned
    # 64 heads x 128: 256 partials of 64 KiB = 16 MiB > the 4 MiB array
    assert f(16, 1024, 64, 128, 16, 16, 16, 16, 16, 16, None) == _lib.ENOSPC
    # few rows: fewer partials, and 8 partials of 64 KiB fit
    need = lambda rows, H, D: min(-(-rows * H // 64), 256) * 8 * H * D
    assert need(8, 64, 128) <= _lib.V3_NOALLOC_SCRATCH_BYTES < need(1024, 64, 128)
    with pytest.raises(ValueError, match="KVMI_ENOSPC"):
        _lib.check(_lib.ENOSPC, "kvmi_v3_compress_noalloc")


@pytest.mark.parametrize("axes", [("channel", "token"), ("token", "channel"), ("tensor", "tensor"),
                                  ("channel", "channel"), ("token", "tensor")])
def test_metadata_dicts_follow_each_axis_and_round_trip(axes):
    """Reference-format section dicts are views of the engine tables with the keepdim
    shapes of quantizer_func.py:52-53 on every axis; tables_from_dicts returns views of
    the same allocation, and a copy elsewhere still converts back to equal tables."""
    import torch

    from kvserve_amd.compression._meta import layer_dict, tables_from_dicts
    from kvserve_amd.engine import meta_shape
    from kvserve_amd.profiles import section_profile

    H, D, B, S, L, G = 4, 32, 3, 16, 2, 2
    prof = section_profile([True, False, True, False], 12, 8, 6, 4)
    shapes = [meta_shape(a, H, D, G, B * S) for a in axes]
    sizes = [L * 2 * r * c for r, c in shapes]
    buf = torch.arange(sum(sizes), dtype=torch.float32).to(torch.bfloat16)
    kmeta = buf[:sizes[0]].view(L, 2, *shapes[0])
    vmeta = buf[sizes[0]:].view(L, 2, *shapes[1])
    dicts = [layer_dict(kmeta[l], vmeta[l], prof, B, S, axes) for l in range(L)]
    want = {"channel": (1, 1, 2, D), "token": (B, S, 1, 1), "tensor": (1, 1, 1, 1)}
    for d in dicts:
        for name, axis in (("low_key_meta", axes[0]), ("high_value_meta", axes[1])):
            assert tuple(d[name]["min_val"].shape) == want[axis], (name, axis)
            assert d[name]["min_val"].untyped_storage().data_ptr() == buf.untyped_storage().data_ptr()
    k2, v2 = tables_from_dicts(dicts, H, D, B, S, "cpu", axes)
    assert k2.data_ptr() == kmeta.data_ptr() and torch.equal(k2, kmeta) and torch.equal(v2, vmeta)
    copies = [{k: ({f: (t.clone() if isinstance(t, torch.Tensor) else t) for f, t in v.items()}
                   if isinstance(v, dict) else v) for k, v in d.items()} for d in dicts]
    k3, v3 = tables_from_dicts(copies, H, D, B, S, "cpu", axes)
    assert k3.data_ptr() != kmeta.data_ptr() and torch.equal(k3, kmeta) and torch.equal(v3, vmeta)


def test_job_table_rows_address_each_layer():
    """The vectorised job table holds, per layer, the address of that layer's slice of
    every table (as indexing the tensors gives it), its chunk's stream and offsets."""
    import torch

    from kvserve_amd import _lib
    from kvserve_amd.engine import FusedKVCodec

    codec = FusedKVCodec(4, 64, 16, 4, axes=("channel", "tensor"))
    L, B = 5, 3
    pools = [torch.zeros((2, 7, 16, 4, 64), dtype=torch.bfloat16) for _ in range(L)]
    ids = torch.arange(B, dtype=torch.int32)
    chunks = [(0, 2), (2, 5)]
    streams = [torch.empty(100, dtype=torch.uint8), torch.empty(200, dtype=torch.uint8)]
    buf = torch.empty(L * 2 * 4 * 64 + L * 2 * 2, dtype=torch.bfloat16)
    kmeta, vmeta = buf[:L * 2 * 4 * 64].view(L, 2, 4, 64), buf[L * 2 * 4 * 64:].view(L, 2, 2, 1)
    signs = torch.zeros((L, 4, 2), dtype=torch.int32)
    prof = torch.zeros((L, 2, 3, 4), dtype=torch.uint8)
    keys = torch.zeros((L, 2, 2, 4, 64), dtype=torch.int32)
    rows = codec._job_rows(pools, ids, streams, chunks, kmeta, vmeta, signs, prof, keys, B)
    assert rows.shape == (L, _lib.JOB_INT64S)
    per = 2 * 4 * B * 16 * 64
    for l in range(L):
        ci = 0 if l < 2 else 1
        s, e = chunks[ci]
        want = [pools[l].data_ptr(), ids.data_ptr(), streams[ci].data_ptr(), kmeta[l].data_ptr(), vmeta[l].data_ptr(),
                signs[l].data_ptr(), prof[l].data_ptr(), keys[l].data_ptr(), 7, 7 * 16 * 4 * 64, (l - s) * per,
                (e - s) * per, B | ((1 if l == s else 0) << 32)]
        assert rows[l].tolist() == want, l


def test_profile_validation_and_table_follow_content():
    """Validation and the device profile table are cached by profile content: a
    profile edited in place after a successful plan is validated (and uploaded) again."""
    import torch

    from kvserve_amd.engine import FusedKVCodec
    from kvserve_amd.profiles import section_profile

    codec = FusedKVCodec(4, 64, 16, 4)
    profs = [section_profile([True, False, False, True], 16, 16, 12, 12) for _ in range(3)]
    key = codec._profile_key(profs)
    codec._validate_profiles(profs, key)
    t0 = codec._profile_table(profs, "cpu")
    assert codec._profile_table(profs, "cpu") is t0
    assert torch.equal(t0, torch.from_numpy(np.stack([p.to_array() for p in profs])))
    profs[1].v_order[0] = profs[1].v_order[1]  # no longer a permutation
    with pytest.raises(ValueError, match="permutation"):
        codec._validate_profiles(profs, codec._profile_key(profs))
    profs[1].v_order[:] = [3, 0, 1, 2]
    codec._validate_profiles(profs, codec._profile_key(profs))
    t1 = codec._profile_table(profs, "cpu")
    assert t1 is not t0 and t1[1, 1, 0].tolist() == [3, 0, 1, 2]


def test_flag_and_error_constants_match_the_header():
    """The Python mirror's KVMI_F_* and KVMI_ERR_* values are the header's."""
    from kvserve_amd import _lib

    text = HEADER.read_text()
    flags = dict(re.findall(r"#define KVMI_F_(\w+) (\d+)u", text))
    errs = dict(re.findall(r"#define KVMI_ERR_(\w+) (\d+)", text))
    assert "ROW_FWHT" in flags and "BLOCK_ID" in errs
    for name, v in flags.items():
        assert getattr(_lib, "F_" + name) == int(v), name
    for name, v in errs.items():
        assert getattr(_lib, "ERR_" + name) == int(v), name


def test_fwht_choice_sets_its_flag():
    """fwht='valu' / 'rows' force the quad-per-row / generic row kernels through their flags."""
    from kvserve_amd import _lib
    from kvserve_amd.engine import FusedKVCodec

    assert FusedKVCodec(8, 128, 16, 4, fwht="mfma")._flags(16) & (_lib.F_VALU_FWHT | _lib.F_ROW_FWHT) == 0
    assert FusedKVCodec(8, 128, 16, 4, fwht="valu")._flags(16) & _lib.F_VALU_FWHT
    assert FusedKVCodec(8, 128, 16, 4, fwht="rows")._flags(16) & _lib.F_ROW_FWHT
    with pytest.raises(ValueError):
        FusedKVCodec(8, 128, 16, 4, fwht="dpp")
