"""GPU parity of the quantization axes (quantizer_func.py:41-49; KVServeQuantizer
axis_key / axis_value, kvserve_quantizer.py:136-139): every (axis_key, axis_value) pair
through the C-ABI paged kernels against the oracle, and the KVServeQuantizer operator
against the golden vectors the reference itself wrote (tests/golden/quantizer_axes.npz).

Non-default axes run on the generic row kernels, whose FWHT stage order is the oracle's:
symbols, metadata and the decompressed KV are bit-exact."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import kvpipe as kp

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
PAIRS = [(a, b) for a in kp.AXES for b in kp.AXES]


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def _oracle_profile(p):
    return kp.LayerProfile(kp.PartProfile(list(p.k_order), list(p.k_levels), list(p.k_groups())),
                           kp.PartProfile(list(p.v_order), list(p.v_levels), list(p.v_group)))


@pytest.mark.parametrize("axes", PAIRS, ids=["-".join(p) for p in PAIRS])
@pytest.mark.parametrize("H,D,bits,layout", [(8, 128, 4, "permuted"), (6, 96, 5, "native")])
def test_axes_match_oracle_exactly(cuda, axes, H, D, bits, layout):
    from kvserve_amd.engine import FusedKVCodec, check_packet
    from kvserve_amd.profiles import section_profile, whole_layer_profile
    from kvserve_amd.workloads import kv_blocks

    g = torch.Generator().manual_seed(PAIRS.index(axes) * 100 + H + D)
    L, B, S, P = 3, 6, 16, 16
    top = 2 ** bits - 1
    pools = [torch.zeros((2, P, S, H, D), dtype=torch.bfloat16) for _ in range(L)]
    ids = torch.randperm(P, generator=g)[:B]
    for p in pools:
        p[:, ids] = kv_blocks(g, B, S, H, D)
    prof = [section_profile([bool(v) for v in torch.randint(0, 2, (H,), generator=g)], top, top - 1,
                            max(2, top - 3), max(2, top - 4)) for _ in range(L - 1)]
    prof.append(whole_layer_profile(H, max(2, top - 2), top, is_low=True))  # one section
    print(f"axes {axes} H={H} D={D} bits={bits} {layout}", flush=True)
    pools = [p.to(cuda) for p in pools]
    dev_ids = ids.to(torch.int32).to(cuda)
    codec = FusedKVCodec(H, D, S, bits, 0xC0FEBABE, layout=layout, axes=axes)
    packet = codec.compress(pools, dev_ids, prof)
    check_packet(packet)
    dst = [torch.zeros_like(p) for p in pools]
    codec.decompress(packet, dst, dev_ids)
    torch.cuda.synchronize()
    per = 2 * H * B * S * D
    stream = packet.streams[0].cpu().numpy()
    for l in range(L):
        x = _bits(pools[l][:, dev_ids.long()])
        op = _oracle_profile(packet.profiles[l])
        ch = kp.compress_request([x], list(range(B)), [op], packet.seed, bits, layout=layout,
                                 layer_ids=[packet.layer_ids[l]], chunks=[(0, 1)], axes=axes)[0]
        nb = per * bits // 8
        assert np.array_equal(stream[16 + l * nb:16 + (l + 1) * nb], ch.stream[16:]), (axes, l)
        m = ch.metas[0]
        for t, (mn, sc) in ((packet.kmeta[l], (m.kmin, m.kscale)), (packet.vmeta[l], (m.vmin, m.vscale))):
            got = t.float().cpu().numpy()
            assert np.array_equal(got[0, :mn.shape[0]], mn) and np.array_equal(got[1, :sc.shape[0]], sc), (axes, l)
        ref = np.zeros_like(x)
        kp.decompress_request([ch], [ref], list(range(B)), [op], packet.seed, bits, layout=layout,
                              layer_ids=[packet.layer_ids[l]], axes=axes)
        assert np.array_equal(_bits(dst[l][:, dev_ids.long()]), ref), (axes, l)


def _golden_cases():
    z = np.load(GOLDEN / "quantizer_axes.npz")
    return sorted({k.rsplit("_x", 1)[0] for k in z.files if k.startswith("a") and k.endswith("_x")})


@pytest.mark.parametrize("key", _golden_cases())
def test_quantizer_operator_axes_match_reference_golden(cuda, key):
    """The KVServeQuantizer operator (C-ABI kernels, transform off, 8-bit native symbols)
    reproduces the reference's own outputs for every non-default axis pair."""
    from kvserve_amd.compression.quantizer.kvserve_quantizer import KVServeQuantizer

    z = np.load(GOLDEN / "quantizer_axes.npz")
    pi, ci, layer = key.split("_")
    ak, av = (kp.AXES[int(a)] for a in z[f"{pi}_axes"])
    cfgs = {1: dict(hybrid_ratio=0.8, high_key_max_value=12, high_value_max_value=8, low_key_max_value=6,
                    low_value_max_value=4, split_type="head"),
            2: dict(high_key_max_value=12, high_value_max_value=12, low_key_max_value=6, low_value_max_value=6,
                    split_type="layer")}
    quant = KVServeQuantizer(model_name="Llama-3.1-8B-Instruct", axis_key=ak, axis_value=av, **cfgs[int(ci[1:])])
    lid = int(layer[1:])
    x = torch.from_numpy(z[key + "_x"].view(np.int16)).view(torch.bfloat16).to(cuda)
    print(f"operator axes {ak}/{av} {key}", flush=True)
    q, meta = quant.quantize(lid, x)
    assert np.array_equal(q.cpu().numpy(), z[key + "_q"]), key
    for sec in ("high_key_meta", "high_value_meta", "low_key_meta", "low_value_meta"):
        mk = f"{key}_{sec}_min"
        if mk not in z.files:
            assert meta[sec]["min_val"] is None, (key, sec)
            continue
        for field, suffix in (("min_val", "min"), ("quant_scale", "scale")):
            want = z[f"{key}_{sec}_{suffix}"]
            got = meta[sec][field]
            assert tuple(got.shape) == want.shape and np.array_equal(_bits(got), want), (key, sec, field)
    deq = quant.dequantize(lid, q, meta)
    assert np.array_equal(_bits(deq), z[key + "_deq"]), key
