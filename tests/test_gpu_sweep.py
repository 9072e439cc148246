"""Seeded sweep of request geometries against the CPU oracle (calls go through the C-ABI).

The fixed geometry lists elsewhere pick one case per kernel variant; this sweep draws
head count (1 - 64), block size, head_dim (power-of-two chunks down to 2 channels),
width, per-head levels, layer and block counts (up to 89 blocks: several workgroups per
job), symbol order, compress path and kernel family (MFMA, or the row or quad-per-row
FWHT forced) together from a fixed seed, so that combinations no list names (ragged
tile runs, several V groups at odd widths, one-block layers, levels at the top of a
width) are compared with the oracle as well.  The cases are the same on every run; each
prints its parameters before it touches the GPU.

Bars: those of the configuration tests (symbols |delta| <= 1 on <= 1e-4 of the elements,
metadata equal, dequantized KV within 1e-2 of the oracle's own round trip).

Levels reach 2^bits up to 6 bits.  From 7 bits on, a symbol can round up to 2^bits at
2^bits levels (quantizer_func.py:62-65 clamps to max_value, not max_value - 1), which
the reference's bitpack rejects (bitpack_codec.py:32, "symbol exceeds bitpack_bits"):
the sweep keeps those widths below 2^bits levels, since on the MFMA kernels the fp32
summation order may round such an element the other way, and a separate test pins the
rejection on the bit-exact row kernels.
"""

import os

import numpy as np
import pytest
import torch

from oracle import fused_v3 as fv
from oracle import kvpipe as kp
from test_gpu_configs import _bits, _check_layer, _oracle_profile

pytestmark = pytest.mark.gpu


def _cases(n: int, seed: int):
    rs = np.random.RandomState(seed)
    out = []
    while len(out) < n:
        H = int(rs.choice([1, 2, 3, 4, 5, 6, 8, 12, 16, 24, 32, 64]))
        S = int(rs.choice([1, 2, 4, 8, 16, 32]))
        D = int(rs.choice([6, 16, 64, 70, 80, 96, 100, 108, 128, 160, 224, 256]))
        bits = int(rs.randint(1, 9))
        if D * bits % 8 or H * (1 << (D - 1).bit_length()) > 8192:
            continue  # outside the engine's geometry range
        L = int(rs.randint(1, 4))
        B = int(rs.randint(1, 14)) if rs.rand() < 0.6 else int(rs.randint(14, 90))
        layout = str(rs.choice(["permuted", "native"]))
        path = str(rs.choice(["two_pass", "one_pass"]))
        fwht = str(rs.choice(["mfma", "mfma", "rows", "valu"]))
        if fwht == "valu" and not (D in (64, 128) and 128 % H == 0 and H <= 16):
            fwht = "mfma"  # the quad-per-row kernels' range
        out.append((H, S, D, bits, L, B, layout, path, fwht, int(rs.randint(1 << 30))))
    return out


# KVSERVE_AMD_SWEEP_CASES=N draws N cases instead of 48 (the same first 48)
@pytest.mark.parametrize("H,S,D,bits,L,B,layout,path,fwht,seed",
                         _cases(int(os.environ.get("KVSERVE_AMD_SWEEP_CASES", "48")), 20261202))
def test_sweep_matches_oracle(cuda, H, S, D, bits, L, B, layout, path, fwht, seed):
    from kvserve_amd.engine import FusedKVCodec, check_packet
    from kvserve_amd.profiles import per_head_profile
    from kvserve_amd.workloads import kv_blocks

    g = torch.Generator().manual_seed(seed)
    P = B + 5
    top = (1 << bits) - (1 if bits >= 7 else 0)
    pools = [torch.zeros((2, P, S, H, D), dtype=torch.bfloat16) for _ in range(L)]
    ids = torch.randperm(P, generator=g)[:B]
    for p in pools:
        p[:, ids] = kv_blocks(g, B, S, H, D, k_outliers=min(4, D))
    # per-head levels in [2, top]
    prof = []
    for _ in range(L):
        kl = [int(v) for v in torch.randint(2, top + 1, (H,), generator=g)]
        vl = [int(v) for v in torch.randint(2, top + 1, (H,), generator=g)]
        prof.append(per_head_profile(kl, vl))
    print(f"sweep H={H} S={S} D={D} bits={bits} L={L} B={B} {layout} {path} {fwht} seed={seed}", flush=True)
    pools = [p.to(cuda) for p in pools]
    dev_ids = ids.to(torch.int32).to(cuda)
    codec = FusedKVCodec(H, D, S, bits, 0xC0FEBABE, layout=layout, compress_path=path, fwht=fwht)
    packet = codec.compress(pools, dev_ids, prof)
    check_packet(packet)
    dst = [torch.zeros_like(p) for p in pools]
    codec.decompress(packet, dst, dev_ids)
    torch.cuda.synchronize()
    for l in range(L):
        _check_layer(packet, l, _bits(pools[l][:, dev_ids.long()]), _bits(dst[l][:, dev_ids.long()]))


def test_symbol_at_the_top_of_the_width_is_rejected_like_the_reference(cuda):
    """128 levels at 7 bits, D = 96 (the generic row kernels, bit-exact with the oracle):
    on this seeded request the oracle rounds some element to symbol 128 and rejects the
    layer; the engine's error check after the run raises the reference's bitpack error.
    With 127 levels the same request compresses and matches the oracle."""
    from kvserve_amd.engine import FusedKVCodec, check_packet
    from kvserve_amd.profiles import per_head_profile
    from kvserve_amd.workloads import kv_blocks

    H, S, D, bits, B = 32, 16, 96, 7, 11
    g = torch.Generator().manual_seed(1007978485)
    P = B + 5
    pool = torch.zeros((2, P, S, H, D), dtype=torch.bfloat16)
    ids = torch.randperm(P, generator=g)[:B]
    pool[:, ids] = kv_blocks(g, B, S, H, D)
    pools = [pool.to(cuda)]
    dev_ids = ids.to(torch.int32).to(cuda)
    x = _bits(pools[0][:, dev_ids.long()])
    for levels, rejects in ((128, True), (127, False)):
        prof = [per_head_profile([levels] * H, [levels] * H)]
        print(f"top of width: H={H} D={D} bits={bits} levels={levels}", flush=True)
        codec = FusedKVCodec(H, D, S, bits, 0xC0FEBABE, layout="native")
        if rejects:
            with pytest.raises(ValueError, match="symbol exceeds bitpack_bits"):
                kp.compress_request([x], list(range(B)), [_oracle_profile(prof[0])], codec.seed, bits,
                                    layout="native", layer_ids=[0], chunks=[(0, 1)])
            # the kernels flag the symbol; the check after the run raises it
            with pytest.raises(RuntimeError, match="symbol exceeds bitpack_bits"):
                check_packet(codec.compress(pools, dev_ids, prof), force=True)
        else:
            packet = codec.compress(pools, dev_ids, prof)
            check_packet(packet)
            _check_layer(packet, 0, x)


def _axes_cases(n: int, seed: int):
    rs = np.random.RandomState(seed)
    out = []
    while len(out) < n:
        H = int(rs.choice([1, 2, 3, 4, 6, 8, 12, 16, 32, 64]))
        S = int(rs.choice([1, 2, 4, 8, 16, 32]))
        D = int(rs.choice([6, 16, 64, 70, 96, 100, 128, 160, 256]))
        bits = int(rs.randint(1, 9))
        if D * bits % 8 or H * (1 << (D - 1).bit_length()) > 8192:
            continue
        axes = (str(rs.choice(kp.AXES)), str(rs.choice(kp.AXES)))
        L = int(rs.randint(1, 4))
        B = int(rs.randint(1, 14)) if rs.rand() < 0.6 else int(rs.randint(14, 60))
        layout = str(rs.choice(["permuted", "native"]))
        out.append((H, S, D, bits, axes[0], axes[1], L, B, layout, int(rs.randint(1 << 30))))
    return out


@pytest.mark.parametrize("H,S,D,bits,ak,av,L,B,layout,seed",
                         _axes_cases(int(os.environ.get("KVSERVE_AMD_SWEEP_CASES", "48")) // 2, 20261203))
def test_axes_sweep_matches_oracle_exactly(cuda, H, S, D, bits, ak, av, L, B, layout, seed):
    """Every quantization axis pair (quantizer_func.py:41-49) on drawn geometries, with
    head-split sections and per-head levels: the generic row kernels run the oracle's
    stage order, so the stream bytes, metadata and decompressed KV are bit-exact (a
    default pair on an MFMA geometry is held to the configuration bars instead)."""
    from kvserve_amd.engine import FusedKVCodec, check_packet
    from kvserve_amd.profiles import per_head_profile, section_profile
    from kvserve_amd.workloads import kv_blocks

    axes = (ak, av)
    g = torch.Generator().manual_seed(seed)
    P = B + 3
    top = (1 << bits) - (1 if bits >= 7 else 0)
    pools = [torch.zeros((2, P, S, H, D), dtype=torch.bfloat16) for _ in range(L)]
    ids = torch.randperm(P, generator=g)[:B]
    for p in pools:
        p[:, ids] = kv_blocks(g, B, S, H, D, k_outliers=min(4, D))
    prof = []
    for _ in range(L):
        lv = [int(v) for v in torch.randint(2, top + 1, (4,), generator=g)]
        # per-head levels need K on the channel axis: a K statistic shared over a group's
        # heads (token, tensor) takes one level count per group (profiles.py rejects others)
        if ak != "channel" or torch.rand(1, generator=g).item() < 0.5:
            prof.append(section_profile([bool(v) for v in torch.randint(0, 2, (H,), generator=g)], *lv))
        else:
            prof.append(per_head_profile([int(v) for v in torch.randint(2, top + 1, (H,), generator=g)],
                                         [int(v) for v in torch.randint(2, top + 1, (H,), generator=g)]))
    print(f"axes sweep {axes} H={H} S={S} D={D} bits={bits} L={L} B={B} {layout} seed={seed}", flush=True)
    pools = [p.to(cuda) for p in pools]
    dev_ids = ids.to(torch.int32).to(cuda)
    codec = FusedKVCodec(H, D, S, bits, 0xC0FEBABE, layout=layout, axes=axes)
    packet = codec.compress(pools, dev_ids, prof)
    check_packet(packet)
    dst = [torch.zeros_like(p) for p in pools]
    codec.decompress(packet, dst, dev_ids)
    torch.cuda.synchronize()
    if axes == ("channel", "token"):
        for l in range(L):
            _check_layer(packet, l, _bits(pools[l][:, dev_ids.long()]), _bits(dst[l][:, dev_ids.long()]))
        return
    per = 2 * H * B * S * D
    nb = per * bits // 8
    for l in range(L):
        x = _bits(pools[l][:, dev_ids.long()])
        ci = next(i for i, (s, e) in enumerate(packet.chunks) if s <= l < e)
        off = 16 + (l - packet.chunks[ci][0]) * nb
        stream = packet.streams[ci].cpu().numpy()
        op = _oracle_profile(packet.profiles[l])
        ch = kp.compress_request([x], list(range(B)), [op], packet.seed, bits, layout=layout,
                                 layer_ids=[packet.layer_ids[l]], chunks=[(0, 1)], axes=axes)[0]
        assert np.array_equal(stream[off:off + nb], ch.stream[16:]), (axes, l)
        m = ch.metas[0]
        for t, (mn, sc) in ((packet.kmeta[l], (m.kmin, m.kscale)), (packet.vmeta[l], (m.vmin, m.vscale))):
            got = t.float().cpu().numpy()
            assert np.array_equal(got[0, :mn.shape[0]], mn) and np.array_equal(got[1, :sc.shape[0]], sc), (axes, l)
        ref = np.zeros_like(x)
        kp.decompress_request([ch], [ref], list(range(B)), [op], packet.seed, bits, layout=layout,
                              layer_ids=[packet.layer_ids[l]], axes=axes)
        assert np.array_equal(_bits(dst[l][:, dev_ids.long()]), ref), (axes, l)


def _rans_cases(n: int, seed: int):
    rs = np.random.RandomState(seed)
    out = []
    for _ in range(n):
        w = int(rs.randint(1, 9))
        size = int(rs.choice([rs.randint(1, 4096), rs.randint(4096, 200000), rs.randint(200000, 700000)]))
        out.append((w, size, float(rs.choice([0.05, 0.3, 1.0, 5.0])), int(rs.randint(1 << 30))))
    return out


@pytest.mark.parametrize("w,n,conc,seed", _rans_cases(int(os.environ.get("KVSERVE_AMD_SWEEP_CASES", "48")) // 2,
                                                      20261204))
def test_rans_sweep_equals_oracle(cuda, w, n, conc, seed):
    """The GPU rANS stream of drawn symbol sequences (width, length, and per-64 Ki-block
    statistics from a Dirichlet of the drawn concentration, with some blocks uniform or
    a single symbol) is byte-equal to oracle/rans.c's, and decodes back on the GPU."""
    from kvserve_amd import ops
    from oracle import crans

    rng = np.random.default_rng(seed)
    A = 1 << w
    s = np.empty(n, np.uint8)
    for lo in range(0, n, 65536):
        m = min(65536, n - lo)
        kind = rng.integers(0, 6)
        if kind == 0:
            s[lo:lo + m] = rng.integers(0, A, m)
        elif kind == 1:
            s[lo:lo + m] = rng.integers(0, A)
        else:
            s[lo:lo + m] = rng.choice(A, m, p=rng.dirichlet(np.full(A, conc)))
    print(f"rans sweep w={w} n={n} conc={conc} seed={seed}", flush=True)
    body = crans.pack(s, w)
    st = ops.rans_encode(torch.from_numpy(body.copy()).to(cuda), n, w)
    ref = crans.encode_packed(body, n, w)
    got = st.cpu().numpy()
    assert got.size == ref.size and np.array_equal(got, ref), (w, n, conc, seed)
    assert np.array_equal(ops.rans_decode(st, n, w).cpu().numpy(), body)


def _runtime_cases(n: int, seed: int):
    rs = np.random.RandomState(seed)
    out = []
    for _ in range(n):
        block = int(rs.choice([8, 16, 32]))
        bpl = int(rs.choice([1, 2, 4]))
        opts = {"split_type": str(rs.choice(["layer", "head"])), "axis_key": str(rs.choice(kp.AXES)),
                "axis_value": str(rs.choice(kp.AXES)), "hybrid_ratio": float(rs.choice([0.0, 0.3, 0.8, 1.0]))}
        for name in ("high_key_num_levels", "low_key_num_levels", "high_value_num_levels", "low_value_num_levels"):
            opts[name] = int(rs.choice([rs.randint(2, 17), rs.randint(2, 257)]))
        out.append((int(rs.randint(1, 7)), int(rs.choice([1, 2, 4, 8])), int(rs.choice([32, 64, 128, 256])), block,
                    bpl, int(rs.randint(1, int(rs.randint(1, 25)) * block + 1)), opts, int(rs.randint(1 << 30))))
    return out


@pytest.mark.parametrize("layers,heads,dim,block,bpl,tokens,opts,seed",
                         _runtime_cases(int(os.environ.get("KVSERVE_AMD_SWEEP_CASES", "48")) // 4, 20261205))
def test_runtime_sweep_matches_oracle(tmp_path, layers, heads, dim, block, bpl, tokens, opts, seed):
    """The fixed-profile runtime on drawn model shapes, block sizes, blocks per logical
    block, partial tails, split types, quantization axes and level counts: payload, aux,
    raw tail, rANS stream and restored caches bit for bit against oracle/runtime_ref.py."""
    from test_gpu_runtime import runtime_vs_oracle

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    print(f"runtime sweep layers={layers} heads={heads} dim={dim} block={block} bpl={bpl} tokens={tokens} "
          f"{opts} seed={seed}", flush=True)
    runtime_vs_oracle(tmp_path, layers, heads, dim, block, bpl, tokens, opts, seed=seed, score_seed=seed + 1)


def _v3_cases(n: int, seed: int):
    rs = np.random.RandomState(seed)
    out = []
    for _ in range(n):
        H = int(rs.choice([1, 2, 4, 8, 16, 32, 64]))
        D = int(rs.choice([64, 128]))
        S = int(rs.choice([1, 3, 7, 16, 32]))
        B = int(rs.randint(1, 12)) if rs.rand() < 0.6 else int(rs.randint(12, 300))
        B = min(B, max(1, (1 << 21) // (S * H * D)))  # keeps the numpy oracle to seconds
        model = "Llama-3.1-8B-Instruct" if (H <= 8 and rs.rand() < 0.5) else None
        kw = {"hybrid_ratio": float(rs.choice([0.0, 0.3, 0.8, 1.0])), "split_type": str(rs.choice(["head", "layer"])),
              "high_key_max_value": int(rs.randint(2, 256)), "low_key_max_value": int(rs.randint(2, 256)),
              "high_value_max_value": int(rs.randint(2, 256)), "low_value_max_value": int(rs.randint(2, 256))}
        out.append((B, S, H, D, model, int(rs.randint(0, 32)), kw, int(rs.randint(1 << 30))))
    return out


@pytest.mark.parametrize("B,S,H,D,model,layer,kw,seed",
                         _v3_cases(int(os.environ.get("KVSERVE_AMD_SWEEP_CASES", "48")) // 4, 20261206))
def test_fused_quantizer_sweep_matches_oracle(cuda, B, S, H, D, model, layer, kw, seed):
    """impl "tilelang_fused" (kvmi_v3_*) on drawn layer shapes, level settings, split types
    and score-CSV head masks with tensor-parallel slices: float16 metadata, symbols and
    the dequantized layer bit for bit against oracle/fused_v3.py."""
    from kvserve_amd.compression.quantizer import FusedHadamardQuantizer

    print(f"v3 sweep B={B} S={S} H={H} D={D} model={model} layer={layer} {kw} seed={seed}", flush=True)
    kw = {"base_seed": seed, **kw}
    if model:
        kw["model_name"] = model
        if H != 8:
            kw.update(tensor_parallel_size=8 // H, tp_rank=(seed % (8 // H)))
    q = FusedHadamardQuantizer(**kw)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((2, B, S, H, D), generator=g)
    x[0, :, :, :, torch.randint(0, D, (3,), generator=g)] *= 10.0
    x = x.to(torch.bfloat16)
    sym, meta = q.quantize(layer, x.to(cuda))
    torch.cuda.synchronize()
    k_lv, v_lv = q.levels(layer, H)
    signs = kp.rademacher_signs(seed, layer, H, D)
    R = B * S
    xb = x.view(torch.int16).numpy().view(np.uint16).reshape(2, R, H, D)
    ref_q, ref_m = fv.compress_layer(xb, signs, k_lv, v_lv)
    km, vm = meta["key_meta"], meta["value_meta"]
    assert np.array_equal(km["min_val"].cpu().numpy(), ref_m["kmin"].astype(np.float16))
    assert np.array_equal(km["quant_scale"].cpu().numpy(), ref_m["kscale"].astype(np.float16))
    assert np.array_equal(vm["min_val"].cpu().numpy(), ref_m["vmin"].astype(np.float16))
    assert np.array_equal(vm["quant_scale"].cpu().numpy(), ref_m["vscale"].astype(np.float16))
    got = sym.cpu().numpy().reshape(2, R, H, D)
    assert np.array_equal(got, ref_q), int(np.count_nonzero(got != ref_q))
    out = q.dequantize(layer, sym, meta)
    torch.cuda.synchronize()
    ref_out = fv.decompress_layer(got, km["min_val"].cpu().numpy(), km["quant_scale"].cpu().numpy(),
                                  vm["min_val"].cpu().numpy(), vm["quant_scale"].cpu().numpy(), signs)
    assert np.array_equal(_bits(out).reshape(2, R, H, D), ref_out)
