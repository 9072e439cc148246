"""The seeded GPU sweeps draw inputs the engine accepts (CPU): every drawn geometry is a
supported one, the fixed seed gives the same cases on every run, a larger case count
extends the default list, and the drawn runtime options pass the configuration's own
validation.  A sweep whose cases the host rejected would pass without touching a kernel."""

import numpy as np
import pytest

import test_gpu_sweep as sw
from kvserve_amd.engine import supported_geometry


def test_sweep_cases_are_supported_and_stable():
    cases = sw._cases(48, 20261202)
    assert cases == sw._cases(48, 20261202)
    assert sw._cases(200, 20261202)[:48] == cases
    for H, S, D, bits, L, B, layout, path, fwht, seed in cases:
        assert supported_geometry(H, D, bits), (H, D, bits)
        assert 1 <= L <= 3 and 1 <= B < 90 and S in (1, 2, 4, 8, 16, 32)
        assert layout in ("permuted", "native") and path in ("two_pass", "one_pass")
        assert fwht in ("mfma", "rows", "valu")
        if fwht == "valu":  # forced only where the quad-per-row kernels run
            assert D in (64, 128) and 128 % H == 0 and H <= 16
    # the draw covers every kernel family, both paths and multi-workgroup jobs
    assert {c[8] for c in cases} == {"mfma", "rows", "valu"}
    assert {c[7] for c in cases} == {"two_pass", "one_pass"}
    assert max(c[5] for c in cases) >= 14


def test_axes_cases_cover_every_pair():
    cases = sw._axes_cases(400, 20261203)
    for H, S, D, bits, ak, av, L, B, layout, seed in cases:
        assert supported_geometry(H, D, bits), (H, D, bits)
    assert {(c[4], c[5]) for c in cases} == {(a, b) for a in ("channel", "token", "tensor")
                                             for b in ("channel", "token", "tensor")}


def test_runtime_cases_pass_config_validation():
    from kvserve_amd.runtime import CompressionConfig

    for layers, heads, dim, block, bpl, tokens, opts, seed in sw._runtime_cases(100, 20261205):
        assert block % bpl == 0 and 1 <= tokens
        cfg = CompressionConfig.from_extra_config({"compression": {"enable-compression-pipeline": True,
                                                                  "logical_blocks_per_chunk": 1, **opts}})
        assert cfg.split_type == opts["split_type"] and cfg.axis_value == opts["axis_value"]


@pytest.mark.parametrize("n", [0, 7])
def test_fused_and_rans_case_counts(n):
    assert len(sw._v3_cases(n, 1)) == n and len(sw._rans_cases(n, 1)) == n
    for B, S, H, D, model, layer, kw, seed in sw._v3_cases(50, 20261206):
        assert 64 % H == 0 and D in (64, 128) and B * S * H * D <= max(1 << 21, S * H * D)
        assert all(2 <= kw[k] <= 255 for k in kw if k.endswith("_max_value"))
    assert np.all([1 <= w <= 8 for w, *_ in sw._rans_cases(50, 20261204)])
