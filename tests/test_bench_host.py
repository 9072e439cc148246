"""bench.py host logic that needs no GPU: reading profiled HBM traffic from the
committed rocprofv3 summaries."""

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import bench  # noqa: E402

TABLE = """Calibration: a 1 GiB device copy reads FETCH_SIZE = 524302 KiB and WRITE_SIZE = 1048576 KiB, so FETCH_SIZE is scaled by 2.000 and WRITE_SIZE by 1.000.

| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | scaled read MiB | scaled write MiB |
|---|---|---|---|---|
| good_kernel | 1024 | 512 | 2.0 | 0.5 |
| bad_kernel | 6 | 4.2 | 4.1 | 4.7 |
"""


def test_profiled_traffic_uses_consistent_rows_only(tmp_path):
    (tmp_path / "k_wlx.md").write_text(TABLE)
    assert bench.profiled_traffic("good_kernel", "wlx", tmp_path) == int(round(2.5 * 2**20))
    # a row whose scaled MiB do not follow from its KiB columns is not evidence
    assert bench.profiled_traffic("bad_kernel", "wlx", tmp_path) is None
    assert bench.profiled_traffic("missing", "wlx", tmp_path) is None
    # no calibration statement: nothing is read
    (tmp_path / "k_wly.md").write_text(TABLE.split("\n", 1)[1])
    assert bench.profiled_traffic("good_kernel", "wly", tmp_path) is None


def test_committed_config2_summary_is_consistent():
    for k in ("encode_mfma_kernel<4, 4, false>", "kstats_mfma_kernel<4>", "kstats_finalize_kernel"):
        assert bench.profiled_traffic(k, "config2") is not None, k


def test_config2_kernel_names_have_committed_profiles():
    """Every kernel the default bench line names for config 2 has a consistent row in the
    committed summary (the roofline's traffic field reads it)."""
    from types import SimpleNamespace

    codec = SimpleNamespace(axes=("channel", "token"), fwht="mfma", transform=True)
    names = bench.hip_kernel_names(codec, 16, 8, 128, 4)
    assert names["kvmi_decode_paged"] == "decode_kt_kernel<8>"
    for k in names.values():
        assert bench.profiled_traffic(k, "config2") is not None, k


def test_kernel_names_follow_the_forced_fwht():
    """The bench names the kernels the forced register-FWHT families launch."""
    from types import SimpleNamespace

    for fwht, enc in (("valu", "encode_kernel<128, 4>"), ("rows", "rows_encode_kernel<8, 4>")):
        codec = SimpleNamespace(axes=("channel", "token"), fwht=fwht, transform=True)
        assert bench.hip_kernel_names(codec, 16, 8, 128, 4)["kvmi_encode_paged"] == enc


def test_settle_phase_is_off_at_zero_and_a_flag_of_the_bench():
    """--settle-ms 0 runs no untimed steps; the default settles before the warmup."""
    calls = []
    assert bench.settle_device(lambda: calls.append(1), 0) == 0 and not calls
    import inspect

    assert "--settle-ms" in inspect.getsource(bench.main)
