"""The kernels.json report (nuvla_forge_amd.bench_kernels).

CPU: the peak lookup and the bandwidth arithmetic.  GPU: a run at tiny
shapes produces the schema the reference's renderer reads
(bench/report.py:45-80) with sane numbers, JSON-serialisable.
"""

from __future__ import annotations

import json

import pytest

from nuvla_forge_amd import bench_kernels as bk


def test_peak_lookup():
    assert bk.device_peak_gb_s("gfx950") == 8000.0
    assert bk.device_peak_gb_s("gfx950", 123.0) == 123.0
    assert bk.device_peak_gb_s("gfx000", 500.0) == 500.0
    with pytest.raises(SystemExit):
        bk.device_peak_gb_s("gfx000")


def test_bandwidth_arithmetic():
    assert bk.gb_per_s(8_000_000_000, 1000.0) == pytest.approx(8.0)
    assert bk.gb_per_s(167_874_560, 0.0262) == pytest.approx(6407.4, rel=1e-4)


@pytest.mark.gpu
def test_kernels_json_schema(cuda):
    import torch

    report = bk.run_all(torch.bfloat16, None, adaln=[(2, 16, 64)], swiglu=[(64, 128)],
                        ce=[(64, 32, 500)], steps=3, warmup=1, log=lambda *_: None)
    assert set(report) == {"device", "peak_bw_gb_s", "dtype", "adaln", "swiglu", "cross_entropy"}
    assert report["peak_bw_gb_s"] == 8000.0 and report["dtype"] == "bfloat16"
    for key in ("adaln", "swiglu"):
        (row,) = report[key]
        assert {"shape", "eager_ms", "fused_ms", "speedup", "achieved_gb_s"} <= set(row)
        assert row["fused_ms"] > 0 and row["eager_ms"] > 0 and row["achieved_gb_s"] > 0
        assert row["hbm_frac"] == pytest.approx(row["achieved_gb_s"] / 8000.0)
    assert report["adaln"][0]["bytes"] == 11 * 32 * 64 * 2
    assert report["swiglu"][0]["bytes"] == 8 * 64 * 128 * 2
    (ce,) = report["cross_entropy"]
    assert ce["shape"] == "M64xH32xV500"
    assert ce["chunked_peak_mib"] > 0 and ce["memory_reduction"] > 0
    json.dumps(report)
