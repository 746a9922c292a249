"""The kernels.json report (counterpart of nuvla_forge/bench/bench_kernels.py).

CPU: the roofline verdict bands and the peak-bandwidth lookup.  GPU: a run at
tiny shapes produces the reference's schema (the keys bench/report.py:45-80
reads) with sane numbers, JSON-serialisable.
"""

from __future__ import annotations

import json

import pytest

from nuvla_forge_amd import bench_kernels as bk


def test_roofline_note_bands():
    assert "saturated" in bk.roofline_note(7000, 8000)
    assert "healthy" in bk.roofline_note(5000, 8000)
    assert "underutilised" in bk.roofline_note(3000, 8000)
    assert "poor" in bk.roofline_note(100, 8000)
    assert bk.roofline_note(4000, 8000).startswith("4000 GB/s = 50% of 8000 GB/s peak")


def test_peak_bandwidth_table():
    assert bk.peak_bw_for("gfx950") == 8000.0
    assert bk.peak_bw_for("gfx950", 123.0) == 123.0
    with pytest.raises(SystemExit):
        bk.peak_bw_for("gfx000")


def test_bandwidth_arithmetic():
    assert bk.bandwidth_gb_s(8_000_000_000, 1000.0) == pytest.approx(8.0)


@pytest.mark.gpu
def test_kernels_json_schema(cuda):
    import torch

    report = bk.run_all(torch.bfloat16, None, adaln=[(2, 16, 64)], swiglu=[(64, 128)],
                        ce=[(64, 32, 500)], iters=3, warmup=1, log=lambda *_: None)
    assert set(report) == {"device", "peak_bw_gb_s", "dtype", "adaln", "swiglu", "cross_entropy"}
    assert report["peak_bw_gb_s"] == 8000.0 and report["dtype"] == "bfloat16"
    for key in ("adaln", "swiglu"):
        (row,) = report[key]
        assert set(row) == {"shape", "dtype", "eager_ms", "fused_ms", "speedup", "achieved_gb_s",
                            "roofline"}
        assert row["fused_ms"] > 0 and row["eager_ms"] > 0 and row["achieved_gb_s"] > 0
    (ce,) = report["cross_entropy"]
    assert ce["shape"] == "M64xH32xV500"
    assert ce["chunked_peak_mib"] > 0 and ce["memory_reduction"] > 0
    json.dumps(report)
