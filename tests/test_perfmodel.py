"""The L0 performance model against the measured times recorded in the
MI355X machine file (predicted-vs-measured calibration)."""
from __future__ import annotations

from dslcompiler_amd import perfmodel


def test_model_tracks_measurements():
    rows = perfmodel.calibration_table()
    assert len(rows) >= 16
    for r in rows:
        assert 0.5 <= r["ratio"] <= 1.5, r
    # the steady-state shapes the constants were fitted on stay within 10%
    fit = [r for r in rows if (r["op"], r["M"]) in {("matmul", 4096), ("fused_swiglu", 8)}]
    assert fit and all(0.9 <= r["ratio"] <= 1.1 for r in fit), fit


def test_model_bounds():
    assert perfmodel.predict("fused_swiglu", 8, 14336, 4096)["bound"] == "hbm"
    assert perfmodel.predict("fused_swiglu", 2048, 11008, 4096)["bound"] == "mfma"
    p = perfmodel.predict("matmul", 255, 5120, 13824)
    assert p["plan"]["splits"] > 1 and p["memory_us"] > 0
