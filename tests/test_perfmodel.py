"""The L0 performance model against the measured times recorded in the
MI355X machine file (predicted-vs-measured calibration)."""
from __future__ import annotations

from dslcompiler_amd import perfmodel


def test_model_tracks_measurements():
    rows = perfmodel.calibration_table()
    assert len(rows) >= 16
    for r in rows:
        assert 0.85 <= r["ratio"] <= 1.15, r
    # the steady-state shapes the constants were fitted on stay within 10%
    fit = [r for r in rows if (r["op"], r["M"]) in {("matmul", 4096), ("fused_swiglu", 8)}]
    assert fit and all(0.9 <= r["ratio"] <= 1.1 for r in fit), fit


def test_model_bounds():
    assert perfmodel.predict("fused_swiglu", 8, 14336, 4096)["bound"] == "hbm"
    assert perfmodel.predict("fused_swiglu", 2048, 11008, 4096)["bound"] == "mfma"
    p = perfmodel.predict("matmul", 255, 5120, 13824)
    assert p["plan"]["splits"] > 1 and p["memory_us"] > 0


def test_model_split_phases():
    """A k-split tile launch: the per-CU load term (one m tile: weights from
    HBM, X from L2) plus the partial-plane write burst of a single round,
    then the reduce kernel as a serial phase."""
    p = perfmodel.predict("fused_swiglu", 255, 13824, 5120)
    assert p["plan"]["kernel"] == "tile" and p["plan"]["splits"] == 2
    assert p["per_cu_us"] > max(p["compute_us"], p["memory_us"])
    assert p["reduce_us"] > 0
    assert abs(p["predicted_us"] - (p["per_cu_us"] + p["reduce_us"] + 3.0)) < 1e-6
    # no split: no reduce phase
    assert perfmodel.predict("fused_swiglu", 2048, 11008, 4096)["reduce_us"] == 0
