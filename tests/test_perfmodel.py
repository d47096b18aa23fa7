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
    p = perfmodel.predict("matmul", 255, 5120, 13824)
    assert p["plan"]["kernel"] == "tile" and p["plan"]["splits"] == 12
    assert p["per_cu_us"] > max(p["compute_us"], p["memory_us"])
    assert p["reduce_us"] > 0
    assert abs(p["predicted_us"] - (p["per_cu_us"] + p["reduce_us"] + 3.0)) < 1e-6


def _engines():
    import yaml
    from pathlib import Path
    path = Path(perfmodel.__file__).resolve().parent / "machines" / "mi355x.yaml"
    doc = yaml.safe_load(path.read_text())
    return doc, {e["name"]: e for e in doc["compute"]["matrix_engines"]}


def _profile_mfma_rates():
    """Register-only MFMA rates (TFLOP/s) from the committed profile table
    `| v_mfma_... | N(0,1) | constant |`."""
    import re
    from pathlib import Path
    text = (Path(__file__).resolve().parents[1] / "profiles" /
            "swiglu_prefill_clock_vs_operand_data.md").read_text()
    rates = {}
    for form, rnd, const in re.findall(
            r"\|\s*`v_mfma_f32_(\d+x\d+x\d+)_bf16`\s*\|\s*([0-9.]+) TFLOP/s\s*\|\s*([0-9.]+) TFLOP/s",
            text):
        rates[form] = (float(rnd), float(const))
    return rates


def test_matrix_engines_match_spec_and_measurements():
    """Both bf16 MFMA forms issue at the full 1024 flops per SIMD-cycle (the
    spec peak), back-to-back issue = flops per instruction / 1024, and the
    sustained rates equal the committed register-only measurements."""
    doc, eng = _engines()
    rates = _profile_mfma_rates()
    assert set(rates) == {"32x32x16", "16x16x32"}, rates
    simds = doc["compute"]["owners"]["vector_engine"]["count"]
    for form, (rnd, const) in rates.items():
        e = eng[f"mfma-bf16-{form}"]
        m, n, k = e["tile_shapes"][0]
        assert e["flops_per_cycle"] == 1024, e
        assert e["issue_cycles"] * e["flops_per_cycle"] == 2 * m * n * k, e
        peak = e["flops_per_cycle"] * e["count"] * doc["clock_hz"]
        assert abs(peak - 2.5e15) / 2.5e15 < 0.02 and e["count"] == simds
        assert abs(e["sustained_flops_random_operands"] - rnd * 1e12) / (rnd * 1e12) < 0.01, form
        assert abs(e["sustained_flops_constant_operands"] - const * 1e12) / (const * 1e12) < 0.01
        assert e["sustained_flops_random_operands"] < e["sustained_flops_constant_operands"] <= peak
    # the 16x16x32 form keeps more of its rate on random data (the tile kernel's choice)
    assert (eng["mfma-bf16-16x16x32"]["sustained_flops_random_operands"] >
            eng["mfma-bf16-32x32x16"]["sustained_flops_random_operands"])
    # the fitted tile-kernel rate cannot exceed the register-only rate of its MFMA form
    cal = doc["calibration"]
    workers = doc["compute"]["owners"]["worker"]["count"]
    assert float(cal["tile_flops_per_cu"]) * workers < eng["mfma-bf16-16x16x32"][
        "sustained_flops_random_operands"]


def test_partial_round_runs_at_a_higher_clock():
    """The tile kernel's partly filled last round costs f_full / f(busy)
    of a full round (the clock climbs from 1.80 GHz with every CU busy
    toward 2.4 GHz as CUs fall idle, profiles/tile_kernel_cycles_per_stage.md):
    config 3's 688 tiles (2 full rounds + 176 of 256) cost between 2.69 and
    3 rounds, a single full round (GEMM 4096^3) exactly one."""
    import dslcompiler_amd as llk
    cal = {k: float(v) for k, v in perfmodel.machine()["calibration"].items() if k != "measured_us"}
    t_round = 2.0 * 256 * 256 * 4096 / cal["tile_flops_per_cu"] * 1e6
    old = llk.get_tunable("tile_wide")
    llk.set_tunable("tile_wide", 0)  # the 128-column kernel (the default plan is the wide one)
    try:
        p3 = perfmodel.predict("fused_swiglu", 2048, 11008, 4096)
    finally:
        llk.set_tunable("tile_wide", old)
    assert p3["plan"]["workgroups"] == 688
    f_full, f_idle = cal["tile_clock_full_hz"], cal["tile_clock_idle_hz"]
    occ = (688 - 512) / 256
    want = (2 + f_full / (f_idle - (f_idle - f_full) * occ)) * t_round
    assert abs(p3["compute_us"] - want) < 1e-6 * want
    # the wide kernel (B = 11): 504 workgroups of 352 MFMA rows, 1 full round
    # + 248 of 256
    pw = perfmodel.predict("fused_swiglu", 2048, 11008, 4096)
    assert (pw["plan"]["kernel"], pw["plan"]["workgroups"]) == ("wide_tile", 504)
    occ = (504 - 256) / 256
    want = (1 + f_full / (f_idle - (f_idle - f_full) * occ)) * t_round * 352 / 256
    assert abs(pw["compute_us"] - want) < 1e-6 * want
    assert 2.69 * t_round < p3["compute_us"] < 3 * t_round
    p2 = perfmodel.predict("matmul", 4096, 4096, 4096)
    assert p2["plan"]["workgroups"] == 256
    assert abs(p2["compute_us"] - t_round) < 1e-6 * t_round
