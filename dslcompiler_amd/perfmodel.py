"""L0 performance model of the gfx950 kernels from the MI355X machine file
(machines/mi355x.yaml, `calibration`), for predicted-vs-measured checks.

For one call the model takes the dispatcher's launch plan
(llk_describe_launch) and returns
    compute = rounds x per-workgroup MFMA work / per-CU rate,
              rounds = ceil(workgroups / CUs)  (one workgroup per CU at a time)
    memory  = (weights + X + Y + split partials written and read back) / stream rate
    per_cu  = small-M kernel only: rounds x max(weight share / per-CU weight rate,
              (weight share + X reads) / per-CU load rate); a workgroup reads
              X once per wave group, so at M = 64 X is as large as the weights
    time    = max(compute, memory, per_cu, shortest launch) + (launches - 1) x launch gap.
The small-M kernel's MFMA work counts whole 32-row groups.
"""
from __future__ import annotations

import math
from functools import lru_cache
from pathlib import Path

import yaml

from .ops import describe_launch

MACHINE = Path(__file__).resolve().parent / "machines" / "mi355x.yaml"


@lru_cache(maxsize=None)
def machine(path: str = str(MACHINE)) -> dict:
    with open(path) as f:
        return yaml.safe_load(f)


def predict(op: str, M: int, N: int, K: int, machine_path: str = str(MACHINE)) -> dict:
    m = machine(machine_path)
    # YAML 1.1 reads 1.0e12 as a string: convert explicitly
    cal = {k: float(v) for k, v in m["calibration"].items() if k != "measured_us"}
    cus = m["compute"]["owners"]["worker"]["count"]
    plan = describe_launch(op, M, N, K)
    nmat = 2 if op == "fused_swiglu" else 1
    S = plan["splits"]
    if plan["kernel"] == "tile":
        rows = 256 if op == "fused_swiglu" else 256  # MFMA rows per workgroup tile
        wg_flops = 2.0 * 256 * rows * math.ceil(K / 64) * 64 / S
        compute = math.ceil(plan["workgroups"] / cus) * wg_flops / cal["tile_flops_per_cu"]
    per_cu = 0.0
    if plan["kernel"] != "tile":
        groups = plan["workgroups"]
        mrows = 32 * math.ceil(M / 32)
        flops = 2.0 * nmat * mrows * N * K
        compute = flops / (min(groups, cus) * cal["small_m_flops_per_cu"])
        # The launcher's shape (SkinnyCfg in kernels/swiglu_decode.hip): a
        # wave covers GW = 2 column groups, except SwiGLU with M <= 32 and
        # workgroup width 1 (GW = 1); wave groups = width / GW.
        width = plan["group_width"]
        gw = 1 if (width == 1 or (nmat == 2 and M <= 32)) else 2
        kpart = math.ceil(K / 64) * 64 / S
        w_wg = width * 32 * kpart * 2.0 * nmat
        x_wg = (width // gw) * M * kpart * 2.0
        per_cu = math.ceil(groups / cus) * max(w_wg / cal["small_m_weight_bytes_per_cu_s"],
                                               (w_wg + x_wg) / cal["small_m_bytes_per_cu_s"])
    partials = 2.0 * plan["workspace_bytes"] if S > 1 else 0.0
    nbytes = 2.0 * nmat * K * N + 2.0 * M * K + 2.0 * M * N + partials
    memory = nbytes / cal["stream_bytes_per_s"]
    t = max(compute, memory, per_cu, cal["launch_min_s"]) + (plan["launches"] - 1) * cal["launch_gap_s"]
    return {"compute_us": compute * 1e6, "memory_us": memory * 1e6, "per_cu_us": per_cu * 1e6,
            "predicted_us": t * 1e6,
            "bound": "mfma" if compute >= max(memory, per_cu) else "hbm", "plan": plan}


def calibration_table(machine_path: str = str(MACHINE)) -> list[dict]:
    """Predicted vs the measured times recorded in the machine file."""
    rows = []
    for r in machine(machine_path)["calibration"]["measured_us"]:
        p = predict(r["op"], r["M"], r["N"], r["K"], machine_path)
        rows.append({**r, "predicted_us": round(p["predicted_us"], 2), "bound": p["bound"],
                     "ratio": round(p["predicted_us"] / r["us"], 3)})
    return rows
