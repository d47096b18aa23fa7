"""L0 performance model of the gfx950 kernels from the MI355X machine file
(machines/mi355x.yaml, `calibration`), for predicted-vs-measured checks.

For one call the model takes the dispatcher's launch plan
(llk_describe_launch) and returns
    compute = rounds x per-workgroup MFMA work / per-CU rate,
              rounds = ceil(workgroups / CUs)  (one workgroup per CU at a time)
    memory  = (weights + X + Y + split partials written and read back) / stream rate
    time    = max(compute, memory) + (launches - 1) x launch gap.
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
    else:
        groups = plan["workgroups"]
        mrows = 32 * math.ceil(M / 32)
        flops = 2.0 * nmat * mrows * N * K
        compute = flops / (min(groups, cus) * cal["small_m_flops_per_cu"])
    partials = 2.0 * plan["workspace_bytes"] if S > 1 else 0.0
    nbytes = 2.0 * nmat * K * N + 2.0 * M * K + 2.0 * M * N + partials
    memory = nbytes / cal["stream_bytes_per_s"]
    t = max(compute, memory) + (plan["launches"] - 1) * cal["launch_gap_s"]
    return {"compute_us": compute * 1e6, "memory_us": memory * 1e6, "predicted_us": t * 1e6,
            "bound": "mfma" if compute >= memory else "hbm", "plan": plan}


def calibration_table(machine_path: str = str(MACHINE)) -> list[dict]:
    """Predicted vs the measured times recorded in the machine file."""
    rows = []
    for r in machine(machine_path)["calibration"]["measured_us"]:
        p = predict(r["op"], r["M"], r["N"], r["K"], machine_path)
        rows.append({**r, "predicted_us": round(p["predicted_us"], 2), "bound": p["bound"],
                     "ratio": round(p["predicted_us"] / r["us"], 3)})
    return rows
