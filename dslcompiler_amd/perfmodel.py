"""L0 performance model of the gfx950 kernels from the MI355X machine file
(machines/mi355x.yaml, `calibration`), for predicted-vs-measured checks.

For one call the model takes the dispatcher's launch plan
(llk_describe_launch) and returns
    compute = rounds x per-workgroup MFMA work / per-CU rate,
              rounds = ceil(workgroups / CUs)  (one workgroup per CU at a time);
              in the tile kernel a partly filled last round counts
              f_full / f(busy fraction), the clock rising linearly from
              f_full (every CU busy) toward f_idle as CUs fall idle
    memory  = (weights + X + Y, or the partial planes written instead of Y) / stream rate
    per_cu  = per-CU loads.  Tile kernel: rounds x (weight panel / weight rate
              + X panel / L2 rate), the weight rate being HBM's when there is
              one m tile (each weight byte is read once, from HBM) and L2's
              otherwise; a single-round k split adds the partial-plane write
              burst that every workgroup issues at the same moment.
              Small-M kernel: rounds x max(weight share / per-CU weight rate,
              (weight share + X reads) / per-CU load rate); a workgroup reads
              X once per wave group, so at M = 64 X is as large as the weights.
              Decode tile kernel: rounds x (ring fill + (weights + M rows of
              X per 64-k step) / its per-CU rate), its weights streamed
              (non-temporal) at its own stream rate; a k split adds the
              reduce pass
    reduce  = tile k split only: the reduce kernel reads the partial planes and
              writes Y, after the main kernel
    time    = max(compute, memory, per_cu, shortest launch) + reduce
              + (launches - 1) x launch gap.
A tile-kernel tail split (head_blocks_n > 0) is two such launches in a row:
the leading columns unsplit, the remaining columns with the k split.  The
wide SwiGLU kernel is the tile kernel's model with 2 x tile_columns MFMA
rows per workgroup (its k split's register-order partials counted like the
partial planes).
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


def _tile_launch(cal: dict, cus: int, nmat: int, M: int, N: int, K: int, S: int,
                 workgroups: int, rows: int = 256) -> tuple[float, float, float, float]:
    """(compute, memory, per_cu, reduce) seconds of one tile-kernel launch
    over N columns with S k splits (and its reduce kernel when S > 1).
    rows: MFMA rows of the workgroup tile -- 256 for mfma_tile_kernel
    (SwiGLU: 128 n of Wg + 128 n of Wu), 2 x 16 B for the wide SwiGLU kernel
    (16 B columns of each matrix)."""
    kpart = math.ceil(K / 64) * 64 / S
    rounds = math.ceil(workgroups / cus)
    # A partly filled round runs at a higher clock: the board holds
    # tile_clock_full_hz with every CU busy and climbs toward
    # tile_clock_idle_hz as CUs fall idle (linear in the busy fraction).
    full, occ = divmod(workgroups, cus)
    occ /= cus
    f_full, f_idle = cal["tile_clock_full_hz"], cal["tile_clock_idle_hz"]
    eff_rounds = full + (f_full / (f_idle - (f_idle - f_full) * occ) if occ else 0.0)
    compute = eff_rounds * 2.0 * 256 * rows * kpart / cal["tile_flops_per_cu"]
    # Per-CU loads: one m tile means every weight byte comes from HBM
    # once; with more m tiles the panels are re-read from L2 / MALL.
    w_rate = (cal["tile_hbm_weight_bytes_per_cu_s"] if math.ceil(M / 256) == 1
              else cal["tile_l2_bytes_per_cu_s"])
    per_cu = rounds * (rows * kpart * 2.0 / w_rate
                       + min(M, 256) * kpart * 2.0 / cal["tile_l2_bytes_per_cu_s"])
    reduce = 0.0
    if S > 1:  # split_reduce_kernel: reads the partial planes, writes Y
        part = S * nmat * M * math.ceil(N / 128) * 128 * 4.0
        reduce = (part + 2.0 * M * N) / cal["stream_bytes_per_s"]
        if rounds == 1:  # every workgroup writes its partials at once, after its loads
            per_cu += part / cal["stream_bytes_per_s"]
        nbytes = 2.0 * nmat * K * N + 2.0 * M * K + part
    else:
        nbytes = 2.0 * nmat * K * N + 2.0 * M * K + 2.0 * M * N
    return compute, nbytes / cal["stream_bytes_per_s"], per_cu, reduce


def predict(op: str, M: int, N: int, K: int, machine_path: str = str(MACHINE)) -> dict:
    m = machine(machine_path)
    # YAML 1.1 reads 1.0e12 as a string: convert explicitly
    cal = {k: float(v) for k, v in m["calibration"].items() if k != "measured_us"}
    cus = m["compute"]["owners"]["worker"]["count"]
    plan = describe_launch(op, M, N, K)
    nmat = 2 if op == "fused_swiglu" else 1
    S = plan["splits"]
    gap = (plan["launches"] - 1) * cal["launch_gap_s"]
    if plan["kernel"] == "tile":
        head_nb = plan["head_blocks_n"]
        segs = [(N, S, plan["workgroups"])]
        head_wgs = 0
        if head_nb:
            head_wgs = math.ceil(M / 256) * (head_nb if nmat == 2 else head_nb // 2)
            segs = [(head_nb * 128, 1, head_wgs),
                    (N - head_nb * 128, S, plan["workgroups"] - head_wgs)]
        parts = [_tile_launch(cal, cus, nmat, M, n, K, s, wgs) for n, s, wgs in segs]
        compute, memory, per_cu, reduce = (sum(p[i] for p in parts) for i in range(4))
        t = sum(max(c, mem, pc, cal["launch_min_s"]) + r for c, mem, pc, r in parts) + gap
    elif plan["kernel"] == "wide_tile":
        compute, memory, per_cu, reduce = _tile_launch(cal, cus, nmat, M, N, K, S,
                                                       plan["workgroups"], 2 * plan["tile_columns"])
        t = max(compute, memory, per_cu, cal["launch_min_s"]) + reduce + gap
    elif plan["kernel"] == "decode_tile":
        # Each workgroup streams, per 64-k step of its split, 16 KiB of
        # weights and M rows x 128 bytes of X (rows >= M move nothing);
        # 128 MFMA columns and 64 MT rows per workgroup (MT = 1 for M <= 64,
        # 2 up to 128 rows, 4 up to 256: the mid-M forms).
        groups = plan["workgroups"]
        rows = 64 * (1 if M <= 64 else 2 if M <= 128 else 4)
        kbs = math.ceil(math.ceil(K / 64) / S)
        flops = 2.0 * rows * 128 * kbs * 64 * groups
        compute = math.ceil(groups / cus) * flops / groups / cal["small_m_flops_per_cu"]
        wg_bytes = kbs * (16384.0 + min(M, rows) * 128.0)
        per_cu = math.ceil(groups / cus) * (cal["decode_tile_fill_s"] +
                                            wg_bytes / cal["decode_tile_bytes_per_cu_s"])
        partials = 2.0 * plan["workspace_bytes"] if S > 1 else 0.0
        nbytes = 2.0 * nmat * K * N + 2.0 * M * K + 2.0 * M * N + partials
        memory = nbytes / cal["decode_tile_stream_bytes_per_s"]
        # the split reduce: its own pass after the main kernel
        reduce = cal["decode_tile_reduce_s"] if S > 1 else 0.0
        t = max(compute, memory, per_cu, cal["launch_min_s"]) + reduce + gap
    else:
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
        reduce = 0.0
        t = max(compute, memory, per_cu, cal["launch_min_s"]) + gap
    return {"compute_us": compute * 1e6, "memory_us": memory * 1e6, "per_cu_us": per_cu * 1e6,
            "reduce_us": reduce * 1e6, "predicted_us": t * 1e6,
            "bound": "mfma" if compute >= max(memory, per_cu) else "hbm", "plan": plan}


def calibration_table(machine_path: str = str(MACHINE)) -> list[dict]:
    """Predicted vs the measured times recorded in the machine file."""
    rows = []
    for r in machine(machine_path)["calibration"]["measured_us"]:
        p = predict(r["op"], r["M"], r["N"], r["K"], machine_path)
        rows.append({**r, "predicted_us": round(p["predicted_us"], 2), "bound": p["bound"],
                     "ratio": round(p["predicted_us"] / r["us"], 3)})
    return rows
