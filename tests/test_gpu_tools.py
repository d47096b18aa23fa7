"""GPU runs of the C++ tools (llk-bench, llk-tune) and parity of launches
chosen by a loaded schedule DB."""
from __future__ import annotations

import json
import re
import subprocess
from pathlib import Path

import pytest

import dslcompiler_amd as llk
from common import assert_parity, swiglu_inputs
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu

BIN = Path(llk.__file__).resolve().parent / "bin"


def test_llk_bench_runs(gpu):
    print("case llk-bench", flush=True)
    r = subprocess.run([str(BIN / "llk-bench"), "--M=8", "--N=1408", "--K=1024",
                        "--warmup-ms=20", "--measure-ms=20", "--reps=2", "--copies=2"],
                       capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stderr
    m = re.search(r"Best: ([0-9.]+) GFLOPS \(([0-9.]+) ms/iter, 2 reps\)", r.stdout)
    assert m and float(m.group(1)) > 0 and float(m.group(2)) > 0, r.stdout


def test_llk_bench_kernel_fn_runs(gpu):
    """llk-bench --kernel-fn: synchronous llk_swiglu_kernel_fn calls on
    row-major device weights, timed by wall clock."""
    print("case llk-bench --kernel-fn", flush=True)
    r = subprocess.run([str(BIN / "llk-bench"), "--M=8", "--N=1408", "--K=1024", "--kernel-fn",
                        "--warmup-ms=20", "--measure-ms=20", "--reps=2", "--copies=2"],
                       capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stderr
    m = re.search(r"Best: ([0-9.]+) GFLOPS \(([0-9.]+) ms/iter, 2 reps\)", r.stdout)
    assert m and float(m.group(1)) > 0 and float(m.group(2)) > 0, r.stdout
    assert "llk_swiglu_kernel_fn: synchronous calls, wall clock per call" in r.stdout


def test_llk_tune_measures_and_writes_db(gpu, tmp_path):
    print("case llk-tune", flush=True)
    out = tmp_path / "tune.json"
    r = subprocess.run([str(BIN / "llk-tune"), "--op=matmul", "--M=300", "--N=640", "--K=2048",
                        "--measure-ms=5", "--top=3", f"-o={out}"],
                       capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stderr
    entries = json.loads(out.read_text())["entries"]
    assert len(entries) == 3
    us = [e["measured_us"] for e in entries]
    assert all(u > 0 for u in us) and us == sorted(us)
    assert all(e["operation"] == "matmul" and e["shape"]["M_bucket"] == 4 for e in entries)


def test_schedule_db_launches_keep_parity(gpu, orc, tmp_path):
    """Launch shapes picked from a schedule DB (group width 4 with 3 splits
    for small M, 5 tile splits) still meet the bar."""
    print("case schedule-db parity", flush=True)
    sched = {"BM": 32, "BN": 128, "BK": 64, "VM": 32, "VN": 32, "vector_width": 8,
             "num_threads": 1024, "parallel_axis": "n", "grain_size": 3}
    tile = dict(sched, BM=256, BN=128, BK=32, num_threads=256, parallel_axis="mn", grain_size=5)
    db = tmp_path / "db.json"
    db.write_text(json.dumps({"version": 1, "entries": [
        {"operation": "fused_swiglu", "target": "gfx950", "shape": {"M_bucket": 2, "N": 0, "K": 0},
         "dtype": "bf16", "math_mode": "strict", "schedule": sched},
        {"operation": "fused_swiglu", "target": "gfx950", "shape": {"M_bucket": 4, "N": 0, "K": 0},
         "dtype": "bf16", "math_mode": "strict", "schedule": tile}]}))
    llk.set_schedule_db(db)
    try:
        for M in (8, 300):
            x, wg, wu = swiglu_inputs(M, 1536, 700, seed=M)
            plan = llk.describe_launch("fused_swiglu", M, 700, 1536)
            assert plan["splits"] == (3 if M == 8 else 5)
            pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
            y = from_dev(llk.fused_swiglu(to_dev(gpu, x), pg, pu, out_dtype=gpu.float32))
            yf_ref, _ = orc.swiglu(x, wg, wu)
            assert_parity(y, yf_ref, f"schedule-db M={M}")
    finally:
        llk.set_schedule_db(None)
