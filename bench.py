"""Benchmark of the fused SwiGLU hot path on one MI355X (BASELINE.json metric).

Headline workload (value): prefill fused SwiGLU, M=2048, K=4096, N=11008,
bf16 inputs, fp32 accumulation, bf16 output -> TFLOP/s (4*M*K*N per step).
One step = one llk_swiglu_bf16 call over the resident inputs.  Also reported
("extra"): the decode shape M=8, K=4096, N=14336 in HBM GB/s with rotated
weight copies (so the 256 MB MALL cannot hold them), and the 4096^3 GEMM.

Prints ONE JSON line.  --gpus N with N > 1 exits: this path runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E

PREFILL = dict(M=2048, K=4096, N=11008)
DECODE = dict(M=8, K=4096, N=14336)
GEMM = dict(M=4096, K=4096, N=4096)


def _time_loop(torch, fn, steps: int, warmup: int) -> float:
    """Average ms per call measured with HIP events on the launch stream."""
    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for i in range(steps):
        fn(i)
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def bench_prefill(torch, llk, steps, warmup):
    from common import STREAM_WG, STREAM_WU, STREAM_X
    from gpu_util import to_dev
    M, K, N = PREFILL["M"], PREFILL["K"], PREFILL["N"]
    x = llk.fill_normal_bf16(42, STREAM_X, (M, K))
    wg = llk.fill_normal_bf16(42, STREAM_WG, (K, N), 1.0 / np.sqrt(K))
    wu = llk.fill_normal_bf16(42, STREAM_WU, (K, N), 1.0 / np.sqrt(K))
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(torch, x)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ms = _time_loop(torch, lambda i: llk.fused_swiglu(xd, pg, pu, out=y), steps, warmup)
    flops = 4.0 * M * K * N
    return dict(ms=ms, tflops=flops / (ms * 1e-3) / 1e12, flops=flops,
                inputs=(x, wg, wu), y=y, packed=(pg, pu))


def bench_decode(torch, llk, steps, warmup, copies=4):
    M, K, N = DECODE["M"], DECODE["K"], DECODE["N"]
    g = torch.Generator(device="cuda")
    g.manual_seed(42)
    sets = []
    for c in range(copies):  # distinct weights, 235 MB per set: > MALL
        wg = (torch.randn((K, N), generator=g, device="cuda") / np.sqrt(K)).to(torch.bfloat16)
        wu = (torch.randn((K, N), generator=g, device="cuda") / np.sqrt(K)).to(torch.bfloat16)
        sets.append((llk.PackedWeights.from_device(wg), llk.PackedWeights.from_device(wu)))
        del wg, wu
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ms = _time_loop(torch, lambda i: llk.fused_swiglu(x, *sets[i % copies], out=y), steps,
                    warmup)
    nbytes = 2.0 * K * N * 2 + M * K * 2 + M * N * 2
    return dict(ms=ms, gbs=nbytes / (ms * 1e-3) / 1e9, bytes=nbytes)


def bench_gemm(torch, llk, steps, warmup):
    M, K, N = GEMM["M"], GEMM["K"], GEMM["N"]
    g = torch.Generator(device="cuda")
    g.manual_seed(42)
    a = (torch.randn((M, K), generator=g, device="cuda") / np.sqrt(K)).to(torch.bfloat16)
    b = (torch.randn((K, N), generator=g, device="cuda") / np.sqrt(K)).to(torch.bfloat16)
    pb = llk.PackedWeights.from_device(b)
    c = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ms = _time_loop(torch, lambda i: llk.matmul(a, pb, out=c), steps, warmup)
    return dict(ms=ms, tflops=2.0 * M * N * K / (ms * 1e-3) / 1e12)


def cpu_baseline(x, wg, wu, budget_s: float = 12.0):
    """The oracle's AVX2 restatement of the reference fused kernel on a bounded
    sample of the headline workload: the first `rows` rows of X (full K, N),
    repeated for about `budget_s` seconds; best rate reported."""
    import oracle
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    threads = max(1, min(threads, os.cpu_count() or 1))
    K, N = wg.shape
    rows = 32  # one BM tile row
    t0 = time.perf_counter()
    oracle.swiglu_avx2(x[:rows], wg, wu, threads)  # warm-up + estimate
    est = time.perf_counter() - t0
    rows = int(min(x.shape[0], max(32, 32 * round(budget_s / 3 / max(est, 1e-3)))))
    rows -= rows % 32
    best = 0.0
    t_end = time.perf_counter() + budget_s
    reps = 0
    while reps < 1 or (time.perf_counter() < t_end and reps < 5):
        t = time.perf_counter()
        oracle.swiglu_avx2(x[:rows], wg, wu, threads)
        dt = time.perf_counter() - t
        best = max(best, 4.0 * rows * K * N / dt / 1e12)
        reps += 1
    return {"value": round(best, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"fused SwiGLU rows 0..{rows - 1} of M=2048 (K=4096, N=11008), "
                      f"best of {reps} runs, AVX2 BM32/BN64/BK64/VM4/VN8 tiles"}


def spot_parity(x, wg, wu, y_dev):
    """Oracle check of a few rows of the benchmarked output."""
    import oracle
    from common import bf16_bits_to_f32, parity
    from gpu_util import from_dev
    rows = [0, 1, 1023, 2047]
    _, yb_ref = oracle.swiglu_rows(x, wg, wu, rows)
    got = from_dev(y_dev)[rows]
    return parity(bf16_bits_to_f32(got), bf16_bits_to_f32(yb_ref))


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this hot path runs on one GPU; multi-GPU runs are not part of this "
              "build (the sharding plan is in DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import torch
    import dslcompiler_amd as llk
    torch.cuda.set_device(0)

    pre = bench_prefill(torch, llk, a.steps, a.warmup)
    x, wg, wu = pre["inputs"]
    par = spot_parity(x, wg, wu, pre["y"])
    extra = {"prefill_parity_rows": {k: round(v, 6) for k, v in par.items()}}
    if not a.no_extra:
        dec = bench_decode(torch, llk, a.steps, a.warmup)
        gem = bench_gemm(torch, llk, max(10, a.steps // 2), a.warmup)
        extra.update({
            "decode_m8_gbs": round(dec["gbs"], 1),
            "decode_m8_us": round(dec["ms"] * 1e3, 2),
            "decode_m8_hbm_frac": round(dec["gbs"] / PEAK_HBM_GBS, 4),
            "gemm_4096_tflops": round(gem["tflops"], 1),
            "gemm_4096_mfma_frac": round(gem["tflops"] / PEAK_BF16_TFLOPS, 4),
        })
    cpu = None if a.no_cpu_baseline else cpu_baseline(x, wg, wu)

    achieved = pre["tflops"]
    line = {
        "metric": "Fused SwiGLU TFLOP/s & % MFMA peak (M=2048,K=4096,N=11008); decode HBM GB/s",
        "value": round(achieved, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(pre["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (splitmix64/Box-Muller seed 42; X~N(0,1), W~N(0,1/sqrt(K)))",
        "config": {"workload": "prefill fused SwiGLU M=2048 K=4096 N=11008, bf16 out",
                   "M": 2048, "K": 4096, "N": 11008, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": None},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
