"""Benchmark of the fused SwiGLU hot path on one MI355X (BASELINE.json metric).

Headline (value): prefill fused SwiGLU, M=2048, K=4096, N=11008 (BASELINE
config 3), bf16 inputs, fp32 accumulation, bf16 output, in TFLOP/s with
4*M*K*N flops per step.  One step = one llk_swiglu_bf16 call over inputs
already resident in HBM; the average launch time comes from HIP events on
the launch stream.  Reported in "extra": decode SwiGLU (config 4,
M in {1, 8, 16, 64}, K=4096, N=14336) in HBM GB/s with weights rotated over four
copies (940 MB, beyond the 256 MB MALL); the 4096^3 GEMM (config 2); the
MLP block (config 5) over its ragged M sweep; the reference's CPU path (the
AVX2 restatement) on configs 1, 4 and 5 beside the headline's cpu_baseline;
torch.matmul (hipBLASLt) on the same shapes for comparison.

Prints ONE JSON line.  --gpus N with N > 1 exits: this path runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (published)
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E (published)
PROFILE = ROOT / "profiles" / "swiglu_prefill_2048x4096x11008.md"

PREFILL = dict(M=2048, K=4096, N=11008)
DECODE = dict(K=4096, N=14336)
DECODE_M = (1, 8, 16, 64)
MLP = dict(K=5120, N=13824)
MLP_M = (1, 17, 255, 1000, 4097)
# Mid M between config 5's rows (the decode tile kernel's 128-row form), reported apart.
MLP_MID_M = (65, 128)
# Every timed workload first runs its --warmup launches, then keeps launching
# until this much time has passed since the first one: the GPU needs ~35 ms of
# load to reach its steady clock (the first 50 prefill launches average
# 386 us, the steady state ~266 us), so a short --warmup alone would time
# the clock ramp.  The headline's warm-up time and launch count are reported.
PREFILL_WARM_S = 0.25
EXTRA_WARM_S = 0.1


def _time_loop(torch, fn, steps: int, warmup: int, min_warm_s: float = 0.0,
               warm_info: dict | None = None, per_launch: list | None = None) -> float:
    """Average ms per call, HIP events on the launch (current) stream.  After
    `warmup` untimed calls, keeps warming until `min_warm_s` seconds have
    passed (the GPU needs ~35 ms of load to reach its steady clock).
    `warm_info`, if given, receives the untimed launch count and seconds.
    `per_launch`, if given, receives each call's ms: an event is recorded
    between consecutive calls, so call i spans events i and i + 1."""
    t0 = time.perf_counter()
    n = 0
    for i in range(warmup):
        fn(i)
        n += 1
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < min_warm_s:
        for i in range(20):
            fn(n)
            n += 1
        torch.cuda.synchronize()
    if warm_info is not None:
        warm_info.update(launches=n, seconds=round(time.perf_counter() - t0, 3))
    s = torch.cuda.current_stream()
    if per_launch is None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for i in range(steps):
            fn(i)
        e1.record(s)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record(s)
    for i in range(steps):
        fn(i)
        ev[i + 1].record(s)
    torch.cuda.synchronize()
    per_launch.extend(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
    return ev[0].elapsed_time(ev[steps]) / steps


def bench_prefill(torch, llk, steps, warmup, fill="normal"):
    """fill "const" (diagnostic, --only runs): every operand the bf16 0x3C3C
    (~0.0115), so the MFMA datapath sees no bit toggling; the time difference
    to "normal" is the data-dependent power / clock effect."""
    from common import STREAM_WG, STREAM_WU, STREAM_X
    from gpu_util import to_dev
    M, K, N = PREFILL["M"], PREFILL["K"], PREFILL["N"]
    if fill == "const":
        x = np.full((M, K), 0x3C3C, np.uint16)
        wg = np.full((K, N), 0x3C3C, np.uint16)
        wu = wg.copy()
    else:
        x = llk.fill_normal_bf16(42, STREAM_X, (M, K))
        wg = llk.fill_normal_bf16(42, STREAM_WG, (K, N), 1.0 / np.sqrt(K))
        wu = llk.fill_normal_bf16(42, STREAM_WU, (K, N), 1.0 / np.sqrt(K))
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(torch, x)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    warm, per = {}, []
    ms = _time_loop(torch, lambda i: llk.fused_swiglu(xd, pg, pu, out=y), steps, warmup,
                    PREFILL_WARM_S, warm, per)
    flops = 4.0 * M * K * N
    per_us = np.array(per) * 1e3
    launch_us = {"min": round(float(per_us.min()), 2), "median": round(float(np.median(per_us)), 2),
                 "max": round(float(per_us.max()), 2), "launches": len(per)}
    return dict(ms=ms, tflops=flops / (ms * 1e-3) / 1e12, inputs=(x, wg, wu), y=y, warm=warm,
                launch_us=launch_us)


def _rand_w(torch, g, K, N):
    return (torch.randn((K, N), generator=g, device="cuda") / np.sqrt(K)).to(torch.bfloat16)


def bench_decode(torch, llk, M, steps, warmup, copies=4):
    K, N = DECODE["K"], DECODE["N"]
    g = torch.Generator(device="cuda")
    g.manual_seed(42)
    sets = [(llk.PackedWeights.from_device(_rand_w(torch, g, K, N)),
             llk.PackedWeights.from_device(_rand_w(torch, g, K, N))) for _ in range(copies)]
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ms = _time_loop(torch, lambda i: llk.fused_swiglu(x, *sets[i % copies], out=y), steps, warmup,
                    EXTRA_WARM_S)
    nbytes = 2.0 * K * N * 2 + M * K * 2 + M * N * 2
    return dict(ms=ms, gbs=nbytes / (ms * 1e-3) / 1e9)


def bench_gemm(torch, llk, steps, warmup, out_dtype=None):
    """Config 2 (fp32 output); out_dtype bf16 for the comparison with the
    vendor GEMM, whose output is bf16."""
    n = 4096
    g = torch.Generator(device="cuda")
    g.manual_seed(42)
    a = _rand_w(torch, g, n, n)
    pb = llk.PackedWeights.from_device(_rand_w(torch, g, n, n))
    c = torch.empty((n, n), dtype=out_dtype or torch.float32, device="cuda")
    ms = _time_loop(torch, lambda i: llk.matmul(a, pb, out=c), steps, warmup, EXTRA_WARM_S)
    return dict(ms=ms, tflops=2.0 * n ** 3 / (ms * 1e-3) / 1e12)


def bench_mlp(torch, llk, steps, warmup, rows=MLP_M):
    """Config 5: Y = SwiGLU(X; K=5120, N=13824), Z = Y Wd; per M in `rows`:
    us, TFLOP/s (6*M*K*N) and GB/s over the compulsory bytes (weights + X +
    Y twice + Z)."""
    K, N = MLP["K"], MLP["N"]
    g = torch.Generator(device="cuda")
    g.manual_seed(42)
    pg = llk.PackedWeights.from_device(_rand_w(torch, g, K, N))
    pu = llk.PackedWeights.from_device(_rand_w(torch, g, K, N))
    pd = llk.PackedWeights.from_device(_rand_w(torch, g, N, K))
    out = {}
    for M in rows:
        x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
        y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        z = torch.empty((M, K), dtype=torch.bfloat16, device="cuda")
        ms = _time_loop(torch, lambda i: llk.mlp(x, pg, pu, pd, y=y, z=z), max(5, steps // 2),
                        warmup, EXTRA_WARM_S)
        nbytes = 3.0 * K * N * 2 + M * K * 2 * 2 + M * N * 2 * 2
        out[f"M{M}"] = {"us": round(ms * 1e3, 1),
                        "tflops": round(6.0 * M * K * N / (ms * 1e-3) / 1e12, 1),
                        "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    return out


def bench_vendor(torch, steps, warmup):
    """The vendor library on the same box, for comparison: torch.matmul
    (hipBLASLt) on config 3 as one GEMM against [Wg | Wu] (2048 x 4096 x
    22016, the fused kernel's flops) followed by torch's SiLU and product
    (the unfused path), and the 4096^3 GEMM with bf16 output (torch has no
    bf16-input, fp32-output matmul)."""
    import torch.nn.functional as F
    g = torch.Generator(device="cuda")
    g.manual_seed(42)
    M, K, N = PREFILL["M"], PREFILL["K"], PREFILL["N"]
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    w = _rand_w(torch, g, K, 2 * N)
    gu = torch.empty((M, 2 * N), dtype=torch.bfloat16, device="cuda")
    ms_gemm = _time_loop(torch, lambda i: torch.matmul(x, w, out=gu), steps, warmup,
                         EXTRA_WARM_S)
    ms_full = _time_loop(torch, lambda i: _unfused_swiglu(torch, F, x, w, gu, N), steps, warmup,
                         EXTRA_WARM_S)
    n = 4096
    a = _rand_w(torch, g, n, n)
    b = _rand_w(torch, g, n, n)
    c = torch.empty((n, n), dtype=torch.bfloat16, device="cuda")
    ms_sq = _time_loop(torch, lambda i: torch.matmul(a, b, out=c), steps, warmup, EXTRA_WARM_S)
    f3 = 4.0 * M * K * N
    return {"swiglu_2048x4096x11008_unfused": {"us": round(ms_full * 1e3, 1),
                                              "tflops": round(f3 / (ms_full * 1e-3) / 1e12, 1)},
            "gemm_2048x4096x22016_only": {"us": round(ms_gemm * 1e3, 1),
                                          "tflops": round(f3 / (ms_gemm * 1e-3) / 1e12, 1)},
            "gemm_4096_bf16_out": {"us": round(ms_sq * 1e3, 1),
                                   "tflops": round(2.0 * n ** 3 / (ms_sq * 1e-3) / 1e12, 1)}}


def _unfused_swiglu(torch, F, x, w, gu, N):
    torch.matmul(x, w, out=gu)
    return F.silu(gu[:, :N]) * gu[:, N:]


def native_kernel_fn_us(M, K, N):
    """us per synchronous llk_swiglu_kernel_fn call timed from C by
    `llk-bench --kernel-fn` (a child process, row-major device weights, one
    weight set as below, wall clock per call, best of 3 windows): the call
    without the Python ctypes wrapper's per-call work."""
    import subprocess
    exe = ROOT / "dslcompiler_amd" / "bin" / "llk-bench"
    r = subprocess.run([str(exe), f"--M={M}", f"--N={N}", f"--K={K}", "--kernel-fn",
                        "--warmup-ms=100", "--measure-ms=200", "--reps=3"],
                       capture_output=True, text=True, timeout=120)
    m = re.search(r"\(([0-9.]+) ms/iter", r.stdout)
    if r.returncode != 0 or not m:
        return {"error": (r.stderr or r.stdout).strip()[-300:]}
    return round(float(m.group(1)) * 1e3, 1)


def bench_kernel_fn(torch, llk, M, K, N, calls=40, warm_s=0.05):
    """The reference-shaped KernelFn (llk_swiglu_kernel_fn, synchronous, raw
    row-major weights in device memory) on an M x K x N SwiGLU: us per call
    reading the weights at every call (the default: the row-major decode
    tile kernel at M <= 128, the 128-column tile kernel's row-major form
    above, else a per-call pack of Wg and Wu) through the Python wrapper and
    from C (native_kernel_fn_us), and with
    packed weights reused (llk_kernel_fn_assume_immutable_weights); beside
    them the same shape through llk_swiglu_bf16 with packed handles; with the
    per-call pack, the difference of the first two is the two packs (GB/s
    over their bytes read and written).
    Each form is called for warm_s seconds before its `calls` timed calls
    (the GPU's clock ramp)."""
    from dslcompiler_amd import cache as cmod
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    wg, wu = _rand_w(torch, g, K, N), _rand_w(torch, g, K, N)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")

    def per_call(fn):
        t_end = time.perf_counter() + warm_s
        fn()
        while time.perf_counter() < t_end:
            fn()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(calls):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t) / calls * 1e6

    out = {}
    # weights read at every call: straight from the row-major buffers --
    # the decode tile kernel's form up to 128 rows, the 128-column tile
    # kernel's above (K % 64 == 0, N % 8 == 0) -- else packed per call
    plan = llk.describe_launch("fused_swiglu", M, N, K)
    out["fresh_weights_path"] = (
        "row-major decode tile" if plan["kernel"] == "decode_tile" and M <= 128
        else "row-major tile (128-column)" if K % 64 == 0 and N % 8 == 0 else "pack per call")
    out["fresh_weights_us"] = round(per_call(lambda: cmod.swiglu_kernel_fn(x, wg, wu, y, y)), 1)
    out["fresh_weights_native_us"] = native_kernel_fn_us(M, K, N)
    old = cmod.kernel_fn_assume_immutable_weights(True)
    try:
        out["reuse_packed_us"] = round(per_call(lambda: cmod.swiglu_kernel_fn(x, wg, wu, y, y)), 1)
    finally:
        cmod.kernel_fn_assume_immutable_weights(old)
        llk.lib().llk_cache_clear(llk.lib().llk_kernel_fn_cache())
    pg, pu = llk.PackedWeights.from_device(wg), llk.PackedWeights.from_device(wu)
    out["swiglu_bf16_us"] = round(_time_loop(torch, lambda i: llk.fused_swiglu(x, pg, pu, out=y),
                                             calls, 5, warm_s) * 1e3, 1)
    if out["fresh_weights_path"] == "pack per call":
        # the two packs' share of a call, and their rate over 2 x K x N x 2
        # bytes read + the same written
        pack_us = out["fresh_weights_us"] - out["reuse_packed_us"]
        out["packs_us"] = round(pack_us, 1)
        out["packs_gbs"] = round(2 * 2.0 * 2 * K * N / max(pack_us, 1e-3) / 1e3, 1)
    return out


def model_vs_measured(pre: dict, extra: dict) -> dict:
    """L0 model predictions (dslcompiler_amd.perfmodel) next to this run's
    measurements, in microseconds."""
    from dslcompiler_amd import perfmodel
    P = lambda op, M, N, K: perfmodel.predict(op, M, N, K)["predicted_us"]  # noqa: E731
    rows = {"prefill": (P("fused_swiglu", 2048, 11008, 4096), pre["ms"] * 1e3),
            "gemm_4096": (P("matmul", 4096, 4096, 4096), extra["gemm_4096"]["us"])}
    for M in DECODE_M:
        rows[f"decode_m{M}"] = (P("fused_swiglu", M, 14336, 4096), extra[f"decode_m{M}"]["us"])
    for M in (1, 17, 255, 1000, 4097):
        pred = P("fused_swiglu", M, 13824, 5120) + P("matmul", M, 5120, 13824)
        rows[f"mlp_M{M}"] = (pred, extra["mlp_k5120_n13824"][f"M{M}"]["us"])
    return {k: {"predicted_us": round(p, 1), "measured_us": round(m, 1),
                "ratio": round(p / m, 3)} for k, (p, m) in rows.items()}


def cpu_baseline(x, wg, wu, budget_s: float = 12.0, budget1_s: float = 4.0):
    """The oracle's AVX2 restatement of the reference fused kernel on a bounded
    sample of the headline workload: the first `rows` rows of X (full K and
    N), best of up to 5 runs within about `budget_s` seconds on every host
    thread, and the same on one thread (llk-bench's --threads 1) within about
    `budget1_s` seconds, with the host CPU's model string."""
    import oracle
    threads = _cpu_threads()
    K, N = wg.shape

    def best_rate(nthreads, budget):
        t0 = time.perf_counter()
        oracle.swiglu_avx2(x[:32], wg, wu, nthreads)  # warm-up + estimate
        est = time.perf_counter() - t0
        rows = int(min(x.shape[0], max(32, 32 * round(budget / 3 / max(est, 1e-3)))))
        rows -= rows % 32
        best, reps = 0.0, 0
        t_end = time.perf_counter() + budget
        while reps < 1 or (time.perf_counter() < t_end and reps < 5):
            t = time.perf_counter()
            oracle.swiglu_avx2(x[:rows], wg, wu, nthreads)
            best = max(best, 4.0 * rows * K * N / (time.perf_counter() - t) / 1e12)
            reps += 1
        return best, rows, reps

    best, rows, reps = best_rate(threads, budget_s)
    best1, rows1, reps1 = best_rate(1, budget1_s)
    return {"value": round(best, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"fused SwiGLU rows 0..{rows - 1} of M=2048 (K=4096, N=11008), best of "
                      f"{reps} runs; AVX2 BM32/BN64/BK64/VM4/VN8 tiles, ThreadPool-style "
                      f"dynamic tile queue",
            "threads1": {"value": round(best1, 5), "unit": "TFLOP/s", "cores": 1,
                         "sample": f"rows 0..{rows1 - 1}, best of {reps1} runs"},
            "cpu_model": _cpu_model(), "host_threads": os.cpu_count()}


def _cpu_model() -> str:
    """The host CPU's model string (/proc/cpuinfo)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _cpu_threads() -> int:
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return max(1, min(threads, os.cpu_count() or 1))


def cpu_port_configs(llk, budget_s: float = 3.0) -> dict:
    """The AVX2 restatement of the reference's fused SwiGLU path (the only
    executable CPU path the reference has for these ops) on the other
    BASELINE SwiGLU configs, full shapes, best of up to 3 runs within about
    `budget_s` seconds each: config 1 in GFLOP/s, decode config 4 (M = 8) in
    GB/s over the same algorithmic bytes as the GPU figure, and config 5's
    SwiGLU half at M = 255 in GFLOP/s.  Config 2 (plain GEMM) has no CPU
    figure: `micro.mma` is verifier-only and `llk.matmul` has no lowering
    in the reference (LLKToLinalg.cpp:621-646), so nothing executes it."""
    from common import STREAM_WG, STREAM_WU, STREAM_X
    threads = _cpu_threads()

    def best_s(M, K, N):
        x = llk.fill_normal_bf16(42, STREAM_X, (M, K))
        wg = llk.fill_normal_bf16(42, STREAM_WG, (K, N), 1.0 / np.sqrt(K))
        wu = llk.fill_normal_bf16(42, STREAM_WU, (K, N), 1.0 / np.sqrt(K))
        import oracle
        best, t_end, reps = float("inf"), time.perf_counter() + budget_s, 0
        while reps < 1 or (time.perf_counter() < t_end and reps < 3):
            t = time.perf_counter()
            oracle.swiglu_avx2(x, wg, wu, threads)
            best = min(best, time.perf_counter() - t)
            reps += 1
        return best

    out = {"threads": threads, "kind": "port"}
    s = best_s(64, 512, 1376)
    out["c1_swiglu_64x512x1376"] = {"us": round(s * 1e6, 1),
                                    "gflops": round(4.0 * 64 * 512 * 1376 / s / 1e9, 1)}
    K, N = DECODE["K"], DECODE["N"]
    s = best_s(8, K, N)
    nbytes = 2.0 * K * N * 2 + 8 * K * 2 + 8 * N * 2
    out["c4_decode_m8"] = {"us": round(s * 1e6, 1), "gbs": round(nbytes / s / 1e9, 1)}
    K, N = MLP["K"], MLP["N"]
    s = best_s(255, K, N)
    out["c5_swiglu_m255"] = {"us": round(s * 1e6, 1),
                             "gflops": round(4.0 * 255 * K * N / s / 1e9, 1)}
    out["c2_gemm"] = None
    return out


def spot_parity(x, wg, wu, y_dev):
    """Oracle check of a few rows of the benchmarked output."""
    import oracle
    from common import bf16_bits_to_f32, parity
    from gpu_util import from_dev
    rows = [0, 1, 1023, 2047]
    _, yb_ref = oracle.swiglu_rows(x, wg, wu, rows)
    got = from_dev(y_dev)[rows]
    return parity(bf16_bits_to_f32(got), bf16_bits_to_f32(yb_ref))


def profiled_traffic():
    """HBM bytes per launch of the prefill kernel from the committed rocprofv3
    summary (FETCH_SIZE and WRITE_SIZE, scaled by the copy-kernel factors)."""
    if not PROFILE.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", PROFILE.read_text())
    return float(m.group(1)) if m else None


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=200,
                    help="untimed launches first (200 prefill launches = ~70 ms, past the "
                         "~35 ms the GPU takes to reach its steady clock under load)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--only", choices=["prefill", "decode8", "decode64", "gemm", "mlp", "vendor",
                                       "copy"],
                    help="run one workload for --steps launches and print its timing only "
                         "(for profiler runs); 'copy' is a 256 MiB device copy used to "
                         "calibrate byte counters")
    ap.add_argument("--fill", choices=["normal", "const"], default="normal",
                    help="operands of --only prefill: N(0,1) data (default) or one constant "
                         "value (diagnostic: MFMA power depends on operand bit toggling)")
    ap.add_argument("--mlp-m", help="comma-separated M values of --only mlp (default: all of "
                                    "config 5's)")
    ap.add_argument("--set", action="append", default=[], metavar="NAME=VALUE",
                    help="set a dispatcher knob (llk_set_tunable) before a --only run, e.g. "
                         "tile_splits=2; repeatable")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this hot path runs on one GPU; multi-GPU runs are not part of this "
              "build (SwiGLU would shard column-parallel over N with no communication)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import dslcompiler_amd as llk
    torch.cuda.set_device(0)

    if a.only:
        for kv in a.set:
            name, value = kv.split("=", 1)
            llk.set_tunable(name, int(value))
        if a.only == "prefill":
            pre = bench_prefill(torch, llk, a.steps, a.warmup, a.fill)
            r = {"ms": pre["ms"], "tflops": pre["tflops"], "fill": a.fill}
        elif a.only in ("decode8", "decode64"):
            r = bench_decode(torch, llk, int(a.only[6:]), a.steps, a.warmup)
        elif a.only == "gemm":
            r = bench_gemm(torch, llk, a.steps, a.warmup)
        elif a.only == "mlp":
            r = bench_mlp(torch, llk, a.steps, a.warmup,
                          tuple(int(v) for v in a.mlp_m.split(",")) if a.mlp_m else MLP_M)
        elif a.only == "vendor":
            g16 = bench_gemm(torch, llk, a.steps, a.warmup, torch.bfloat16)
            r = {"vendor_hipblaslt": bench_vendor(torch, a.steps, a.warmup),
                 "llk_gemm_4096_bf16_out": {"us": round(g16["ms"] * 1e3, 1),
                                            "tflops": round(g16["tflops"], 1)}}
        else:
            src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
            dst = torch.empty_like(src)
            r = {"ms": _time_loop(torch, lambda i: dst.copy_(src), a.steps, a.warmup)}
        print(json.dumps({"only": a.only, **({"set": a.set} if a.set else {}), **r}), flush=True)
        return

    pre = bench_prefill(torch, llk, a.steps, a.warmup)
    x, wg, wu = pre["inputs"]
    par = spot_parity(x, wg, wu, pre["y"])
    extra = {"prefill_parity_rows": {k: round(v, 6) for k, v in par.items()}}
    if not a.no_extra:
        for M in DECODE_M:
            d = bench_decode(torch, llk, M, a.steps, a.warmup)
            extra[f"decode_m{M}"] = {"us": round(d["ms"] * 1e3, 2), "gbs": round(d["gbs"], 1),
                                     "hbm_frac": round(d["gbs"] / PEAK_HBM_GBS, 4)}
        gem = bench_gemm(torch, llk, max(10, a.steps // 2), a.warmup)
        extra["gemm_4096"] = {"us": round(gem["ms"] * 1e3, 1), "tflops": round(gem["tflops"], 1),
                              "mfma_frac": round(gem["tflops"] / PEAK_BF16_TFLOPS, 4)}
        extra["mlp_k5120_n13824"] = bench_mlp(torch, llk, a.steps, a.warmup)
        extra["mlp_k5120_n13824_mid_m"] = bench_mlp(torch, llk, a.steps, a.warmup, MLP_MID_M)
        extra["vendor_hipblaslt"] = bench_vendor(torch, max(10, a.steps // 2), a.warmup)
        g16 = bench_gemm(torch, llk, max(10, a.steps // 2), a.warmup, torch.bfloat16)
        extra["gemm_4096_bf16_out"] = {"us": round(g16["ms"] * 1e3, 1),
                                       "tflops": round(g16["tflops"], 1)}
        extra["model_vs_measured"] = model_vs_measured(pre, extra)
        extra["kernel_fn_c3"] = bench_kernel_fn(torch, llk, PREFILL["M"], PREFILL["K"],
                                                PREFILL["N"])
        extra["kernel_fn_decode_m8"] = bench_kernel_fn(torch, llk, 8, DECODE["K"], DECODE["N"])
    cpu = None if a.no_cpu_baseline else cpu_baseline(x, wg, wu)
    if not a.no_cpu_baseline and not a.no_extra:
        extra["cpu_port_other_configs"] = cpu_port_configs(llk)

    achieved = pre["tflops"]
    line = {
        "metric": "Fused SwiGLU TFLOP/s & % MFMA peak (M=2048,K=4096,N=11008); decode HBM GB/s",
        "value": round(achieved, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "warm_untimed": {**pre["warm"], "rule": f"--warmup launches, then more until "
                                                f"{PREFILL_WARM_S} s have passed"},
        "ms_per_step": round(pre["ms"], 5),
        "launch_us": pre["launch_us"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (splitmix64/Box-Muller seed 42; X~N(0,1), W~N(0,1/sqrt(K)))",
        "config": {"workload": "prefill fused SwiGLU M=2048 K=4096 N=11008, bf16 out "
                               "(BASELINE config 3)",
                   "M": 2048, "K": 4096, "N": 11008, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": profiled_traffic()},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
