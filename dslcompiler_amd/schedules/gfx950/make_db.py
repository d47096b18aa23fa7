"""Regenerates schedule_db.json (this directory) from measurements: runs
llk-tune (GPU required) on every BASELINE shape, then for each (operation,
M bucket) keeps the launch setting with the lowest total time relative to
each shape's best, so the loader's first-match rule picks one setting that
serves all shapes of the bucket.

    python -m dslcompiler_amd.schedules.gfx950.make_db [--measure-ms 100] [--out PATH]
"""
from __future__ import annotations

import argparse
import json
import subprocess
import tempfile
from collections import defaultdict
from pathlib import Path

HERE = Path(__file__).resolve().parent
TUNE = HERE.parents[1] / "bin" / "llk-tune"

# (op, M, N, K): BASELINE configs 1-5 (config 5 = SwiGLU + down projection).
SHAPES = [("fused_swiglu", 64, 1376, 512), ("matmul", 4096, 4096, 4096),
          ("fused_swiglu", 2048, 11008, 4096)]
SHAPES += [("fused_swiglu", m, 14336, 4096) for m in (1, 8, 16)]
SHAPES += [("fused_swiglu", m, 13824, 5120) for m in (1, 17, 255, 1000, 4097)]
SHAPES += [("matmul", m, 5120, 13824) for m in (1, 17, 255, 1000, 4097)]
# decode batch sizes so that every M bucket has an entry (buckets 1 and 2 of
# the down projection, bucket 1 of SwiGLU)
SHAPES += [("fused_swiglu", 4, 14336, 4096), ("matmul", 4, 5120, 13824),
           ("matmul", 8, 5120, 13824), ("matmul", 16, 5120, 13824)]
# batch-64 decode: bucket 3 also spans two 32-row groups
SHAPES += [("fused_swiglu", 64, 14336, 4096), ("matmul", 64, 5120, 13824)]


def tune(op: str, M: int, N: int, K: int, measure_ms: int) -> list[dict]:
    with tempfile.TemporaryDirectory() as d:
        out = Path(d) / "t.json"
        subprocess.run([str(TUNE), f"--op={op}", f"--M={M}", f"--N={N}", f"--K={K}",
                        f"--measure-ms={measure_ms}", "--top=100", f"-o={out}"],
                       check=True, stdout=subprocess.DEVNULL, timeout=600)
        return json.loads(out.read_text())["entries"]


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--measure-ms", type=int, default=100)
    ap.add_argument("--out", default=str(HERE / "schedule_db.json"))
    a = ap.parse_args()
    # (op, bucket) -> setting -> [time / best time of each shape]
    scores: dict = defaultdict(lambda: defaultdict(list))
    measured = []
    schedules = {}
    for op, M, N, K in SHAPES:
        entries = tune(op, M, N, K, a.measure_ms)
        best = entries[0]["measured_us"]
        bucket = entries[0]["shape"]["M_bucket"]
        for e in entries:
            s = dict(e["schedule"])
            # a setting is (column groups, splits) for M <= 64 (BN 0: the
            # decode tile kernel; 32 G: the small-M kernel of width G) and
            # the splits for the tile kernels, whose width the dispatcher
            # picks per shape (BN 0 in the merged record); BM and the thread
            # count follow from the shape
            if s["BM"] == 256:
                s["BN"] = 0
            key = (s["BN"], s["grain_size"])
            scores[(op, bucket)][key].append(e["measured_us"] / best)
            schedules[(op, bucket, key)] = s
        measured.append(f"{op} M={M} N={N} K={K}: best {best:.2f} us")
        print(measured[-1], flush=True)
    out = []
    for (op, bucket), settings in sorted(scores.items()):
        n_shapes = max(len(v) for v in settings.values())
        full = {k: sum(v) for k, v in settings.items() if len(v) == n_shapes}
        key = min(full, key=full.get)
        out.append({"operation": op, "target": "gfx950",
                    "shape": {"M_bucket": bucket, "N": 0, "K": 0}, "dtype": "bf16",
                    "math_mode": "strict", "schedule": schedules[(op, bucket, key)],
                    "source": "make_db.py",
                    "relative_time": round(full[key] / n_shapes, 4)})
    doc = {
        "version": 1,
        "comment": (
            "gfx950 (MI355X) schedules in the schedule_db.json record schema, measured with "
            "llk-tune over the BASELINE shapes by make_db.py (one entry per operation and M "
            "bucket; relative_time = mean of time / best time over the bucket's shapes). Field "
            "meaning on this target: BM/BN = workgroup tile rows / columns per weight matrix "
            "(small-M kernel: BN / 32 = column groups per workgroup; BN 0: the decode tile "
            "kernel for M <= 64, the width the dispatcher picks per shape for the tile kernels); "
            "BK = k per step; VM/VN = MFMA tile (small-M and decode tile kernels "
            "v_mfma_f32_32x32x16_bf16, tile kernels v_mfma_f32_16x16x32_bf16); "
            "vector_width = bf16 per lane operand; "
            "num_threads = threads per workgroup; parallel_axis = grid decomposition; "
            "grain_size = k splits across workgroups (0 = chosen from the shape)."),
        "measured": measured,
        "entries": out,
    }
    Path(a.out).write_text(json.dumps(doc, indent=1) + "\n")
    print(f"wrote {len(out)} entries to {a.out}")


if __name__ == "__main__":
    main()
