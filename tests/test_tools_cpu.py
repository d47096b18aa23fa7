"""Host-side tools and dispatch on the CPU: llk-compile over MLIR text in the
reference's syntax (shape_specialization.mlir:1-46 buckets, ops_invalid.mlir
verifier messages), llk-tune's candidate generation and schedule-DB output,
the exported verifiers, and schedule-DB-driven launch plans."""
from __future__ import annotations

import json
import subprocess
from pathlib import Path

import pytest

import dslcompiler_amd as llk

BIN = Path(llk.__file__).resolve().parent / "bin"


def _swiglu_fn(name, M, K, N, outM=None, Kg=None, mode="bounded_fast"):
    outM = M if outM is None else outM
    Kg = K if Kg is None else Kg
    return f"""
func.func @{name}(%x: tensor<{M}x{K}xbf16>, %wg: tensor<{Kg}x{N}xbf16>, %wu: tensor<{K}x{N}xbf16>, %init: tensor<{outM}x{N}xbf16>) -> tensor<{outM}x{N}xbf16> {{
  %y = llk.fused_swiglu ins(%x, %wg, %wu : tensor<{M}x{K}xbf16>, tensor<{Kg}x{N}xbf16>, tensor<{K}x{N}xbf16>)
      outs(%init : tensor<{outM}x{N}xbf16>)
      {{accumulator_type = f32, activation = #llk.activation<silu>, math_mode = #llk.math_mode<{mode}>}}
      -> tensor<{outM}x{N}xbf16>
  return %y : tensor<{outM}x{N}xbf16>
}}
"""


def _compile(tmp_path, text, *args):
    f = tmp_path / "in.mlir"
    f.write_text(text)
    return subprocess.run([str(BIN / "llk-compile"), str(f), *args], capture_output=True,
                          text=True, timeout=60)


@pytest.fixture(scope="module", autouse=True)
def _tools_built():
    for t in ("llk-compile", "llk-tune", "llk-bench"):
        assert (BIN / t).exists(), f"{t} not built (run __graft_entry__.build())"


def test_compile_buckets_follow_shape_specialization(tmp_path):
    """shape_specialization.mlir: M = 1, 4, 16, 64, 128 -> buckets 0..4."""
    text = "".join(_swiglu_fn(f"bucket_M{m}", m, 256, 512) for m in (1, 4, 16, 64, 128))
    r = _compile(tmp_path, text)
    assert r.returncode == 0, r.stderr
    for m, b in zip((1, 4, 16, 64, 128), range(5)):
        assert f"@bucket_M{m}: llk.fused_swiglu M={m} N=512 K=256 -> bucket {b}" in r.stdout
    assert r.stdout.rstrip().endswith("Compilation successful")
    # every M here (at most 256) runs on the decode tile kernel: M = 128
    # on its 128-row form
    assert r.stdout.count("kernel=decode_tile") == 5, r.stdout


@pytest.mark.parametrize("kw,msg", [
    (dict(M=2, K=4, N=8, outM=3), "M dimension mismatch: X=2 vs init=3"),
    (dict(M=2, K=4, N=8, Kg=5), "K dimension mismatch between X=4 and Wg=5"),
])
def test_compile_verifier_errors(tmp_path, kw, msg):
    """ops_invalid.mlir cases: the reference verifier's messages, exit 1."""
    r = _compile(tmp_path, _swiglu_fn("bad", **kw))
    assert r.returncode == 1
    assert msg in r.stderr
    assert "Compilation successful" not in r.stdout


def test_compile_dynamic_dims_and_matmul(tmp_path):
    text = _swiglu_fn("dyn", "?", 4096, 14336) + """
func.func @mm(%a: tensor<32x64xbf16>, %b: tensor<64x32xbf16>, %c: tensor<32x32xf32>) -> tensor<32x32xf32> {
  %0 = llk.matmul ins(%a, %b : tensor<32x64xbf16>, tensor<64x32xbf16>)
      outs(%c : tensor<32x32xf32>) -> tensor<32x32xf32>
  return %0 : tensor<32x32xf32>
}
"""
    r = _compile(tmp_path, text)
    assert r.returncode == 1 and "dynamic dimension" in r.stderr
    r = _compile(tmp_path, text, "--M=8")
    assert r.returncode == 0, r.stderr
    assert "@dyn: llk.fused_swiglu M=8 N=14336 K=4096 -> bucket 2" in r.stdout
    assert "@mm: llk.matmul M=32 N=32 K=64 -> bucket 3" in r.stdout
    r = _compile(tmp_path, text.replace("tensor<64x32xbf16>", "tensor<32x32xbf16>"), "--M", "8")
    assert r.returncode == 1 and "K dimension must match: 64 vs 32" in r.stderr


def test_compile_missing_input(tmp_path):
    r = subprocess.run([str(BIN / "llk-compile"), str(tmp_path / "none.mlir")],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "Failed to parse" in r.stderr


def _tool(name, *args):
    return subprocess.run([str(BIN / name), *args], capture_output=True, text=True, timeout=60)


@pytest.mark.parametrize("args", [
    ["--M", "2048", "--N", "11008", "--K", "4096"],   # --name value
    ["-M=2048", "-N=11008", "-K=4096"],               # -name=value
    ["-M", "2048", "--N=11008", "-K", "4096"],        # mixed
])
def test_bench_options_in_llvm_cl_forms(args):
    """llk-bench takes the reference's llvm::cl options (llk-bench.cpp:21-35)
    in every form cl accepts; --dry-run reports the parsed shape and plan
    without a GPU.  --threads (the reference's CPU thread count) is
    accepted."""
    r = _tool("llk-bench", *args, "--threads", "16", "--dry-run")
    assert r.returncode == 0, r.stderr
    assert "M=2048 N=11008 K=4096 threads=16" in r.stdout
    assert "kernel=swiglu_wide splits=1" in r.stdout and "workgroups=504" in r.stdout


def test_bench_kernel_fn_option():
    """llk-bench --kernel-fn (timing llk_swiglu_kernel_fn by wall clock per
    call, as the reference's harness times its function) parses with the
    other options; the dry run names it."""
    r = _tool("llk-bench", "-M", "8", "-N", "14336", "-K", "4096", "--kernel-fn", "--dry-run")
    assert r.returncode == 0, r.stderr
    assert "M=8 N=14336 K=4096" in r.stdout and r.stdout.split("\n")[0].endswith("kernel-fn")
    assert "kernel=decode_tile" in r.stdout


@pytest.mark.parametrize("tool,args,msg", [
    ("llk-bench", ["--bogus"], "Unknown command line argument '--bogus'"),
    ("llk-bench", ["--threads=2", "-x"], "Unknown command line argument '-x'"),
    ("llk-bench", ["-M"], "for the -M option: requires a value!"),
    ("llk-bench", ["-M", "12x"], "'12x' value invalid for integer argument"),
    ("llk-bench", ["--kernel-fn", "--op=matmul"], "--kernel-fn: llk_swiglu_kernel_fn computes"),
    ("llk-bench", ["--kernel-fn", "--out=f32"], "--kernel-fn: llk_swiglu_kernel_fn computes"),
    ("llk-tune", ["--dry-run=maybe"], "invalid value for boolean argument"),
    ("llk-tune", ["--threads=8", "--dry-run"], "Unknown command line argument '--threads=8'"),
    ("llk-compile", [], "Not enough positional command line arguments"),
    ("llk-compile", ["a.mlir", "b.mlir"], "Too many positional arguments"),
])
def test_tools_reject_bad_options(tool, args, msg):
    """Unknown options and malformed values exit 1 with cl's message instead
    of silently running the defaults."""
    r = _tool(tool, *args)
    assert r.returncode == 1, r.stdout
    assert msg in r.stderr


def test_tune_output_option_forms(tmp_path):
    """llk-tune -o <file> (llk-tune.cpp:27-28) writes that file in every
    form; the default stays tune_result.json in the working directory."""
    for i, form in enumerate((["-o", "a.json"], ["-o=b.json"], ["--o", "c.json"])):
        r = subprocess.run([str(BIN / "llk-tune"), "-M", "2048", "--N=11008", "-K", "4096",
                            "--dry-run", *form], capture_output=True, text=True, timeout=60,
                           cwd=tmp_path)
        assert r.returncode == 0, r.stderr
        name = "abc"[i] + ".json"
        assert (tmp_path / name).exists() and f"to {name}" in r.stdout
        assert "M=2048 (bucket 4) N=11008 K=4096" in r.stdout
    r = subprocess.run([str(BIN / "llk-tune"), "--dry-run"], capture_output=True, text=True,
                       timeout=60, cwd=tmp_path)
    assert r.returncode == 0 and (tmp_path / "tune_result.json").exists()
    assert "M=128 (bucket 4) N=4096 K=4096" in r.stdout  # the reference's defaults


def test_compile_string_keyed_entry(tmp_path):
    """llk-compile derives the reference's cache key, "llk_" + hash of the
    module + "_M.._N.._K.." (llk-compile.cpp:298-310), and obtains the
    module's KernelFn through the string-keyed lookupOrCompile."""
    r = _compile(tmp_path, _swiglu_fn("f", 8, 4096, 14336), "-M", "8", "-N=14336", "--K", "4096")
    assert r.returncode == 0, r.stderr
    line = [l for l in r.stdout.splitlines() if l.startswith("entry: llk_")]
    assert len(line) == 1 and line[0].endswith("_M8_N14336_K4096"), r.stdout


def test_verifiers_exported():
    L = llk.lib()
    assert L.llk_verify_fused_swiglu(2, 4, 4, 8, 4, 8, 2, 8) == 0
    assert L.llk_verify_fused_swiglu(-1, 4, 4, 8, 4, 8, 3, 8) == 0  # dynamic M skips
    assert L.llk_verify_fused_swiglu(2, 4, 4, 8, 4, 9, 2, 8) == -2
    assert b"N dimension mismatch between Wg=8 and Wu=9" in L.llk_last_error()
    assert L.llk_verify_matmul(64, 64) == 0 and L.llk_verify_matmul(-1, 3) == 0
    assert L.llk_verify_matmul(64, 32) == -2


def test_tune_dry_run_writes_loadable_db(tmp_path):
    out = tmp_path / "tune.json"
    r = subprocess.run([str(BIN / "llk-tune"), "--op=fused_swiglu", "--M=8", "--N=14336",
                        "--K=4096", "--dry-run", f"-o={out}", "--top=4"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert "M=8 (bucket 2) N=14336 K=4096" in r.stdout
    db = json.loads(out.read_text())
    assert len(db["entries"]) == 4
    e = db["entries"][0]
    assert e["operation"] == "fused_swiglu" and e["shape"]["M_bucket"] == 2
    assert set(e["schedule"]) == {"BM", "BN", "BK", "VM", "VN", "vector_width", "num_threads",
                                  "parallel_axis", "grain_size"}
    sel, n, st = llk.select_schedule(str(out), "fused_swiglu", 2)
    assert st == 0 and n == 4
    assert sel.BN == e["schedule"]["BN"] and sel.grain_size == e["schedule"]["grain_size"]


def test_tune_mid_m_candidates(tmp_path):
    """Mid M (the dispatcher's plan is the decode tile kernel's 128-row
    form): llk-tune's candidates are that kernel at decode_splits S, its
    records BM = 128 rows, BN = 0 (the decode tile kernel), grain_size = S;
    the same shape with midm_max_m at 64 would be a tile-kernel shape."""
    out = tmp_path / "tune.json"
    r = subprocess.run([str(BIN / "llk-tune"), "--op=fused_swiglu", "--M=100", "--N=13824",
                        "--K=5120", "--dry-run", f"-o={out}", "--top=7"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert "kernel=decode_tile (mid M)" in r.stdout
    assert "Generated 7 candidate launches" in r.stdout
    entries = json.loads(out.read_text())["entries"]
    assert [e["schedule"]["grain_size"] for e in entries] == [0, 1, 2, 3, 4, 6, 8]
    assert all(e["schedule"]["BM"] == 128 and e["schedule"]["BN"] == 0 for e in entries)
    assert all(e["shape"]["M_bucket"] == 4 for e in entries)


def _db(tmp_path, entries):
    p = tmp_path / "db.json"
    p.write_text(json.dumps({"version": 1, "entries": entries}))
    return p


def _entry(op, bucket, BN, grain):
    return {"operation": op, "target": "gfx950", "shape": {"M_bucket": bucket, "N": 1, "K": 1},
            "dtype": "bf16", "math_mode": "strict",
            "schedule": {"BM": 32, "BN": BN, "BK": 64, "VM": 32, "VN": 32, "vector_width": 8,
                         "num_threads": 256, "parallel_axis": "n", "grain_size": grain}}


def test_schedule_db_drives_launch(tmp_path):
    base_small = llk.describe_launch("fused_swiglu", 8, 14336, 4096)
    base_tile = llk.describe_launch("matmul", 255, 5120, 13824)
    base_m1 = llk.describe_launch("fused_swiglu", 1, 14336, 4096)
    db = _db(tmp_path, [_entry("fused_swiglu", 2, 128, 3), _entry("fused_swiglu", 2, 32, 1),
                        _entry("matmul", 4, 256, 5)])
    llk.set_schedule_db(db)
    try:
        p = llk.describe_launch("fused_swiglu", 8, 14336, 4096)
        assert (p["group_width"], p["splits"]) == (4, 3)  # first match wins
        assert llk.describe_launch("matmul", 255, 5120, 13824)["splits"] == 5
        # no entry for bucket 0: heuristics
        assert llk.describe_launch("fused_swiglu", 1, 14336, 4096) == base_m1
        old = llk.get_tunable("decode_splits")
        llk.set_tunable("decode_splits", 2)  # a forced knob beats the DB
        try:
            assert llk.describe_launch("fused_swiglu", 8, 14336, 4096)["splits"] == 2
        finally:
            llk.set_tunable("decode_splits", old)
    finally:
        llk.set_schedule_db(None)
    assert llk.describe_launch("fused_swiglu", 8, 14336, 4096) == base_small
    assert llk.describe_launch("matmul", 255, 5120, 13824) == base_tile
    with pytest.raises(llk.LLKError, match="NOT_FOUND"):
        llk.set_schedule_db(tmp_path / "missing.json")


def test_describe_launch_configs():
    """Plans of the BASELINE configs (kernel choice and grid sizes)."""
    p = llk.describe_launch("fused_swiglu", 2048, 11008, 4096)
    assert (p["kernel"], p["workgroups"], p["splits"], p["workspace_bytes"], p["tile_columns"]) == \
        ("wide_tile", 504, 1, 0, 176)
    # the fp32 result (pre-truncf) keeps the 128-column kernel: 688 tiles
    p = llk.describe_launch("fused_swiglu", 2048, 11008, 4096, out_f32=True)
    assert (p["kernel"], p["workgroups"], p["splits"], p["tile_columns"]) == ("tile", 688, 1, 128)
    # config 5's SwiGLU at M = 1000: 112-column tiles, 496 of them
    p = llk.describe_launch("fused_swiglu", 1000, 13824, 5120)
    assert (p["kernel"], p["workgroups"], p["tile_columns"]) == ("wide_tile", 496, 112)
    # config 4: the decode tile kernel, 64-column workgroups, unsplit
    p = llk.describe_launch("fused_swiglu", 8, 14336, 4096)
    assert (p["kernel"], p["workgroups"], p["threads_per_workgroup"], p["splits"],
            p["tile_columns"], p["workspace_bytes"], p["launches"]) == \
        ("decode_tile", 224, 256, 1, 64, 0, 1)
    # unaligned X rows: the small-M kernel
    p = llk.describe_launch("fused_swiglu", 8, 14336, 4096, x_aligned=False)
    assert p["kernel"] == "small_m" and p["workgroups"] * p["threads_per_workgroup"] >= 256 * 256
    p = llk.describe_launch("matmul", 4096, 4096, 4096)
    assert (p["kernel"], p["workgroups"]) == ("tile", 256)
    p = llk.describe_launch("fused_swiglu", 100, 1000, 1000, x_aligned=False)
    assert p["pad_x"] and p["workspace_bytes"] >= 100 * 1024 * 2
    assert llk.describe_launch("fused_swiglu", 100, 1000, 1000)["workspace_bytes"] == \
        llk.swiglu_scratch_size(100, 1000, 1000)
    from dslcompiler_amd._lib import LaunchPlan
    import ctypes as C
    plan = LaunchPlan()
    assert llk.lib().llk_describe_launch(1, 8, 8, 8, 1, C.byref(plan)) == -1  # RoPE: no kernel
    assert llk.lib().llk_describe_launch(0, 0, 8, 8, 1, C.byref(plan)) == -2


def test_tile_tail_split_plans():
    """Config 5 at M = 4097: 17 m-tiles leave a nearly empty last wave, so the
    whole n-tile columns of the first waves run unsplit and only the rest
    take a k split (GEMM: 15 columns x 17 = 255 tiles, then 5 x 17 x 3;
    SwiGLU: 105 x 17 = 1785 tiles, then 3 x 17 x 5).  Shapes whose tiles fill
    their waves, or fill too little of one, keep one launch; the knob turns it
    off; a forced split count wins."""
    p = llk.describe_launch("matmul", 4097, 5120, 13824)
    assert (p["head_blocks_n"], p["splits"], p["workgroups"], p["launches"]) == (30, 3, 510, 3)
    assert p["workspace_bytes"] == 3 * 4097 * 10 * 128 * 4  # the tail columns' planes
    p = llk.describe_launch("fused_swiglu", 4097, 13824, 5120)
    assert (p["head_blocks_n"], p["splits"], p["workgroups"], p["launches"]) == (105, 5, 2040, 3)
    for op, M, N, K in [("matmul", 4096, 4096, 4096), ("matmul", 1000, 5120, 13824),
                        ("matmul", 255, 5120, 13824)]:
        assert llk.describe_launch(op, M, N, K)["head_blocks_n"] == 0, (op, M)
    for name, value in [("tile_tail_split", 0), ("tile_splits", 2)]:
        old = llk.get_tunable(name)
        llk.set_tunable(name, value)
        try:
            p = llk.describe_launch("matmul", 4097, 5120, 13824)
            assert p["head_blocks_n"] == 0 and p["workgroups"] == 340 * p["splits"]
        finally:
            llk.set_tunable(name, old)


def test_decode_tile_split_choices():
    """The decode tile kernel's k splits for the BASELINE decode shapes:
    config 4 and the config-5 SwiGLU unsplit (224 and 216 workgroups), the
    config-5 down projection (40 n-blocks) in 6 splits, 240 workgroups in
    one round; a narrow N spreads K over more splits; a forced count is
    kept; unaligned X, `decode_tile` = 0 and a forced group width route to
    the small-M kernel."""
    plan = lambda op, M, N, K, **kw: (lambda p: (p["kernel"], p["splits"], p["workgroups"]))(  # noqa: E731
        llk.describe_launch(op, M, N, K, **kw))
    for M in (1, 8, 16, 64):
        assert plan("fused_swiglu", M, 14336, 4096) == ("decode_tile", 1, 224)
    for M in (1, 17):
        assert plan("fused_swiglu", M, 13824, 5120) == ("decode_tile", 1, 216)
    for M in (1, 17, 64):
        assert plan("matmul", M, 5120, 13824) == ("decode_tile", 6, 240)
    assert plan("fused_swiglu", 8, 128, 4096)[1] > 8
    assert plan("fused_swiglu", 8, 14336, 4096, x_aligned=False)[0] == "small_m"
    assert plan("fused_swiglu", 8, 14336, 4000)[0] == "small_m"  # K % 64 != 0
    for name, value in (("decode_splits", 3), ("decode_tile", 0), ("decode_group_width", 2)):
        old = llk.get_tunable(name)
        llk.set_tunable(name, value)
        try:
            p = plan("fused_swiglu", 8, 14336, 4096)
            assert p[0] == ("decode_tile" if name == "decode_splits" else "small_m"), (name, p)
            if name == "decode_splits":
                assert p[1:] == (3, 672)
        finally:
            llk.set_tunable(name, old)
    assert llk.get_tunable("decode_tile") == 1


def test_small_m_cost_model_choices():
    """The small-M dispatcher's (width, splits) -- for X the decode tile
    kernel does not take, here with `decode_tile` = 0 -- against llk-tune's
    measured best on MI355X for the BASELINE decode shapes: config 1 (M=64,
    N=1376, K=512: 8.27 us at width 1 unsplit; every split adds ~2.8 us),
    config 4 (width 2 unsplit, 224 workgroups), M=64 decode (width 2: 53.9
    us vs 68.0 at width 1), the config-5 down projection (width 2, 3 splits:
    240 workgroups in one round)."""
    old_t = llk.get_tunable("decode_tile")
    llk.set_tunable("decode_tile", 0)
    try:
        _small_m_choices()
    finally:
        llk.set_tunable("decode_tile", old_t)


def _small_m_choices():
    plan = lambda op, M, N, K: (lambda p: (p["group_width"], p["splits"]))(  # noqa: E731
        llk.describe_launch(op, M, N, K))
    assert plan("fused_swiglu", 64, 1376, 512) == (1, 1)
    for M in (1, 8, 16, 64):
        assert plan("fused_swiglu", M, 14336, 4096) == (2, 1)
    assert plan("fused_swiglu", 17, 13824, 5120) == (2, 1)
    for M in (1, 17, 64):
        assert plan("matmul", M, 5120, 13824) == (2, 3)
    # a narrow N spreads K over splits instead
    w, s = plan("fused_swiglu", 8, 128, 4096)
    assert s > 8
    # forced knobs are kept as given
    old_w, old_s = llk.get_tunable("decode_group_width"), llk.get_tunable("decode_splits")
    try:
        llk.set_tunable("decode_group_width", 4)
        assert plan("fused_swiglu", 64, 1376, 512)[0] == 4
        llk.set_tunable("decode_splits", 2)
        assert plan("fused_swiglu", 8, 14336, 4096) == (4, 2)
    finally:
        llk.set_tunable("decode_group_width", old_w)
        llk.set_tunable("decode_splits", old_s)
    assert old_w == 0 and old_s == 0  # defaults: chosen by the cost model


def test_tile_kernel_k_limit():
    """K beyond the tile kernel's 32-bit offsets is an error, not a launch;
    M <= 256 runs it on the decode tile kernel, and at M <= 64 a K beyond that
    kernel's 32-bit offsets (a weight panel of 2 GiB) on the small-M kernel,
    which has no such limit."""
    K = 1 << 22
    with pytest.raises(llk.LLKError, match="too large"):
        llk.describe_launch("fused_swiglu", 300, 256, K)
    assert llk.describe_launch("fused_swiglu", 8, 256, K)["kernel"] == "decode_tile"
    assert llk.describe_launch("fused_swiglu", 8, 256, 1 << 27)["kernel"] == "small_m"
    assert llk.describe_launch("fused_swiglu", 300, 256, K - 128)["kernel"] == "tile"
    # mid M (the decode tile kernel's 128- and 256-row forms) up to its own
    # limit: 256 rows of X and a weight panel within 32-bit offsets
    assert llk.describe_launch("fused_swiglu", 100, 256, K)["kernel"] == "decode_tile"
    assert llk.describe_launch("fused_swiglu", 120, 256, K - 128)["kernel"] == "decode_tile"
    assert llk.describe_launch("fused_swiglu", 200, 256, K - 128)["kernel"] == "tile"
