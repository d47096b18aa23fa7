"""Entries of the object-code level run the kernels of their operation's
gfx950 code object, loaded with hipModuleLoadData and resolved with
hipModuleGetFunction (the reference's lookupOrCompile hands back the
JIT-compiled entry of a key: JitCache.cpp:182-245).  The objects are built
from the same sources as the library, so every launch path must give the
library's own output bit for bit: the decode tile and small-M kernels
with and without k splits, tile kernels with and without k splits, the wide SwiGLU kernel at
both widths and with a k split, padded X and the K = 0 fill; two cases are
also held to the oracle."""
from __future__ import annotations

import re

import numpy as np
import pytest

from common import assert_parity, assert_parity_bf16, normal_bf16, swiglu_inputs
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu

OUT = {"bf16": 0, "fp32": 2}

# (operation, M, N, K, output, launch the dispatcher picks)
CASES = [
    ("fused_swiglu", 1, 1024, 4096, "bf16", "decode tile, S = 16"),
    ("fused_swiglu", 40, 640, 512, "fp32", "decode tile, S = 4"),
    ("fused_swiglu", 64, 1376, 512, "bf16", "decode tile (config 1)"),
    ("fused_swiglu", 1, 1024, 4000, "bf16", "small-M, S = 8"),
    ("fused_swiglu", 40, 640, 1000, "fp32", "small-M, two row groups, S = 8"),
    ("fused_swiglu", 300, 640, 1000, "bf16", "tile, S = 4, padded X"),
    ("fused_swiglu", 600, 1280, 512, "bf16", "wide tile, B = 7"),
    ("fused_swiglu", 2048, 11008, 512, "bf16", "wide tile, B = 11"),
    ("fused_swiglu", 255, 13824, 5120, "bf16", "wide tile, B = 7, S = 2 (config 5)"),
    ("matmul", 1, 5120, 13824, "bf16", "decode tile, S = 6"),
    ("matmul", 64, 1024, 4096, "fp32", "decode tile, S = 22"),
    ("matmul", 64, 1024, 4000, "fp32", "small-M, S = 16"),
    ("matmul", 300, 640, 1000, "fp32", "tile, S = 4, padded X"),
    ("matmul", 1000, 1024, 512, "bf16", "tile, S = 2"),
]


def _entry(llk, cache, op, N, K, out):
    key = llk.KernelKey(operation=0 if op == "fused_swiglu" else 3, isa=7, N=N, K=K,
                        output_type=OUT[out], M_bucket=llk.classify_m(1))
    return cache.lookup_or_compile_packed(key)


@pytest.mark.parametrize("op,M,N,K,out,what", CASES, ids=[f"{c[0]}-{c[1]}x{c[2]}x{c[3]}"
                                                           for c in CASES])
def test_entry_matches_library_kernels(llk, gpu, op, M, N, K, out, what):
    print(f"case code object {op} M={M} N={N} K={K} {out} ({what})", flush=True)
    plan = llk.describe_launch(op, M, N, K, x_aligned=K % 64 == 0)
    assert (plan["kernel"] == "small_m") == what.startswith("small-M")
    assert (plan["kernel"] == "decode_tile") == what.startswith("decode tile")
    assert (plan["kernel"] == "wide_tile") == what.startswith("wide")
    wide = re.search(r"B = (\d+)", what)
    if wide:
        assert plan["tile_columns"] == 16 * int(wide.group(1)), plan
    assert plan["pad_x"] == ("padded" in what)
    splits = re.search(r"S = (\d+)", what)
    assert plan["splits"] == (int(splits.group(1)) if splits else 1)
    dtype = {"bf16": gpu.bfloat16, "fp32": gpu.float32}[out]
    cache = llk.JitCache()
    fn = _entry(llk, cache, op, N, K, out)
    x, wg, wu = swiglu_inputs(M, K, N, seed=11)
    xd = to_dev(gpu, x)
    pg = llk.PackedWeights.from_host(wg)
    y = gpu.full((M, N), float("nan"), dtype=dtype, device="cuda")
    if op == "fused_swiglu":
        pu = llk.PackedWeights.from_host(wu)
        fn(xd, pg, pu, y)
        ref = llk.fused_swiglu(xd, pg, pu, out_dtype=dtype)
    else:
        fn(xd, pg, None, y)
        ref = llk.matmul(xd, pg, out_dtype=dtype)
    gpu.cuda.synchronize()
    got = from_dev(y)
    assert np.array_equal(got, from_dev(ref)), f"{op} {what}: differs from the library's kernels"
    cache.close()


def test_entries_against_oracle(llk, gpu, orc):
    print("case code object entries vs oracle", flush=True)
    cache = llk.JitCache()
    M, K, N = 300, 1000, 640
    x, wg, wu = swiglu_inputs(M, K, N, seed=12)
    xd = to_dev(gpu, x)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    y = gpu.empty((M, N), dtype=gpu.bfloat16, device="cuda")
    _entry(llk, cache, "fused_swiglu", N, K, "bf16")(xd, pg, pu, y)
    c = gpu.empty((M, N), dtype=gpu.float32, device="cuda")
    _entry(llk, cache, "matmul", N, K, "fp32")(xd, pg, None, c)
    gpu.cuda.synchronize()
    yf_ref, _ = orc.swiglu(x, wg, wu)
    assert_parity_bf16(from_dev(y), yf_ref, "swiglu entry")
    cf_ref, _ = orc.gemm(x, wg, want_bf16=False)
    assert_parity(from_dev(c), cf_ref, "matmul entry")
    cache.close()


def test_k0_and_output_type_binding(llk, gpu):
    print("case code object K=0 and dtype binding", flush=True)
    cache = llk.JitCache()
    M, N = 17, 256
    fn = _entry(llk, cache, "fused_swiglu", N, 64, "bf16")
    x = gpu.empty((M, 0), dtype=gpu.bfloat16, device="cuda")
    pz = llk.PackedWeights.from_host(np.zeros((0, N), np.uint16))
    y = gpu.full((M, N), float("nan"), dtype=gpu.bfloat16, device="cuda")
    fn(x, pz, pz, y)  # K = 0: the object's fill kernel writes +0
    gpu.cuda.synchronize()
    assert not np.any(from_dev(y))
    # the entry of a bf16 key refuses another output type
    xk = to_dev(gpu, normal_bf16(3, 0, (M, 64)))
    pw = llk.PackedWeights.from_host(normal_bf16(3, 1, (64, N), 0.125))
    yf = gpu.empty((M, N), dtype=gpu.float32, device="cuda")
    with pytest.raises(llk.LLKError, match="DTYPE.*output type 0 called with output type 2"):
        fn(xk, pw, pw, yf)
    cache.close()
