"""GPU tests of contract edge cases of the two ops: the empty reduction
(K = 0), which the reference's verifiers accept (LLKOps.cpp:42-83 for
llk.fused_swiglu, LLKOps.cpp:336-348 for llk.matmul) and whose zero-filled
fp32 accumulators (FuseDoubleContraction.cpp:119-135) give SiLU(0) * 0 = +0
and C = 0, on both the small-M and the tile kernels' paths."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import from_dev

pytestmark = pytest.mark.gpu


def _garbage(gpu, M, N, dtype, stride=None):
    """An output buffer full of non-zero bits (NaN for floats), optionally a
    view with a wider row stride whose padding must stay untouched."""
    cols = N if stride is None else stride
    y = gpu.full((M, cols), float("nan"), dtype=dtype, device="cuda")
    return y if stride is None else y[:, :N]


@pytest.mark.parametrize("M,N", [(1, 256), (8, 1000), (64, 130), (300, 1000), (2049, 384)])
@pytest.mark.parametrize("out", ["bf16", "fp32"])
def test_swiglu_k0(llk, gpu, M, N, out):
    print(f"case swiglu K=0 M={M} N={N} out={out}", flush=True)
    dtype = {"bf16": gpu.bfloat16, "fp32": gpu.float32}[out]
    x = gpu.empty((M, 0), dtype=gpu.bfloat16, device="cuda")
    pg = llk.PackedWeights.from_host(np.zeros((0, N), np.uint16))
    pu = llk.PackedWeights.from_host(np.zeros((0, N), np.uint16))
    y = _garbage(gpu, M, N, dtype, stride=N + 8)
    llk.fused_swiglu(x, pg, pu, out=y)
    gpu.cuda.synchronize()
    got = from_dev(y)
    assert not np.any(got.view(np.uint16 if out == "bf16" else np.uint32)), "K=0 must give +0"
    pad = from_dev(y.as_strided((M, 8), (N + 8, 1), y.storage_offset() + N))
    assert np.all(np.isnan(pad.view(np.float32) if out == "fp32" else
                           (pad.astype(np.uint32) << 16).view(np.float32))), "row padding written"


@pytest.mark.parametrize("M,N", [(1, 256), (17, 640), (256, 512), (1000, 130)])
@pytest.mark.parametrize("out", ["bf16", "fp16", "fp32"])
def test_gemm_k0(llk, gpu, M, N, out):
    print(f"case gemm K=0 M={M} N={N} out={out}", flush=True)
    dtype = {"bf16": gpu.bfloat16, "fp16": gpu.float16, "fp32": gpu.float32}[out]
    a = gpu.empty((M, 0), dtype=gpu.bfloat16, device="cuda")
    pb = llk.PackedWeights.from_host(np.zeros((0, N), np.uint16))
    c = _garbage(gpu, M, N, dtype)
    llk.matmul(a, pb, out=c)
    gpu.cuda.synchronize()
    got = c.cpu().float().numpy()
    assert np.all(got == 0) and not np.any(np.signbit(got)), "K=0 must give C = +0"


def test_k0_plan_and_mlp(llk, gpu):
    """K = 0 through the MLP block: Y = 0, then Z = Y Wd = 0."""
    print("case mlp K=0", flush=True)
    M, N, Ko = 5, 256, 128
    x = gpu.empty((M, 0), dtype=gpu.bfloat16, device="cuda")
    pg = llk.PackedWeights.from_host(np.zeros((0, N), np.uint16))
    pu = llk.PackedWeights.from_host(np.zeros((0, N), np.uint16))
    rng = np.random.default_rng(0)
    wd = (rng.standard_normal((N, Ko)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    pd = llk.PackedWeights.from_host(wd)
    y, z = llk.mlp(x, pg, pu, pd)
    gpu.cuda.synchronize()
    assert not np.any(from_dev(y)) and not np.any(from_dev(z))
