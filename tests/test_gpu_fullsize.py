"""GPU tests at the BASELINE.json sizes.  The CPU oracle is too slow for whole
outputs, so each test checks sampled rows against the oracle (to the
north-star bar) plus size-independent properties: bit-identical reruns,
and bf16 output = RNE of the same kernel's fp32 output."""
from __future__ import annotations

import numpy as np
import pytest

from common import (STREAM_WD, assert_parity, assert_parity_bf16, bf16_bits_to_f32, normal_bf16,
                    outliers, swiglu_inputs, to_bf16_bits)
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _swiglu_dev(llk, torch, xd, pg, pu, dtype):
    y = llk.fused_swiglu(xd, pg, pu, out_dtype=dtype)
    torch.cuda.synchronize()
    return from_dev(y)


def test_config3_prefill_2048x4096x11008(llk, gpu, orc):
    """Config 3: prefill SwiGLU M=2048, K=4096, N=11008, bf16 out."""
    print("case config3 full size", flush=True)
    M, K, N = 2048, 4096, 11008
    x, wg, wu = swiglu_inputs(M, K, N, seed=42)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x)
    yb = _swiglu_dev(llk, gpu, xd, pg, pu, gpu.bfloat16)
    yb2 = _swiglu_dev(llk, gpu, xd, pg, pu, gpu.bfloat16)
    assert np.array_equal(yb, yb2), "reruns differ"
    yf = _swiglu_dev(llk, gpu, xd, pg, pu, gpu.float32)
    assert np.array_equal(yb, to_bf16_bits(yf))
    rows = [0, 255, 256, 1023, 2047]
    yf_ref, _ = orc.swiglu_rows(x, wg, wu, rows)
    assert_parity(yf[rows], yf_ref, "config3 fp32 rows")
    assert_parity_bf16(yb[rows], yf_ref, "config3 bf16 rows")


@pytest.mark.parametrize("M", [1, 8, 16])
def test_config4_decode(llk, gpu, orc, M):
    """Config 4: decode SwiGLU M in {1, 8, 16}, K=4096, N=14336 (all rows)."""
    print(f"case config4 M={M}", flush=True)
    K, N = 4096, 14336
    x, wg, wu = swiglu_inputs(M, K, N, seed=42)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x)
    yb = _swiglu_dev(llk, gpu, xd, pg, pu, gpu.bfloat16)
    yf = _swiglu_dev(llk, gpu, xd, pg, pu, gpu.float32)
    assert np.array_equal(yb, _swiglu_dev(llk, gpu, xd, pg, pu, gpu.bfloat16))
    assert np.array_equal(yb, to_bf16_bits(yf))
    yf_ref, _ = orc.swiglu(x, wg, wu)
    assert_parity(yf, yf_ref, f"config4 M={M} fp32")
    assert_parity_bf16(yb, yf_ref, f"config4 M={M} bf16")


def test_config2_gemm_4096(llk, gpu, orc):
    """Config 2: C = A B, 4096^3, fp32 out (sampled rows + fp64 brute force)."""
    print("case config2 gemm 4096^3", flush=True)
    n = 4096
    s = 1.0 / np.sqrt(n)
    a = normal_bf16(42, 0, (n, n), s)
    b = normal_bf16(42, 1, (n, n), s)
    pb = llk.PackedWeights.from_host(b)
    c = from_dev(llk.matmul(to_dev(gpu, a), pb, out_dtype=gpu.float32))
    rows = [0, 1, 2048, 4095]
    cf_ref, _ = orc.gemm(a[rows], b)
    assert_parity(c[rows], cf_ref, "config2 rows")
    c64 = orc.gemm_fp64(a[rows[:1]], b)
    assert np.max(np.abs(c[rows[:1]] - c64)) < 1e-4


@pytest.mark.parametrize("M", [1, 17, 255, 1000, 4097])
def test_config5_mlp(llk, gpu, orc, M):
    """Config 5: SwiGLU (K=5120, N=13824) then Z = Y Wd, Wd [13824, 5120];
    ragged M; 1% of X scaled x20; bf16 out.  Each stage against the oracle on
    sampled rows; Z against the oracle applied to the GPU's own Y."""
    print(f"case config5 M={M}", flush=True)
    K, N = 5120, 13824
    x, wg, wu = swiglu_inputs(M, K, N, seed=42)
    x = outliers(x, seed=42)
    wd = normal_bf16(42, STREAM_WD, (N, K), 1.0 / np.sqrt(N))
    pg, pu, pd = (llk.PackedWeights.from_host(w) for w in (wg, wu, wd))
    yd, zd = llk.mlp(to_dev(gpu, x), pg, pu, pd)
    gpu.cuda.synchronize()
    y, z = from_dev(yd), from_dev(zd)
    rows = sorted({0, M // 2, M - 1})
    yf_ref, _ = orc.swiglu_rows(x, wg, wu, rows)
    assert_parity_bf16(y[rows], yf_ref, f"config5 M={M} Y")
    zf_ref, _ = orc.gemm(y[rows], wd)
    assert_parity_bf16(z[rows], zf_ref, f"config5 M={M} Z")


def test_x_beyond_32bit_offsets_launches_in_chunks(llk, gpu, orc):
    """M * K * 2 bytes > 2^31: the tile kernel's 32-bit X offsets force row
    chunks (aligned X, and padded X with K % 64 != 0)."""
    for K in (4096, 4000):
        M, N = 270_000, 128
        print(f"case chunked X M={M} K={K}", flush=True)
        assert M * K * 2 >= 1 << 31
        x = gpu.randn((M, K), device="cuda").to(gpu.bfloat16)
        wg = normal_bf16(7, 1, (K, N), 1.0 / np.sqrt(K))
        wu = normal_bf16(7, 2, (K, N), 1.0 / np.sqrt(K))
        pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
        plan = llk.describe_launch("fused_swiglu", M, N, K)
        assert plan["launches"] >= 2
        y = llk.fused_swiglu(x, pg, pu, out_dtype=gpu.float32)
        gpu.cuda.synchronize()
        rows = [0, 131071, 131072, 262143, 262144, M - 1]
        xs = from_dev(x[rows])
        yf_ref, _ = orc.swiglu(xs, wg, wu)
        assert_parity(from_dev(y[rows]), yf_ref, f"chunked K={K}")
        del x, y
        gpu.cuda.empty_cache()
