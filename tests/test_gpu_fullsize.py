"""GPU tests at the BASELINE.json sizes.  Every output row is compared with
the oracle (to the north-star bar) through its multithreaded AVX2 legs,
which are bit-equal to the scalar sequential-k oracle (test_oracle.py), so a
misplaced or swapped tile anywhere in the output fails; plus size-independent
properties: bit-identical reruns, and bf16 output = RNE of the same kernel's
fp32 output."""
from __future__ import annotations

import os

import numpy as np
import pytest

from common import (STREAM_WD, assert_parity, assert_parity_bf16, bf16_bits_to_f32, normal_bf16,
                    outliers, swiglu_inputs, to_bf16_bits)
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _threads() -> int:
    """Host threads for the oracle legs (at most 16: the GPU box's CPU share)."""
    return max(1, min(16, os.cpu_count() or 1))


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
    _, yf_ref = orc.swiglu_avx2(x, wg, wu, _threads(), want_f32=True)
    assert_parity(yf, yf_ref, "config3 fp32 (all rows)")
    assert_parity_bf16(yb, yf_ref, "config3 bf16 (all rows)")
    # every 256 x 128 output tile on its own (a swapped tile would pass a
    # global norm only if the two tiles were alike)
    for m0 in range(0, M, 256):
        for n0 in range(0, N, 128):
            t = (slice(m0, m0 + 256), slice(n0, n0 + 128))
            assert_parity(yf[t], yf_ref[t], f"config3 tile m0={m0} n0={n0}")


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
    """Config 2: C = A B, 4096^3, fp32 out (all rows + fp64 brute force)."""
    print("case config2 gemm 4096^3", flush=True)
    n = 4096
    s = 1.0 / np.sqrt(n)
    a = normal_bf16(42, 0, (n, n), s)
    b = normal_bf16(42, 1, (n, n), s)
    pb = llk.PackedWeights.from_host(b)
    c = from_dev(llk.matmul(to_dev(gpu, a), pb, out_dtype=gpu.float32))
    cf_ref, _ = orc.gemm_avx2(a, b, _threads(), want_bf16=False)
    assert_parity(c, cf_ref, "config2 (all rows)")
    for m0 in range(0, n, 256):
        for n0 in range(0, n, 256):
            t = (slice(m0, m0 + 256), slice(n0, n0 + 256))
            assert_parity(c[t], cf_ref[t], f"config2 tile m0={m0} n0={n0}")
    c64 = orc.gemm_fp64(a[:1], b)
    assert np.max(np.abs(c[:1] - c64)) < 1e-4


@pytest.mark.parametrize("M", [1, 17, 65, 128, 255, 1000, 4097])
def test_config5_mlp(llk, gpu, orc, M):
    """Config 5: SwiGLU (K=5120, N=13824) then Z = Y Wd, Wd [13824, 5120];
    ragged M (65 and 128: the mid-M forms, between config 5's rows); 1% of X
    scaled x20; bf16 out.  Each stage against the oracle on every row; Z
    against the oracle applied to the GPU's own Y."""
    print(f"case config5 M={M}", flush=True)
    K, N = 5120, 13824
    x, wg, wu = swiglu_inputs(M, K, N, seed=42)
    x = outliers(x, seed=42)
    wd = normal_bf16(42, STREAM_WD, (N, K), 1.0 / np.sqrt(N))
    pg, pu, pd = (llk.PackedWeights.from_host(w) for w in (wg, wu, wd))
    yd, zd = llk.mlp(to_dev(gpu, x), pg, pu, pd)
    gpu.cuda.synchronize()
    y, z = from_dev(yd), from_dev(zd)
    _, yf_ref = orc.swiglu_avx2(x, wg, wu, _threads(), want_f32=True)
    assert_parity_bf16(y, yf_ref, f"config5 M={M} Y (all rows)")
    zf_ref, _ = orc.gemm_avx2(y, wd, _threads(), want_bf16=False)
    assert_parity_bf16(z, zf_ref, f"config5 M={M} Z (all rows)")
    for m0 in range(0, M, 256):
        rs = slice(m0, m0 + 256)
        assert_parity_bf16(y[rs], yf_ref[rs], f"config5 M={M} Y rows {m0}..")
        assert_parity_bf16(z[rs], zf_ref[rs], f"config5 M={M} Z rows {m0}..")


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
