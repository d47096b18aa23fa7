"""The accumulating GEMM, C += A B: micro.mma's  acc += lhs * rhs
(MicroOps.td:196-222) and llk.matmul with a non-zero outs(init).

Two checks per launch path (small-M kernel with and without k splits, tile
kernel with one or more splits, padded X) and output type:
- bit-exact against the kernel's own C = A B: the accumulating call sums
  the products in the same order, then adds C in fp32 and rounds once, so
  it must equal  round(P + widen(C0))  computed here from the fp32 P;
- against the oracle with the same initial accumulator (orc_gemm_init,
  pinned in test_oracle.py by the integer closed form C0 + A B), to the
  north-star bar.
K = 0 leaves C untouched bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

from common import (assert_parity, assert_parity_bf16, bf16_bits_to_f32, normal_bf16,
                    to_bf16_bits)
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu

CASES = [  # M, N, K: the plan C = A B takes
    (8, 1024, 512),      # small-M, no split
    (64, 1024, 4096),    # small-M, S = 16
    (1, 5120, 13824),    # small-M, S = 3
    (700, 768, 384),     # tile, no split (accumulating: one partial plane)
    (1000, 1024, 512),   # tile, S = 2
    (300, 640, 1000),    # tile, S = 4, padded X
]
OUTS = ["fp32", "bf16", "fp16"]


def _c0(gpu, M, N, out, seed):
    c0 = normal_bf16(seed, 9, (M, N))  # bf16 bits of N(0, 1)
    f = bf16_bits_to_f32(c0)
    if out == "fp32":
        return gpu.from_numpy(f).cuda(), f
    if out == "bf16":
        return to_dev(gpu, c0), f
    h = f.astype(np.float16)
    return gpu.from_numpy(h).cuda(), h.astype(np.float32)


def _round(v: np.ndarray, out: str) -> np.ndarray:
    """fp32 values rounded to the output type, compared as raw bits."""
    if out == "fp32":
        return v.astype(np.float32).view(np.uint32)
    if out == "bf16":
        return to_bf16_bits(v.astype(np.float32))
    return v.astype(np.float32).astype(np.float16).view(np.uint16)


def _bits(t, out: str) -> np.ndarray:
    a = t.cpu().contiguous().numpy() if out != "bf16" else from_dev(t)
    return a.view(np.uint32) if out == "fp32" else a.view(np.uint16)


@pytest.mark.parametrize("out", OUTS)
@pytest.mark.parametrize("M,N,K", CASES)
def test_accumulate_is_rounded_sum(llk, gpu, M, N, K, out):
    print(f"case gemm accumulate M={M} N={N} K={K} {out}", flush=True)
    assert llk.describe_launch("matmul", M, N, K, K % 64 == 0)["head_blocks_n"] == 0
    a = normal_bf16(21, 0, (M, K))
    b = normal_bf16(21, 1, (K, N), 1.0 / np.sqrt(K))
    ad, pb = to_dev(gpu, a), llk.PackedWeights.from_host(b)
    p = from_dev(llk.matmul(ad, pb, out_dtype=gpu.float32))  # the kernel's fp32 P
    c, c0 = _c0(gpu, M, N, out, seed=M + K)
    llk.matmul(ad, pb, out=c, accumulate=True)
    gpu.cuda.synchronize()
    want = _round(p + c0, out)
    got = _bits(c, out)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} elements differ from round(P + C0); first {bad[:5]}"


@pytest.mark.parametrize("M,N,K", [(64, 1024, 4096), (1000, 1024, 512), (300, 640, 1000)])
def test_accumulate_against_oracle(llk, gpu, orc, M, N, K):
    print(f"case gemm accumulate vs oracle M={M} N={N} K={K}", flush=True)
    a = normal_bf16(22, 0, (M, K))
    b = normal_bf16(22, 1, (K, N), 1.0 / np.sqrt(K))
    ad, pb = to_dev(gpu, a), llk.PackedWeights.from_host(b)
    cf, c0 = _c0(gpu, M, N, "fp32", seed=5)
    cb, _ = _c0(gpu, M, N, "bf16", seed=5)
    llk.matmul(ad, pb, out=cf, accumulate=True)
    llk.matmul(ad, pb, out=cb, accumulate=True)
    gpu.cuda.synchronize()
    ref, _ = orc.gemm_avx2(a, b, 8, c_init=c0, want_bf16=False)
    assert_parity(from_dev(cf), ref, "accumulate fp32")
    assert_parity_bf16(from_dev(cb), ref, "accumulate bf16")
    # the accumulator matters: C0 + A B is not A B
    assert np.abs(from_dev(cf) - from_dev(llk.matmul(ad, pb, out_dtype=gpu.float32))).max() > 1.0


def test_accumulate_k0_leaves_c(llk, gpu):
    print("case gemm accumulate K=0", flush=True)
    M, N = 17, 640
    a = gpu.empty((M, 0), dtype=gpu.bfloat16, device="cuda")
    pb = llk.PackedWeights.from_host(np.zeros((0, N), np.uint16))
    c = gpu.full((M, N), -0.0, dtype=gpu.float32, device="cuda")
    c[0, :5] = gpu.tensor([1.0, float("nan"), -3.5, float("inf"), 7.0])
    before = c.cpu().numpy().view(np.uint32).copy()
    llk.matmul(a, pb, out=c, accumulate=True)
    gpu.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy().view(np.uint32), before)
