"""The decode tile kernel (M <= 64, K a multiple of 64, 16-byte aligned X
rows): weights and X streamed through an LDS-DMA ring, against the CPU
oracle -- SwiGLU (bf16 and fp32 results) and the GEMM (bf16, fp16, fp32,
accumulate), ragged M and N, X row strides wider than K, forced k splits --
and the routing around it: unaligned X and K % 64 != 0 take the small-M
kernel, `decode_tile` = 0 or a forced group width too, with results that
agree with the decode tile kernel's."""
from __future__ import annotations

import numpy as np
import pytest

from common import (assert_parity, assert_parity_bf16, normal_bf16, swiglu_inputs,
                    to_bf16_bits)
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu


class _Tunable:
    def __init__(self, llk, name, value):
        self.llk, self.name, self.value = llk, name, value

    def __enter__(self):
        self.old = self.llk.get_tunable(self.name)
        self.llk.set_tunable(self.name, self.value)

    def __exit__(self, *exc):
        self.llk.set_tunable(self.name, self.old)


def _swiglu(llk, gpu, x, pg, pu, dtype, x_stride=None):
    xd = to_dev(gpu, x, x_stride)
    y = llk.fused_swiglu(xd, pg, pu, out_dtype=dtype)
    gpu.cuda.synchronize()
    return from_dev(y)


def _check(llk, gpu, orc, M, K, N, seed, what, x_stride=None, kernel="decode_tile"):
    x, wg, wu = swiglu_inputs(M, K, N, seed=seed)
    plan = llk.describe_launch("fused_swiglu", M, N, K,
                               x_aligned=(x_stride or K) % 8 == 0 and K % 8 == 0)
    assert plan["kernel"] == kernel, (what, plan)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    yf_ref, _ = orc.swiglu(x, wg, wu)
    yb = _swiglu(llk, gpu, x, pg, pu, gpu.bfloat16, x_stride)
    yf = _swiglu(llk, gpu, x, pg, pu, gpu.float32, x_stride)
    assert_parity_bf16(yb, yf_ref, what + " bf16")
    assert_parity(yf, yf_ref, what + " fp32")
    assert np.array_equal(yb, to_bf16_bits(yf)), what + ": bf16 != RNE(fp32)"
    return x, pg, pu, yf


# (M, K, N): one and two 32-row tiles, ragged M, ragged N (partial 64- and
# 128-column groups), one 64-k step, odd step counts, wide N.
SHAPES = [(1, 512, 392), (8, 1024, 1376), (17, 576, 600), (32, 64, 200), (33, 640, 200),
          (64, 512, 1376), (64, 4096, 256), (5, 128, 96), (48, 1984, 2112)]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_swiglu_against_oracle(llk, gpu, orc, M, K, N):
    print(f"case decode tile swiglu M={M} K={K} N={N}", flush=True)
    _check(llk, gpu, orc, M, K, N, seed=M * 7 + K, what=f"swiglu M{M} K{K} N{N}")


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_gemm_against_oracle(llk, gpu, orc, M, K, N):
    print(f"case decode tile gemm M={M} K={K} N={N}", flush=True)
    a = normal_bf16(31, 0, (M, K))
    b = normal_bf16(31, 1, (K, N), 1.0 / np.sqrt(K))
    assert llk.describe_launch("matmul", M, N, K)["kernel"] == "decode_tile"
    cf_ref, _ = orc.gemm(a, b)
    ad, pb = to_dev(gpu, a), llk.PackedWeights.from_host(b)
    cf = from_dev(llk.matmul(ad, pb, out_dtype=gpu.float32))
    cb = from_dev(llk.matmul(ad, pb, out_dtype=gpu.bfloat16))
    ch = llk.matmul(ad, pb, out_dtype=gpu.float16).cpu().numpy()
    assert_parity(cf, cf_ref, f"gemm M{M} fp32")
    assert_parity_bf16(cb, cf_ref, f"gemm M{M} bf16")
    assert np.array_equal(cb, to_bf16_bits(cf)), "bf16 != RNE(fp32)"
    assert np.array_equal(ch.view(np.uint16), cf.astype(np.float16).view(np.uint16)), \
        "fp16 != RNE(fp32)"


@pytest.mark.parametrize("S", [2, 3, 5, 8])
def test_forced_splits(llk, gpu, orc, S):
    """k splits through the partial planes and the split-order reduce, for
    both operations (the last split shorter than the others at S = 3, 5; S = 8
    over 20 k-steps runs as 7 splits of 3 steps: no empty split)."""
    print(f"case decode tile splits S={S}", flush=True)
    M, K, N = 24, 1280, 720
    kbs = -(-(K // 64) // S)
    with _Tunable(llk, "decode_splits", S):
        plan = llk.describe_launch("fused_swiglu", M, N, K)
        assert plan["kernel"] == "decode_tile" and plan["splits"] == -(-(K // 64) // kbs), plan
        assert plan["launches"] == 2 and plan["workspace_bytes"] > 0
        _check(llk, gpu, orc, M, K, N, seed=S, what=f"swiglu S{S}")
        a = normal_bf16(32, 0, (M, K))
        b = normal_bf16(32, 1, (K, N), 1.0 / np.sqrt(K))
        cf_ref, _ = orc.gemm(a, b)
        cf = from_dev(llk.matmul(to_dev(gpu, a), llk.PackedWeights.from_host(b),
                                 out_dtype=gpu.float32))
    assert_parity(cf, cf_ref, f"gemm S{S}")


@pytest.mark.parametrize("S", [1, 4])
def test_gemm_accumulate(llk, gpu, orc, S):
    """C += A B on the decode tile kernel: in its epilogue (S = 1) and in
    the split reduce (S = 4); the result is the oracle's C0 + A B."""
    print(f"case decode tile gemm accumulate S={S}", flush=True)
    M, K, N = 40, 2048, 640
    a = normal_bf16(33, 0, (M, K))
    b = normal_bf16(33, 1, (K, N), 1.0 / np.sqrt(K))
    c0 = np.random.default_rng(S).standard_normal((M, N)).astype(np.float32)
    ref, _ = orc.gemm_avx2(a, b, 8, c_init=c0, want_bf16=False)
    with _Tunable(llk, "decode_splits", S):
        plan = llk.describe_launch("matmul", M, N, K, accumulate=True)
        assert plan["kernel"] == "decode_tile" and plan["splits"] == S, plan
        c = gpu.from_numpy(c0.copy()).cuda()
        llk.matmul(to_dev(gpu, a), llk.PackedWeights.from_host(b), out=c, accumulate=True)
        gpu.cuda.synchronize()
    assert_parity(c.cpu().numpy(), ref, f"accumulate S{S}")


def test_wide_x_stride(llk, gpu, orc):
    """X rows wider than K (stride a multiple of 8 elements): the kernel reads
    only the first K columns of each row."""
    print("case decode tile wide X stride", flush=True)
    _check(llk, gpu, orc, 20, 512, 300, seed=5, what="stride K + 72", x_stride=512 + 72)


def test_routing_and_agreement_with_small_m_kernel(llk, gpu, orc):
    """Shapes the decode tile kernel does not take run on the small-M kernel
    (X rows not 16-byte aligned; K not a multiple of 64), and with the
    kernel turned off or a group width forced the same call runs on the
    small-M kernel; both stay on the oracle and agree to the bar."""
    print("case decode tile routing", flush=True)
    _check(llk, gpu, orc, 16, 520, 256, seed=6, what="unaligned X", x_stride=521,
           kernel="small_m")
    _check(llk, gpu, orc, 16, 1000, 256, seed=7, what="K % 64 != 0", kernel="small_m")
    x, pg, pu, yf_tile = _check(llk, gpu, orc, 12, 1024, 520, seed=8, what="decode tile")
    for knob, value in (("decode_tile", 0), ("decode_group_width", 2)):
        with _Tunable(llk, knob, value):
            assert llk.describe_launch("fused_swiglu", 12, 520, 1024)["kernel"] == "small_m"
            yf = _swiglu(llk, gpu, x, pg, pu, gpu.float32)
        assert_parity(yf, yf_tile, f"small-M vs decode tile ({knob}={value})")


def test_exact_integers(llk, gpu, orc):
    """Small-integer inputs: every partial sum is exact, so the GEMM result
    equals the oracle's bit for bit at any k split."""
    print("case decode tile exact integers", flush=True)
    rng = np.random.default_rng(2)
    M, K, N = 37, 768, 264
    a = to_bf16_bits(rng.integers(-4, 5, (M, K)).astype(np.float32))
    b = to_bf16_bits(rng.integers(-4, 5, (K, N)).astype(np.float32))
    cf_ref, _ = orc.gemm(a, b)
    ad, pb = to_dev(gpu, a), llk.PackedWeights.from_host(b)
    for S in (1, 3):
        with _Tunable(llk, "decode_splits", S):
            assert llk.describe_launch("matmul", M, N, K)["kernel"] == "decode_tile"
            cf = from_dev(llk.matmul(ad, pb, out_dtype=gpu.float32))
        assert np.array_equal(cf, cf_ref), f"S={S}: not bit-exact"
