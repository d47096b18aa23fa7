"""Mid M (65..256 rows) on the decode tile kernel's 128- and 256-row forms
(two and four 32-row MFMA tiles per wave; rows 129..256 with `midm_max_m`
raised to 256 from its default 128): SwiGLU (bf16 and fp32 results)
and the GEMM (bf16, fp16, fp32) against the CPU oracle at ragged M and N,
odd k-step counts, forced k splits, accumulate in the epilogue and in the
split reduce, exact integers bit for bit; and the routing around it
(`midm_max_m` at or below 64, or unaligned X, sends the same shapes to the
tile kernels, whose results agree to the bar)."""
from __future__ import annotations

import numpy as np
import pytest

from common import assert_parity, assert_parity_bf16, normal_bf16, swiglu_inputs, to_bf16_bits
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


@pytest.fixture(autouse=True)
def _midm_256(llk):
    """Every test here routes up to 256 rows to the mid-M forms."""
    with _Tunable(llk, "midm_max_m", 256):
        yield


def _swiglu(llk, gpu, x, pg, pu, dtype, x_stride=None):
    y = llk.fused_swiglu(to_dev(gpu, x, x_stride), pg, pu, out_dtype=dtype)
    gpu.cuda.synchronize()
    return from_dev(y)


# (M, K, N): first rows of the 128-row form (65), a partly filled last
# 32-row tile, exactly 128 and 256 rows, config 5's 255 (with a smaller K and
# N), ragged N (partial 64- and 128-column groups), one and odd 64-k steps.
SHAPES = [(65, 640, 392), (96, 1024, 1376), (128, 576, 600), (129, 64, 200),
          (200, 1984, 264), (255, 1280, 1000), (256, 512, 136)]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_swiglu_against_oracle(llk, gpu, orc, M, K, N):
    print(f"case mid-M swiglu M={M} K={K} N={N}", flush=True)
    assert llk.describe_launch("fused_swiglu", M, N, K)["kernel"] == "decode_tile"
    x, wg, wu = swiglu_inputs(M, K, N, seed=M + K)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    yf_ref, _ = orc.swiglu(x, wg, wu)
    yb = _swiglu(llk, gpu, x, pg, pu, gpu.bfloat16)
    yf = _swiglu(llk, gpu, x, pg, pu, gpu.float32)
    assert_parity_bf16(yb, yf_ref, f"swiglu M{M} bf16")
    assert_parity(yf, yf_ref, f"swiglu M{M} fp32")
    assert np.array_equal(yb, to_bf16_bits(yf)), "bf16 != RNE(fp32)"


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_gemm_against_oracle(llk, gpu, orc, M, K, N):
    print(f"case mid-M gemm M={M} K={K} N={N}", flush=True)
    a = normal_bf16(41, M, (M, K))
    b = normal_bf16(41, K, (K, N), 1.0 / np.sqrt(K))
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


@pytest.mark.parametrize("M,S", [(100, 2), (255, 3), (130, 7), (256, 5)])
def test_forced_splits(llk, gpu, orc, M, S):
    """k splits through the partial planes (256 rows at most) and the
    split-order reduce, both operations; S = 7 over 20 k-steps runs as 7
    splits of 3 (the last of 2)."""
    print(f"case mid-M splits M={M} S={S}", flush=True)
    K, N = 1280, 456
    kbs = -(-(K // 64) // S)
    x, wg, wu = swiglu_inputs(M, K, N, seed=S + M)
    yf_ref, _ = orc.swiglu(x, wg, wu)
    a = normal_bf16(42, S, (M, K))
    b = normal_bf16(42, M, (K, N), 1.0 / np.sqrt(K))
    cf_ref, _ = orc.gemm(a, b)
    with _Tunable(llk, "decode_splits", S):
        for op in ("fused_swiglu", "matmul"):
            plan = llk.describe_launch(op, M, N, K)
            assert plan["kernel"] == "decode_tile", plan
            assert plan["splits"] == -(-(K // 64) // kbs) and plan["launches"] == 2, plan
        pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
        yb = _swiglu(llk, gpu, x, pg, pu, gpu.bfloat16)
        yf = _swiglu(llk, gpu, x, pg, pu, gpu.float32)
        cf = from_dev(llk.matmul(to_dev(gpu, a), llk.PackedWeights.from_host(b),
                                 out_dtype=gpu.float32))
    assert_parity(yf, yf_ref, f"swiglu M{M} S{S}")
    assert_parity_bf16(yb, yf_ref, f"swiglu M{M} S{S} bf16")
    assert np.array_equal(yb, to_bf16_bits(yf)), "bf16 != RNE(fp32)"
    assert_parity(cf, cf_ref, f"gemm M{M} S{S}")


@pytest.mark.parametrize("S", [1, 4])
def test_gemm_accumulate(llk, gpu, orc, S):
    """C += A B at M = 190 (the 256-row form): in the epilogue (S = 1) and in
    the split reduce (S = 4); the result is the oracle's C0 + A B."""
    print(f"case mid-M gemm accumulate S={S}", flush=True)
    M, K, N = 190, 2048, 640
    a = normal_bf16(43, 0, (M, K))
    b = normal_bf16(43, 1, (K, N), 1.0 / np.sqrt(K))
    c0 = np.random.default_rng(S).standard_normal((M, N)).astype(np.float32)
    ref, _ = orc.gemm_avx2(a, b, 8, c_init=c0, want_bf16=False)
    with _Tunable(llk, "decode_splits", S):
        plan = llk.describe_launch("matmul", M, N, K, accumulate=True)
        assert plan["kernel"] == "decode_tile" and plan["splits"] == S, plan
        c = gpu.from_numpy(c0.copy()).cuda()
        llk.matmul(to_dev(gpu, a), llk.PackedWeights.from_host(b), out=c, accumulate=True)
        gpu.cuda.synchronize()
    assert_parity(c.cpu().numpy(), ref, f"accumulate S{S}")


@pytest.mark.parametrize("M", [97, 250])
def test_exact_integers(llk, gpu, orc, M):
    """Small-integer inputs: every partial sum is exact, so the GEMM result
    equals the oracle's bit for bit at any k split, on both mid-M forms."""
    print(f"case mid-M exact integers M={M}", flush=True)
    rng = np.random.default_rng(M)
    K, N = 768, 264
    a = to_bf16_bits(rng.integers(-4, 5, (M, K)).astype(np.float32))
    b = to_bf16_bits(rng.integers(-4, 5, (K, N)).astype(np.float32))
    cf_ref, _ = orc.gemm(a, b)
    ad, pb = to_dev(gpu, a), llk.PackedWeights.from_host(b)
    for S in (1, 3):
        with _Tunable(llk, "decode_splits", S):
            assert llk.describe_launch("matmul", M, N, K)["kernel"] == "decode_tile"
            cf = from_dev(llk.matmul(ad, pb, out_dtype=gpu.float32))
        assert np.array_equal(cf, cf_ref), f"M={M} S={S}: not bit-exact"


def test_routing_and_agreement_with_tile_kernels(llk, gpu, orc):
    """With `midm_max_m` at 64 the same mid-M call runs on the tile kernels;
    X rows that are not 16-byte aligned always do; both agree with the decode
    tile kernel's result and the oracle to the bar."""
    print("case mid-M routing", flush=True)
    M, K, N = 180, 1024, 520
    x, wg, wu = swiglu_inputs(M, K, N, seed=11)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    yf_ref, _ = orc.swiglu(x, wg, wu)
    assert llk.describe_launch("fused_swiglu", M, N, K)["kernel"] == "decode_tile"
    yf_mid = _swiglu(llk, gpu, x, pg, pu, gpu.float32)
    assert_parity(yf_mid, yf_ref, "mid-M")
    with _Tunable(llk, "midm_max_m", 64):
        assert llk.describe_launch("fused_swiglu", M, N, K, out_f32=True)["kernel"] == "tile"
        yf_tile = _swiglu(llk, gpu, x, pg, pu, gpu.float32)
    assert_parity(yf_tile, yf_ref, "tile")
    assert_parity(yf_tile, yf_mid, "tile vs mid-M")
    assert llk.describe_launch("fused_swiglu", M, N, K, x_aligned=False,
                               out_f32=True)["kernel"] == "tile"
    yf_un = _swiglu(llk, gpu, x, pg, pu, gpu.float32, x_stride=K + 3)
    assert_parity(yf_un, yf_ref, "unaligned X on the tile kernel")


def _random_cases(n=16, seed=2027):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        out.append(dict(op=str(rng.choice(["swiglu", "gemm"])), M=int(rng.integers(65, 257)),
                        K=64 * int(rng.integers(1, 33)), N=int(rng.integers(1, 1300)),
                        pad=8 * int(rng.integers(0, 5)), splits=int(rng.choice([0, 0, 2, 3, 7])),
                        seed=int(rng.integers(0, 1 << 30))))
    return out


@pytest.mark.parametrize("c", _random_cases(), ids=lambda c: f"{c['op']}-M{c['M']}-K{c['K']}-N{c['N']}")
def test_random_mid_m(llk, gpu, orc, c):
    """Seeded random mid-M shapes (K a multiple of 64, X strides a multiple
    of 8 elements) on the decode tile kernel, automatic or forced k splits,
    against the oracle; the bf16 result is the rounding of the fp32 one."""
    print(f"case mid-M random {c}", flush=True)
    M, K, N = c["M"], c["K"], c["N"]
    s = 1.0 / np.sqrt(K)
    x = normal_bf16(c["seed"], 0, (M, K))
    w0 = normal_bf16(c["seed"], 1, (K, N), s)
    w1 = normal_bf16(c["seed"], 2, (K, N), s)
    xd = to_dev(gpu, x, K + c["pad"] if c["pad"] else None)
    p0, p1 = llk.PackedWeights.from_host(w0), llk.PackedWeights.from_host(w1)
    with _Tunable(llk, "decode_splits", c["splits"]):
        op = "fused_swiglu" if c["op"] == "swiglu" else "matmul"
        assert llk.describe_launch(op, M, N, K)["kernel"] == "decode_tile"
        if c["op"] == "swiglu":
            yf = from_dev(llk.fused_swiglu(xd, p0, p1, out_dtype=gpu.float32))
            yb = from_dev(llk.fused_swiglu(xd, p0, p1, out_dtype=gpu.bfloat16))
            ref, _ = orc.swiglu(x, w0, w1)
        else:
            yf = from_dev(llk.matmul(xd, p0, out_dtype=gpu.float32))
            yb = from_dev(llk.matmul(xd, p0, out_dtype=gpu.bfloat16))
            ref, _ = orc.gemm(x, w0)
    assert_parity(yf, ref, f"mid-M random {c}")
    assert np.array_equal(yb, to_bf16_bits(yf))
