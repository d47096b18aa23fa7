"""CPU tests that pin the oracle (oracle/oracle.cpp) to the reference.

Every check compares the oracle against something other than a retyping of
its own formula: the reference's known-answer values, the reference's own
routines compiled from its sources (oracle/_ref), golden vectors produced
from the reference tests' own input streams, closed forms, exact integer
arithmetic, or brute force in fp64.
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest

from common import (bf16_bits_to_f32, normal_bf16, normal_bf16_np, parity, swiglu_inputs,
                    to_bf16_bits)

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def ref(orc):
    r = orc.ref()
    if r is None:
        pytest.skip("oracle/_ref not built (the reference tree is absent on this machine)")
    return r


# ---------------------------------------------------------------------------
# bf16 conversions
# ---------------------------------------------------------------------------

def test_bf16_rne_special_cases(orc):
    o = orc.orc()
    f = np.array([1.0, -1.0, 0.0, -0.0, 3.14, 65504.0, 1e-40, np.inf, -np.inf], np.float32)
    for v in f:
        h = o.orc_f32_to_bf16_rne(float(v))
        back = o.orc_bf16_to_f32(h)
        if np.isinf(v):
            assert back == v
        else:
            assert abs(back - v) <= abs(v) * 2.0 ** -8 + 1e-38
    # ties go to even: 1 + 2^-8 lies exactly between bf16 1.0 and 1.0078125
    tie_even = np.array([0x3F808000], np.uint32).view(np.float32)[0]
    assert o.orc_f32_to_bf16_rne(float(tie_even)) == 0x3F80
    tie_odd = np.array([0x3F818000], np.uint32).view(np.float32)[0]
    assert o.orc_f32_to_bf16_rne(float(tie_odd)) == 0x3F82
    nan = np.array([0x7FC00001], np.uint32).view(np.float32)[0]
    h = o.orc_f32_to_bf16_rne(float(nan))
    assert (h & 0x7F80) == 0x7F80 and (h & 0x7F) != 0


def test_bf16_rne_matches_independent_numpy(orc):
    """The C oracle and the numpy statement (tests/common.py) agree on 2^20
    random bit patterns, including NaN/Inf/denormals."""
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    assert np.array_equal(orc.f32_to_bf16(f), to_bf16_bits(f))


def test_bf16_roundtrip_reference_values(orc):
    """swiglu_reference.cpp:145-154 and vector_vs_scalar.cpp:122-139:
    bf16(f32(v)) stays within 1e-2 (relative 2e-2) of v."""
    for v in [-3.14, -1.0, 0.0, 1.0, 3.14, 42.0, -100.0, -10.0, -0.5, -0.01, 0.01, 0.5, 10.0, 100.0]:
        back = orc.orc().orc_bf16_to_f32(orc.orc().orc_f32_to_bf16_rne(v))
        assert abs(back - v) <= 1e-2 * max(1.0, abs(v))


def test_testhelper_conversion_matches_reference(orc, ref):
    """orc_f32_to_bf16_testhelper restates the reference tests' own helper
    (bits + 0x8000 + lsb); compared with that helper compiled from
    swiglu_reference.cpp on 2^18 random and all tie patterns."""
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, 1 << 18, dtype=np.uint64).astype(np.uint32)
    ties = (np.arange(1 << 12, dtype=np.uint32) << 20) | np.uint32(0x8000)
    allb = np.concatenate([bits, ties, ties | np.uint32(0x10000), ties - np.uint32(1)])
    o = orc.orc()
    for b in allb[::7]:
        f = float(np.array([b], np.uint32).view(np.float32)[0])
        assert o.orc_f32_to_bf16_testhelper(f) == ref.ref_f32_to_bf16(f)
    # ... and it is not round-to-nearest-even: ties with an even lsb round up.
    tie_even = float(np.array([0x3F808000], np.uint32).view(np.float32)[0])
    assert ref.ref_f32_to_bf16(tie_even) == 0x3F81
    assert o.orc_f32_to_bf16_rne(tie_even) == 0x3F80


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------

def test_known_values(orc):
    """swiglu_reference.cpp:156-175 (1, 2, 3 -> 5.2847825) and
    edge_cases.cpp:47-60 (2, .5, .3 -> 0.43863515), through both the fp64
    closed form and the fused bf16/fp32 path."""
    y = orc.swiglu_fp64(np.array([[1.0]]), np.array([[2.0]]), np.array([[3.0]]))
    assert abs(y[0, 0] - (2.0 / (1.0 + math.exp(-2.0))) * 3.0) < 1e-12
    assert abs(y[0, 0] - 5.284782468) < 1e-8
    y = orc.swiglu_fp64(np.array([[2.0]]), np.array([[0.5]]), np.array([[0.3]]))
    assert abs(y[0, 0] - (1.0 / (1.0 + math.exp(-1.0))) * 0.6) < 1e-12
    assert abs(y[0, 0] - 0.4386351472) < 1e-9
    # fused path: 1, 2, 3 are exact in bf16
    x = to_bf16_bits(np.array([[1.0]], np.float32))
    g = to_bf16_bits(np.array([[2.0]], np.float32))
    u = to_bf16_bits(np.array([[3.0]], np.float32))
    yf, yb = orc.swiglu(x, g, u)
    assert abs(yf[0, 0] - 5.284782468) < 1e-4 * 5.28  # swiglu_reference.cpp:173 bar (1e-4 abs)
    assert abs(yf[0, 0] - 5.284782468) < 1e-4


def test_edge_cases(orc):
    """edge_cases.cpp:62-150: K=1 uniform -> identical outputs; zeros -> 0;
    negative inputs finite; +-10 saturation."""
    x = to_bf16_bits(np.ones((3, 1), np.float32))
    wg = to_bf16_bits(np.full((1, 2), 0.5, np.float32))
    wu = to_bf16_bits(np.full((1, 2), 0.3, np.float32))
    yf, _ = orc.swiglu(x, wg, wu)
    assert np.all(yf == yf[0, 0])
    z = to_bf16_bits(np.zeros((2, 4), np.float32))
    zw = to_bf16_bits(np.zeros((4, 3), np.float32))
    yf, _ = orc.swiglu(z, zw, zw)
    assert np.all(yf == 0.0)
    x = to_bf16_bits(np.array([[-2.0, 3.0]], np.float32))
    wg = to_bf16_bits(np.array([[0.5, -1.0, 0.0, 2.0], [-3.0, 0.5, 1.0, 0.0]], np.float32))
    wu = to_bf16_bits(np.array([[1.0, 0.5, -0.5, 0.0], [2.0, -1.0, 0.0, -2.0]], np.float32))
    yf, _ = orc.swiglu(x, wg, wu)
    assert np.isfinite(yf).all()
    x = to_bf16_bits(np.array([[10.0, -10.0]], np.float32))
    eye = to_bf16_bits(np.eye(2, dtype=np.float32))
    yf, _ = orc.swiglu(x, eye, eye)
    assert yf[0, 0] > 90.0 and abs(yf[0, 1]) < 1.0
    # M = 0 is valid and empty (edge_cases.cpp:84-97)
    yf, yb = orc.swiglu(np.zeros((0, 4), np.uint16), zw[:4, :3], zw[:4, :3])
    assert yf.shape == (0, 3)


def test_fused_matches_reference_fp32_routine(orc, ref):
    """On bf16-valued inputs, the reference's fp32 routine
    (swiglu_reference.cpp:38-70, compiled from source) sums in the same
    sequential order; its products are exact, so outputs agree to an ulp or
    two (the reference divides by (1+e) where the fused path multiplies by
    1/(1+e))."""
    for (M, N, K) in [(1, 4, 2), (2, 3, 4), (4, 8, 16), (7, 33, 257)]:
        x, wg, wu = swiglu_inputs(M, K, N, seed=M * 100 + K)
        yf, _ = orc.swiglu(x, wg, wu)
        y_ref = np.empty((M, N), np.float32)
        ref.ref_swiglu_fp32(bf16_bits_to_f32(x), bf16_bits_to_f32(wg), bf16_bits_to_f32(wu),
                            y_ref, M, N, K)
        ulp = np.spacing(np.abs(y_ref).astype(np.float32))
        assert np.all(np.abs(yf - y_ref) <= 3 * ulp + 1e-30), (M, N, K)


def test_fp64_matches_reference_fp64_routines(orc, ref):
    """orc_swiglu_fp64 against swiglu_reference_fp64 and the edge-case copy
    (edge_cases.cpp:18-40), both compiled from the reference sources."""
    rng = np.random.default_rng(3)
    for (M, N, K) in [(1, 1, 1), (3, 5, 7), (16, 64, 100)]:
        x, wg, wu = (rng.standard_normal(s) for s in ((M, K), (K, N), (K, N)))
        y = orc.swiglu_fp64(x, wg, wu)
        y1 = np.empty((M, N))
        ref.ref_swiglu_fp64(x, wg, wu, y1, M, N, K)
        y2 = np.empty((M, N))
        ref.ref_edge_swiglu_fp64(x, wg, wu, y2, M, N, K)
        np.testing.assert_allclose(y, y1, rtol=1e-13, atol=1e-13)
        np.testing.assert_allclose(y, y2, rtol=1e-13, atol=1e-13)


def _golden():
    p = GOLDEN / "ref_vectors.npz"
    return np.load(p) if p.exists() else None


@pytest.mark.parametrize("shape", [(32, 128, 256), (16, 512, 512), (32, 256, 127), (4, 8, 3)])
def test_golden_reference_test_inputs(orc, shape):
    """Golden vectors: inputs reproduced from the reference tests' own streams
    (swiglu_vector_avx2.cpp:248-270), expected values from the reference's
    fp64 routine.  The oracle's fp32 (pre-truncf) result must match to fp32
    accumulation accuracy; its bf16 result is RNE of that."""
    g = _golden()
    assert g is not None, "tests/golden/ref_vectors.npz missing"
    M, N, K = shape
    t = f"vec_M{M}_N{N}_K{K}"
    x, wg, wu, y64 = g[t + "_x"], g[t + "_wg"], g[t + "_wu"], g[t + "_y_fp64"]
    yf, yb = orc.swiglu(x, wg, wu)
    p = parity(yf, y64)
    assert p["rel_l2"] < 2e-6 and p["max_abs_over_rms"] < 2e-5, p
    assert np.array_equal(yb, to_bf16_bits(yf))


@pytest.mark.parametrize("shape", [(1, 4, 2), (2, 3, 4), (4, 8, 16)])
def test_golden_reference_small_shapes(orc, shape):
    """swiglu_reference.cpp:109-141 shapes with its fp32 inputs (not bf16):
    the reference's fp32 and fp64 outputs bound each other as its test
    requires (max err < 1e-2), and the oracle's fp64 closed form reproduces
    the reference fp64 output."""
    g = _golden()
    M, N, K = shape
    t = f"ref_M{M}_N{N}_K{K}"
    x, wg, wu = g[t + "_x"], g[t + "_wg"], g[t + "_wu"]
    assert np.max(np.abs(g[t + "_y_fp32"] - g[t + "_y_fp64"])) < 1e-2
    y = orc.swiglu_fp64(x.astype(np.float64), wg.astype(np.float64), wu.astype(np.float64))
    np.testing.assert_allclose(y, g[t + "_y_fp64"], rtol=1e-13, atol=1e-13)


def test_golden_config1_samples(orc):
    """Config 1 (M=64, K=512, N=1376, seed 42): sampled oracle outputs are
    unchanged (regression pin) and the generator reproduces its inputs."""
    s = np.load(GOLDEN / "config1_samples.npz")
    x, wg, wu = swiglu_inputs(64, 512, 1376, seed=42)
    assert int(x.astype(np.uint64).sum()) == int(s["x_checksum"][0])
    assert int(wg.astype(np.uint64).sum() + wu.astype(np.uint64).sum()) == int(s["w_checksum"][0])
    yf, yb = orc.swiglu(x, wg, wu)
    idx = s["index"]
    assert np.array_equal(yb.ravel()[idx], s["y_bf16"])
    np.testing.assert_allclose(yf.ravel()[idx], s["y_fp32"], rtol=0, atol=0)


def test_exact_integer_swiglu(orc):
    """Integer-valued inputs: gate and up are exact in fp32 and equal the
    integer matmul, independent of summation order."""
    rng = np.random.default_rng(4)
    M, K, N = 9, 40, 17
    xi = rng.integers(-3, 4, (M, K))
    gi = rng.integers(-3, 4, (K, N))
    ui = rng.integers(-3, 4, (K, N))
    x, wg, wu = (to_bf16_bits(a.astype(np.float32)) for a in (xi, gi, ui))
    g, u = orc.swiglu_accumulators(x, wg, wu)
    assert np.array_equal(g, (xi @ gi).astype(np.float32))
    assert np.array_equal(u, (xi @ ui).astype(np.float32))
    yf, _ = orc.swiglu(x, wg, wu)
    gd, ud = (xi @ gi).astype(np.float64), (xi @ ui).astype(np.float64)
    np.testing.assert_allclose(yf, gd / (1 + np.exp(-gd)) * ud, rtol=1e-6, atol=1e-6)


def test_fused_vs_fp64_closed_form(orc):
    """The fused fp32 path is within fp32 accumulation error of the fp64
    closed form on bf16 inputs (a dropped term or transposed operand fails)."""
    x, wg, wu = swiglu_inputs(24, 300, 70, seed=8)
    yf, _ = orc.swiglu(x, wg, wu)
    y64 = orc.swiglu_fp64(*(bf16_bits_to_f32(a).astype(np.float64) for a in (x, wg, wu)))
    p = parity(yf, y64)
    assert p["rel_l2"] < 1e-6, p
    # a transposed weight (a plausible mistake) is far outside that bar
    y_bad = orc.swiglu_fp64(*(bf16_bits_to_f32(a).astype(np.float64)
                              for a in (x, wg[:, ::-1].copy(), wu)))
    assert parity(yf, y_bad)["rel_l2"] > 0.1


# ---------------------------------------------------------------------------
# GEMM (micro.mma contract)
# ---------------------------------------------------------------------------

def test_gemm_exact_integers(orc):
    rng = np.random.default_rng(5)
    ai = rng.integers(-8, 9, (13, 70))
    bi = rng.integers(-8, 9, (70, 29))
    cf, cb = orc.gemm(to_bf16_bits(ai.astype(np.float32)), to_bf16_bits(bi.astype(np.float32)))
    assert np.array_equal(cf, (ai @ bi).astype(np.float32))
    assert np.array_equal(cb, to_bf16_bits((ai @ bi).astype(np.float32)))


def test_gemm_vs_fp64_and_identity(orc):
    a = normal_bf16(6, 0, (33, 129), 0.1)
    b = normal_bf16(6, 1, (129, 65), 0.1)
    cf, _ = orc.gemm(a, b)
    c64 = orc.gemm_fp64(a, b)
    assert parity(cf, c64)["rel_l2"] < 1e-6
    eye = to_bf16_bits(np.eye(129, dtype=np.float32))
    ci, _ = orc.gemm(a, eye)
    assert np.array_equal(ci, bf16_bits_to_f32(a))


def test_gemm_init_closed_form(orc):
    """micro.mma's acc += lhs * rhs: with integer-valued operands and an
    integer initial accumulator every partial sum is exact in fp32, so the
    result equals C0 + A B computed in integers; a dropped or doubled C0 (or
    a transposed operand) fails it."""
    rng = np.random.default_rng(15)
    ai = rng.integers(-8, 9, (21, 75))
    bi = rng.integers(-8, 9, (75, 37))
    ci = rng.integers(-1000, 1001, (21, 37))
    a, b = to_bf16_bits(ai.astype(np.float32)), to_bf16_bits(bi.astype(np.float32))
    cf, cb = orc.gemm_init(a, b, ci.astype(np.float32))
    want = (ci + ai @ bi).astype(np.float32)
    assert np.array_equal(cf, want)
    assert np.array_equal(cb, to_bf16_bits(want))
    assert not np.array_equal(cf, (ai @ bi).astype(np.float32))
    f0, _ = orc.gemm_init(a, b, None)
    assert np.array_equal(f0, (ai @ bi).astype(np.float32))


@pytest.mark.parametrize("threads", [1, 4])
def test_gemm_avx2_equals_oracle(orc, threads):
    """The multithreaded AVX2 GEMM leg used for full-size checks: bit-equal
    to the scalar sequential-k oracle on ragged shapes, with and without an
    initial accumulator."""
    if not orc.orc().orc_cpu_has_avx2_fma():
        pytest.skip("host CPU lacks AVX2/FMA")
    for M, N, K in ((37, 67, 131), (64, 128, 64), (3, 5, 7), (70, 9, 200)):
        a = normal_bf16(16, 0, (M, K))
        b = normal_bf16(16, 1, (K, N), 1.0 / np.sqrt(K))
        c0 = bf16_bits_to_f32(normal_bf16(16, 2, (M, N)))
        for ci in (None, c0):
            f1, b1 = orc.gemm_init(a, b, ci)
            f2, b2 = orc.gemm_avx2(a, b, threads, ci)
            assert np.array_equal(f1.view(np.uint32), f2.view(np.uint32)), (M, N, K)
            assert np.array_equal(b1, b2)


def test_mlp_composition(orc):
    x, wg, wu = swiglu_inputs(5, 64, 96, seed=9)
    wd = normal_bf16(9, 3, (96, 64), 0.1)
    y, z = orc.mlp(x, wg, wu, wd)
    _, yb = orc.swiglu(x, wg, wu)
    _, zb = orc.gemm(yb, wd)
    assert np.array_equal(y, yb) and np.array_equal(z, zb)


# ---------------------------------------------------------------------------
# CPU baseline (AVX2 restatement of the reference tile structure)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("threads", [1, 3])
def test_avx2_baseline_equals_oracle(orc, threads):
    """BM32/BN64/BK64/VM4/VN8 tiles with ragged edges: sequential-k order per
    element, so identical bits to the scalar oracle."""
    if not orc.orc().orc_cpu_has_avx2_fma():
        pytest.skip("host CPU lacks AVX2/FMA")
    x, wg, wu = swiglu_inputs(37, 131, 67, seed=10)
    yb, yf = orc.swiglu_avx2(x, wg, wu, threads, grain=2, want_f32=True)
    yf_ref, yb_ref = orc.swiglu(x, wg, wu)
    assert np.array_equal(yb, yb_ref)
    assert np.array_equal(yf, yf_ref)


# ---------------------------------------------------------------------------
# Input generator
# ---------------------------------------------------------------------------

def test_generator_c_matches_numpy():
    """The library's C generator and the numpy statement agree (same libm on
    one host; tolerate one-ulp transcendental differences)."""
    a = normal_bf16_np(42, 1, (257, 63), 0.05)
    b = normal_bf16(42, 1, (257, 63), 0.05)
    d = np.abs(a.astype(np.int32) - b.astype(np.int32))
    assert d.max() <= 1 and np.mean(d == 0) > 0.999
    f = bf16_bits_to_f32(b).astype(np.float64) / 0.05
    assert abs(f.mean()) < 0.05 and abs(f.std() - 1.0) < 0.05
