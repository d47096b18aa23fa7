"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Bar (north star): rel-L2 <= 1e-3 and max-abs <= 2e-2 * RMS(output) on
identical seeded inputs; bf16 outputs are compared bf16 against the
oracle's own RNE-rounded bf16, fp32 outputs against the oracle's pre-truncf
fp32.  Integer-valued inputs whose sums are exact in fp32 must match bit for
bit.
"""
from __future__ import annotations

import numpy as np
import pytest

from common import (assert_parity, assert_parity_bf16, bf16_bits_to_f32, normal_bf16, outliers,
                    parity, swiglu_inputs, to_bf16_bits)
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu

# [M, N, K] shapes of the reference's own SwiGLU tests:
# swiglu_reference.cpp:109-113, swiglu_scalar.cpp:355, swiglu_vector_avx2.cpp:214-218,
# vector_vs_scalar.cpp:77-81.
REF_SHAPES = [(1, 4, 2), (2, 3, 4), (4, 8, 16), (4, 8, 3), (32, 128, 256), (16, 512, 512),
              (32, 256, 127), (1, 128, 256), (64, 256, 128)]


def _run_swiglu(llk, torch, x, wg, wu, out_dtype, x_stride=None, y_stride=None):
    M, K = x.shape
    N = wg.shape[1]
    xd = to_dev(torch, x, x_stride)
    pg = llk.PackedWeights.from_host(wg)
    pu = llk.PackedWeights.from_host(wu)
    if y_stride is None:
        y = torch.empty((M, N), dtype=out_dtype, device="cuda")
    else:
        y = torch.zeros((M, y_stride), dtype=out_dtype, device="cuda")[:, :N]
    llk.fused_swiglu(xd, pg, pu, out=y)
    torch.cuda.synchronize()
    out = from_dev(y)
    pg.free()
    pu.free()
    return out


def _check_swiglu(llk, gpu, orc, x, wg, wu, what, **kw):
    yf_ref, _ = orc.swiglu(x, wg, wu)
    yb = _run_swiglu(llk, gpu, x, wg, wu, gpu.bfloat16, **kw)
    yf = _run_swiglu(llk, gpu, x, wg, wu, gpu.float32, **kw)
    p1 = assert_parity_bf16(yb, yf_ref, what + " bf16")
    p2 = assert_parity(yf, yf_ref, what + " fp32")
    # the bf16 result is exactly RNE of the same kernel's fp32 result
    assert np.array_equal(yb, to_bf16_bits(yf)), what + ": bf16 != RNE(fp32)"
    return p1, p2


@pytest.mark.parametrize("M,N,K", REF_SHAPES)
def test_swiglu_reference_shapes(llk, gpu, orc, M, N, K):
    print(f"case swiglu ref-shape M={M} N={N} K={K}", flush=True)
    x, wg, wu = swiglu_inputs(M, K, N, seed=42)
    _check_swiglu(llk, gpu, orc, x, wg, wu, f"M{M}N{N}K{K}")


@pytest.mark.parametrize("M", [1, 8, 16, 17, 33, 64, 65, 255, 256, 257, 300])
def test_swiglu_m_sweep(llk, gpu, orc, M):
    """Covers the decode kernels (M <= 64), the decode tile kernel's 128-row
    form (M = 65) and the prefill tile kernels (M > 128), including ragged M
    edge tiles."""
    print(f"case swiglu m-sweep M={M} K=576 N=392", flush=True)
    x, wg, wu = swiglu_inputs(M, 576, 392, seed=7)
    _check_swiglu(llk, gpu, orc, x, wg, wu, f"M{M}")


def test_swiglu_config1(llk, gpu, orc):
    """M=64, K=512, N=1376, fp32 output (and bf16)."""
    print("case swiglu config1", flush=True)
    x, wg, wu = swiglu_inputs(64, 512, 1376, seed=42)
    _check_swiglu(llk, gpu, orc, x, wg, wu, "config1")


def test_swiglu_config1_prefill_path(llk, gpu, orc):
    """Config 1 forced through the prefill tile kernel."""
    print("case swiglu config1 prefill path", flush=True)
    old = llk.get_tunable("decode_max_m")
    llk.set_tunable("decode_max_m", 0)
    try:
        x, wg, wu = swiglu_inputs(64, 512, 1376, seed=42)
        _check_swiglu(llk, gpu, orc, x, wg, wu, "config1-prefill")
    finally:
        llk.set_tunable("decode_max_m", old)


@pytest.mark.parametrize("case", ["k_ragged", "odd_stride", "misaligned_base", "aligned"])
def test_tile_x_layouts(llk, gpu, orc, case):
    """The tile kernel reads X straight into LDS when rows are 16-byte
    aligned and K % 64 == 0; otherwise X is first copied into a padded
    buffer.  Both routes, on ragged M and N edge tiles, for SwiGLU and GEMM."""
    print(f"case tile x layout {case}", flush=True)
    M, N = 300, 392
    K = {"k_ragged": 200, "odd_stride": 256, "misaligned_base": 256, "aligned": 320}[case]
    x, wg, wu = swiglu_inputs(M, K, N, seed=len(case))
    if case == "odd_stride":
        xd = to_dev(gpu, x, stride0=K + 3)
    elif case == "misaligned_base":
        big = np.zeros((M, K + 8), np.uint16)
        big[:, 1:K + 1] = x
        xd = to_dev(gpu, big)[:, 1:K + 1]
    else:
        xd = to_dev(gpu, x)
    yf_ref, _ = orc.swiglu(x, wg, wu)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    yf = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.float32))
    assert_parity(yf, yf_ref, f"swiglu {case}")
    s = 1.0 / np.sqrt(K)
    b = normal_bf16(9, 1, (K, N), s)
    cf_ref, _ = orc.gemm(x, b)
    pb = llk.PackedWeights.from_host(b)
    cf = from_dev(llk.matmul(xd, pb, out_dtype=gpu.float32))
    assert_parity(cf, cf_ref, f"gemm {case}")


@pytest.mark.parametrize("M", [1, 17, 40, 64])
def test_gemm_small_m(llk, gpu, orc, M):
    """Small-M GEMM (the down projection of decode-sized MLP blocks) runs on
    the bandwidth kernel, with and without the cross-workgroup k split."""
    print(f"case gemm small M={M}", flush=True)
    K, N = 1536, 640
    s = 1.0 / np.sqrt(K)
    a = normal_bf16(4, 0, (M, K), s)
    b = normal_bf16(4, 1, (K, N), s)
    cf_ref, _ = orc.gemm(a, b)
    pb = llk.PackedWeights.from_host(b)
    ad = to_dev(gpu, a)
    for splits in (0, 1, 3):
        old = llk.get_tunable("decode_splits")
        llk.set_tunable("decode_splits", splits)
        try:
            cf = from_dev(llk.matmul(ad, pb, out_dtype=gpu.float32))
            cb = from_dev(llk.matmul(ad, pb, out_dtype=gpu.bfloat16))
        finally:
            llk.set_tunable("decode_splits", old)
        assert_parity(cf, cf_ref, f"gemm small M={M} S={splits}")
        assert np.array_equal(cb, to_bf16_bits(cf)), "bf16 != RNE(fp32)"


@pytest.mark.parametrize("splits", [1, 2, 3, 16])
def test_swiglu_decode_splits(llk, gpu, orc, splits):
    print(f"case swiglu decode splits={splits}", flush=True)
    old = llk.get_tunable("decode_splits")
    llk.set_tunable("decode_splits", splits)
    try:
        x, wg, wu = swiglu_inputs(8, 1024, 640, seed=3)
        _check_swiglu(llk, gpu, orc, x, wg, wu, f"S{splits}")
    finally:
        llk.set_tunable("decode_splits", old)


def test_swiglu_decode_workspace_reuse(llk, gpu, orc):
    """Regression: a large split-K decode call followed by smaller ones with a
    different partial-sum layout in the shared workspace must not see stale
    workspace contents."""
    print("case swiglu decode workspace reuse", flush=True)
    for (M, K, N, S) in [(64, 4096, 1376, 8), (8, 1024, 640, 2), (1, 256, 128, 2),
                         (33, 2048, 2000, 5), (3, 512, 96, 3)]:
        old = llk.get_tunable("decode_splits")
        llk.set_tunable("decode_splits", S)
        try:
            x, wg, wu = swiglu_inputs(M, K, N, seed=M + K)
            _check_swiglu(llk, gpu, orc, x, wg, wu, f"reuse M{M}K{K}N{N}S{S}")
        finally:
            llk.set_tunable("decode_splits", old)


class _Tunable:
    """Sets a dispatch knob for the duration of a with-block."""

    def __init__(self, llk, name, value):
        self.llk, self.name, self.value = llk, name, value

    def __enter__(self):
        self.old = self.llk.get_tunable(self.name)
        self.llk.set_tunable(self.name, self.value)

    def __exit__(self, *exc):
        self.llk.set_tunable(self.name, self.old)


@pytest.mark.parametrize("G", [1, 2, 4])
@pytest.mark.parametrize("M,S", [(1, 1), (8, 3), (40, 1), (64, 2)])
def test_decode_group_width(llk, gpu, orc, G, M, S):
    """Small-M kernel with 1, 2 or 4 column groups per workgroup, with and
    without the cross-workgroup k split; SwiGLU and GEMM, ragged N."""
    print(f"case decode G={G} M={M} S={S}", flush=True)
    K, N = 1280, 600
    x, wg, wu = swiglu_inputs(M, K, N, seed=G * 100 + M)
    with _Tunable(llk, "decode_group_width", G), _Tunable(llk, "decode_splits", S):
        _check_swiglu(llk, gpu, orc, x, wg, wu, f"decode G={G} M={M} S={S}")
        cf_ref, _ = orc.gemm(x, wg)
        cf = from_dev(llk.matmul(to_dev(gpu, x), llk.PackedWeights.from_host(wg),
                                 out_dtype=gpu.float32))
    assert_parity(cf, cf_ref, f"decode gemm G={G} M={M} S={S}")


# (M, K, N, forced splits): aligned and padded X (K % 64 != 0), ragged M and
# N, splits that leave a short last split (K=1000: 16 k-steps over 3 -> 6,6,4)
# and split counts that collapse (16 steps over 5 -> 4 splits of 4).
TILE_SPLIT_CASES = [(300, 1024, 700, 2), (300, 1000, 700, 3), (65, 4096, 384, 5),
                    (513, 640, 130, 7), (256, 128, 256, 2)]


@pytest.mark.parametrize("M,K,N,S", TILE_SPLIT_CASES)
def test_swiglu_tile_splits(llk, gpu, orc, M, K, N, S):
    """Prefill SwiGLU with K split across workgroups (gate/up partials, then
    the reduce kernel applies the epilogue)."""
    print(f"case swiglu tile splits M={M} K={K} N={N} S={S}", flush=True)
    x, wg, wu = swiglu_inputs(M, K, N, seed=M + S)
    with _Tunable(llk, "tile_splits", S):
        _check_swiglu(llk, gpu, orc, x, wg, wu, f"tile split S={S}")


@pytest.mark.parametrize("M,K,N,S", TILE_SPLIT_CASES)
def test_gemm_tile_splits(llk, gpu, orc, M, K, N, S):
    print(f"case gemm tile splits M={M} K={K} N={N} S={S}", flush=True)
    s = 1.0 / np.sqrt(K)
    a = normal_bf16(M + S, 0, (M, K), s)
    b = normal_bf16(M + S, 1, (K, N), s)
    cf_ref, _ = orc.gemm(a, b)
    pb = llk.PackedWeights.from_host(b)
    ad = to_dev(gpu, a)
    with _Tunable(llk, "tile_splits", S):
        cf = from_dev(llk.matmul(ad, pb, out_dtype=gpu.float32))
        cb = from_dev(llk.matmul(ad, pb, out_dtype=gpu.bfloat16))
    assert_parity(cf, cf_ref, f"gemm tile split S={S}")
    assert_parity_bf16(cb, cf_ref, f"gemm tile split S={S} bf16")
    assert np.array_equal(cb, to_bf16_bits(cf)), "bf16 != RNE(fp32)"


@pytest.mark.parametrize("K", [1, 32, 64, 96, 192, 320])
def test_tile_short_k_pipeline(llk, gpu, orc, K):
    """The tile kernel's prologue fills three 64-k X slots and four 32-k
    weight stages before the loop; with one to five k-blocks most of those
    loads fall past the end and are clamped.  K below one block (1, 32),
    exactly one (64), one and a half (96, padded), and odd block counts
    (3, 5), each with and without a k split, on two M tiles and a ragged N."""
    print(f"case tile short k K={K}", flush=True)
    M, N = 260, 200
    x, wg, wu = swiglu_inputs(M, K, N, seed=K)
    s = 1.0 / np.sqrt(K)
    b = normal_bf16(K, 1, (K, N), s)
    cf_ref, _ = orc.gemm(x, b)
    pb = llk.PackedWeights.from_host(b)
    for S in (1, 3):
        with _Tunable(llk, "decode_max_m", 0), _Tunable(llk, "tile_splits", S):
            _check_swiglu(llk, gpu, orc, x, wg, wu, f"tile short k K={K} S={S}")
            cf = from_dev(llk.matmul(to_dev(gpu, x), pb, out_dtype=gpu.float32))
        assert_parity(cf, cf_ref, f"gemm short k K={K} S={S}")


@pytest.mark.parametrize("M,K,N", [(300, 1024, 600), (300, 1000, 600), (300, 640, 1100)])
def test_tile_tail_split(llk, gpu, orc, M, K, N):
    """Tail split: with 4 workgroups per wave the leading n-tile columns run
    as one unsplit launch and the remaining (ragged) columns as a k-split
    launch into the same Y -- aligned and padded X, SwiGLU and GEMM."""
    print(f"case tile tail split M={M} K={K} N={N}", flush=True)
    x, wg, wu = swiglu_inputs(M, K, N, seed=M + N)
    s = 1.0 / np.sqrt(K)
    b = normal_bf16(N, 1, (K, N), s)
    cf_ref, _ = orc.gemm(x, b)
    pb = llk.PackedWeights.from_host(b)
    with _Tunable(llk, "tile_wgs_per_wave", 4):
        for op in ("fused_swiglu", "matmul"):
            plan = llk.describe_launch(op, M, N, K, x_aligned=K % 64 == 0)
            assert plan["head_blocks_n"] > 0 and plan["splits"] > 1, plan
        _check_swiglu(llk, gpu, orc, x, wg, wu, f"tail split M={M} K={K} N={N}")
        xd = to_dev(gpu, x)
        cf = from_dev(llk.matmul(xd, pb, out_dtype=gpu.float32))
        cb = from_dev(llk.matmul(xd, pb, out_dtype=gpu.bfloat16))
    assert_parity(cf, cf_ref, f"gemm tail split M={M} K={K} N={N}")
    assert np.array_equal(cb, to_bf16_bits(cf)), "bf16 != RNE(fp32)"


def test_tile_splits_exact_and_reuse(llk, gpu, orc):
    """Integer inputs make every partial sum exact, so any k split must give
    the oracle's gate/up bit for bit: GEMM fp32 output equal, SwiGLU within
    one bf16 ulp (expf only).  Calls alternate split counts and shapes so a
    stale partial plane in the shared workspace would show."""
    print("case tile splits exact + workspace reuse", flush=True)
    rng = np.random.default_rng(7)
    for (M, K, N, S) in [(200, 1024, 300, 4), (100, 192, 160, 3), (257, 512, 96, 2),
                         (100, 192, 160, 1), (200, 1024, 300, 8)]:
        a = to_bf16_bits(rng.integers(-4, 5, (M, K)).astype(np.float32))
        b = to_bf16_bits(rng.integers(-4, 5, (K, N)).astype(np.float32))
        wu = to_bf16_bits(rng.integers(-2, 3, (K, N)).astype(np.float32) * 0.125)
        with _Tunable(llk, "tile_splits", S):
            cf = from_dev(llk.matmul(to_dev(gpu, a), llk.PackedWeights.from_host(b),
                                     out_dtype=gpu.float32))
            wg = to_bf16_bits(bf16_bits_to_f32(b) * np.float32(0.0625))
            yb = _run_swiglu(llk, gpu, a, wg, wu, gpu.bfloat16)
        cf_ref, _ = orc.gemm(a, b)
        assert np.array_equal(cf, cf_ref), f"gemm M={M} K={K} N={N} S={S}"
        _, yb_ref = orc.swiglu(a, wg, wu)
        d = np.abs(yb.astype(np.int32) - yb_ref.astype(np.int32))
        assert d.max() <= 1 and np.mean(d == 0) > 0.99, f"swiglu M={M} K={K} N={N} S={S}"


def test_swiglu_strided(llk, gpu, orc):
    print("case swiglu strided", flush=True)
    x, wg, wu = swiglu_inputs(130, 200, 136, seed=11)
    _check_swiglu(llk, gpu, orc, x, wg, wu, "strided", x_stride=216, y_stride=140)
    x, wg, wu = swiglu_inputs(9, 200, 136, seed=12)
    _check_swiglu(llk, gpu, orc, x, wg, wu, "strided-decode", x_stride=216, y_stride=141)


def test_swiglu_outliers(llk, gpu, orc):
    """1% of X scaled x20 (config 5's input distribution)."""
    print("case swiglu outliers", flush=True)
    x, wg, wu = swiglu_inputs(96, 640, 384, seed=5)
    x = outliers(x, seed=5)
    _check_swiglu(llk, gpu, orc, x, wg, wu, "outliers")


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_y_misaligned_base(llk, gpu, orc, dtype):
    """Outputs written to a view that starts one element into its buffer (no
    16-byte row alignment, 2- or 4-byte aligned) on ragged tiles: the
    epilogue's element-wise stores, for SwiGLU (bf16, f32) and GEMM (every
    result type); the columns either side of the view stay untouched."""
    print(f"case y misaligned base {dtype}", flush=True)
    M, K, N = 300, 256, 200
    x, wg, wu = swiglu_inputs(M, K, N, seed=77)
    tdt = {"bf16": gpu.bfloat16, "f16": gpu.float16, "f32": gpu.float32}[dtype]
    xd = to_dev(gpu, x)

    def run(fn, *w):
        buf = gpu.full((M, N + 8), 7.0, dtype=tdt, device="cuda")
        y = buf[:, 1:N + 1]
        fn(xd, *w, out=y)
        gpu.cuda.synchronize()
        host = from_dev(buf)
        edge = np.concatenate([host[:, :1], host[:, N + 1:]], axis=1)
        as_f32 = edge.astype(np.float32) if dtype != "bf16" else bf16_bits_to_f32(edge)
        assert np.all(as_f32 == 7.0), "wrote outside the view"
        return host[:, 1:N + 1]

    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    yf_ref, _ = orc.swiglu(x, wg, wu)
    if dtype == "f32":
        assert_parity(run(llk.fused_swiglu, pg, pu), yf_ref, "swiglu misaligned f32")
    elif dtype == "bf16":
        assert_parity_bf16(run(llk.fused_swiglu, pg, pu), yf_ref, "swiglu misaligned bf16")
    b = normal_bf16(9, 1, (K, N), 1.0 / np.sqrt(K))
    cf_ref, _ = orc.gemm(x, b)
    pb = llk.PackedWeights.from_host(b)
    c = run(llk.matmul, pb)
    if dtype == "f32":
        assert_parity(c, cf_ref, "gemm misaligned f32")
    elif dtype == "bf16":
        assert_parity_bf16(c, cf_ref, "gemm misaligned bf16")
    else:
        # fp16 result = RNE of the kernel's fp32 sum (the same kernel, aligned)
        cf = from_dev(llk.matmul(xd, pb, out_dtype=gpu.float32))
        assert_parity(cf, cf_ref, "gemm misaligned f16 (fp32 run)")
        assert np.array_equal(c.view(np.uint16), cf.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("M", [3, 100])
def test_swiglu_exact_integers(llk, gpu, orc, M):
    """Small-integer inputs: every product and partial sum is exact in fp32,
    so gate/up are exact whatever the summation order and the bf16 result
    must equal the oracle's bit for bit."""
    print(f"case swiglu exact M={M}", flush=True)
    rng = np.random.default_rng(1)
    K, N = 192, 160
    x = to_bf16_bits(rng.integers(-3, 4, (M, K)).astype(np.float32))
    wg = to_bf16_bits(rng.integers(-2, 3, (K, N)).astype(np.float32) * 0.0625)
    wu = to_bf16_bits(rng.integers(-2, 3, (K, N)).astype(np.float32) * 0.125)
    yb = _run_swiglu(llk, gpu, x, wg, wu, gpu.bfloat16)
    _, yb_ref = orc.swiglu(x, wg, wu)
    # gate/up exact; the epilogue differs from the CPU's only by the expf
    # implementation, so allow 1 bf16 ulp there.
    d = np.abs(yb.astype(np.int32) - yb_ref.astype(np.int32))
    assert d.max() <= 1, d.max()
    assert np.mean(d == 0) > 0.99


@pytest.mark.parametrize("M", [1, 65])
def test_swiglu_epilogue_accuracy(llk, gpu, M):
    """The SiLU(g) * u epilogue alone (K = 1, X = 1, Wg = g, Wu = 1, so gate
    and up are exact) on every finite bf16 g with |g| <= 80, on the small-M
    (M = 1) and tile (M = 65) kernels: within 4 ulp of the correctly rounded
    g / (1 + exp(-g)) (fp64 closed form; expf plus an IEEE divide is within
    3 ulp on the same set)."""
    print(f"case swiglu epilogue accuracy M={M}", flush=True)
    bits = np.arange(1 << 16, dtype=np.uint32)
    gv = (bits << 16).view(np.float32)
    gv = np.unique(gv[np.isfinite(gv) & (np.abs(gv) <= 80.0)])
    N = gv.size
    x = to_bf16_bits(np.ones((M, 1), np.float32))
    wg = to_bf16_bits(gv.reshape(1, N))
    wu = to_bf16_bits(np.ones((1, N), np.float32))
    yf = _run_swiglu(llk, gpu, x, wg, wu, gpu.float32)
    g = gv.astype(np.float64)
    ref = (g / (1.0 + np.exp(-g))).astype(np.float32)
    def ordered(a):  # float32 -> integers in value order (+0 and -0 both 0)
        i = a.view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    for row in (0, M - 1):
        ulp = np.abs(ordered(yf[row]) - ordered(ref))
        assert ulp.max() <= 4, (ulp.max(), gv[ulp.argmax()])


def test_swiglu_known_values(llk, gpu):
    """swiglu_reference.cpp:156-175 (X=1, Wg=2, Wu=3 -> 5.2847825) and
    edge_cases.cpp:47-60 (x=2, wg=.5, wu=.3 -> 0.43863515)."""
    print("case swiglu known values", flush=True)
    for xv, gv, uv, want in [(1.0, 2.0, 3.0, 5.284782468), (2.0, 0.5, 0.3, 0.4386351472)]:
        x = to_bf16_bits(np.array([[xv]], np.float32))
        wg = to_bf16_bits(np.array([[gv]], np.float32))
        wu = to_bf16_bits(np.array([[uv]], np.float32))
        yf = _run_swiglu(llk, gpu, x, wg, wu, gpu.float32)
        # inputs are bf16-rounded (0.3 -> 0.30078125), so compare with the
        # closed form on the rounded values, and the named value loosely.
        xr, gr, ur = (float(bf16_bits_to_f32(a)[0, 0]) for a in (x, wg, wu))
        g, u = xr * gr, xr * ur
        exact = g / (1 + np.exp(-g)) * u
        assert abs(yf[0, 0] - exact) <= 2e-6 * abs(exact)
        assert abs(yf[0, 0] - want) <= 3e-3 * abs(want)


def test_swiglu_all_zero_and_k1_uniform(llk, gpu):
    """edge_cases.cpp:62-82 (K=1 uniform -> all equal) and :139-150 (zeros)."""
    print("case swiglu zeros / K=1", flush=True)
    x = to_bf16_bits(np.zeros((2, 4), np.float32))
    w = to_bf16_bits(np.zeros((4, 3), np.float32))
    y = _run_swiglu(llk, gpu, x, w, w, gpu.float32)
    assert np.all(y == 0.0)
    x = to_bf16_bits(np.ones((3, 1), np.float32))
    wg = to_bf16_bits(np.full((1, 2), 0.5, np.float32))
    wu = to_bf16_bits(np.full((1, 2), 0.3, np.float32))
    y = _run_swiglu(llk, gpu, x, wg, wu, gpu.float32)
    assert np.all(y == y[0, 0]) and np.isfinite(y).all()


def test_swiglu_saturation(llk, gpu, orc):
    """edge_cases.cpp:116-137: +-10 inputs, identity-like weights."""
    print("case swiglu saturation", flush=True)
    x = to_bf16_bits(np.array([[10.0, -10.0]], np.float32))
    w = to_bf16_bits(np.eye(2, dtype=np.float32))
    y = _run_swiglu(llk, gpu, x, w, w, gpu.float32)
    yf_ref, _ = orc.swiglu(x, w, w)
    assert y[0, 0] > 90.0 and abs(y[0, 1]) < 1.0
    np.testing.assert_allclose(y, yf_ref, rtol=1e-6, atol=1e-9)


def test_swiglu_m0(llk, gpu):
    """edge_cases.cpp:84-97: M=0 is valid and produces an empty output."""
    print("case swiglu M=0", flush=True)
    wg = normal_bf16(1, 1, (4, 8))
    pg = llk.PackedWeights.from_host(wg)
    x = gpu.empty((0, 4), dtype=gpu.bfloat16, device="cuda")
    y = llk.fused_swiglu(x, pg, pg)
    assert y.shape == (0, 8)


def test_empty_weights_both_pack_paths(llk, gpu):
    """An empty weight matrix (N = 0) packs on the host and on the device
    into usable handles: SwiGLU and GEMM give empty outputs."""
    print("case empty weights", flush=True)
    x = gpu.ones((3, 4), dtype=gpu.bfloat16, device="cuda")
    w_host = normal_bf16(1, 1, (4, 0))
    for pw in (llk.PackedWeights.from_host(w_host),
               llk.PackedWeights.from_device(gpu.empty((4, 0), dtype=gpu.bfloat16, device="cuda"))):
        assert pw.N == 0 and pw.K == 4
        assert llk.fused_swiglu(x, pw, pw).shape == (3, 0)
        assert llk.matmul(x, pw).shape == (3, 0)


def test_swiglu_deterministic_and_row_permutation(llk, gpu):
    """Size-independent properties: two runs are bit-identical, and
    permuting the rows of X permutes the rows of Y bit for bit (every row is
    computed with the same arithmetic)."""
    print("case swiglu determinism/permutation", flush=True)
    M, K, N = 512, 1024, 768
    x, wg, wu = swiglu_inputs(M, K, N, seed=9)
    y1 = _run_swiglu(llk, gpu, x, wg, wu, gpu.bfloat16)
    y2 = _run_swiglu(llk, gpu, x, wg, wu, gpu.bfloat16)
    assert np.array_equal(y1, y2)
    perm = np.random.default_rng(0).permutation(M)
    y3 = _run_swiglu(llk, gpu, x[perm], wg, wu, gpu.bfloat16)
    assert np.array_equal(y3, y1[perm])


@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (300, 200, 320), (256, 512, 128),
                                   (1, 128, 64), (77, 300, 129), (513, 257, 96)])
def test_gemm(llk, gpu, orc, M, N, K):
    print(f"case gemm M={M} N={N} K={K}", flush=True)
    s = 1.0 / np.sqrt(K)
    a = normal_bf16(42, 0, (M, K), s)
    b = normal_bf16(42, 1, (K, N), s)
    cf_ref, cb_ref = orc.gemm(a, b)
    pb = llk.PackedWeights.from_host(b)
    ad = to_dev(gpu, a)
    cf = from_dev(llk.matmul(ad, pb, out_dtype=gpu.float32))
    cb = from_dev(llk.matmul(ad, pb, out_dtype=gpu.bfloat16))
    assert_parity(cf, cf_ref, "gemm fp32")
    assert_parity_bf16(cb, cf_ref, "gemm bf16")
    assert np.array_equal(cb, to_bf16_bits(cf)), "gemm bf16 != RNE(fp32)"


def test_gemm_exact_integers(llk, gpu, orc):
    print("case gemm exact", flush=True)
    rng = np.random.default_rng(2)
    M, N, K = 200, 300, 256
    a = to_bf16_bits(rng.integers(-4, 5, (M, K)).astype(np.float32))
    b = to_bf16_bits(rng.integers(-4, 5, (K, N)).astype(np.float32))
    cf_ref, _ = orc.gemm(a, b)
    pb = llk.PackedWeights.from_host(b)
    cf = from_dev(llk.matmul(to_dev(gpu, a), pb, out_dtype=gpu.float32))
    assert np.array_equal(cf, cf_ref)


def test_gemm_identity(llk, gpu):
    """A * I = A exactly (closed form)."""
    print("case gemm identity", flush=True)
    a = normal_bf16(3, 0, (70, 96))
    eye = to_bf16_bits(np.eye(96, dtype=np.float32))
    pb = llk.PackedWeights.from_host(eye)
    cf = from_dev(llk.matmul(to_dev(gpu, a), pb, out_dtype=gpu.float32))
    assert np.array_equal(cf, bf16_bits_to_f32(a))


def test_pack_device_matches_host(llk, gpu):
    """The device pack kernel writes the same payload as the host packer."""
    print("case pack device vs host", flush=True)
    from dslcompiler_amd._lib import lib
    w = normal_bf16(5, 1, (200, 300))
    host = llk.pack_device_layout(w)
    pw = llk.PackedWeights.from_device(to_dev(gpu, w))
    n = pw.device_bytes
    assert n == host.size

    class _View:  # zero-copy view of the payload through __cuda_array_interface__
        __cuda_array_interface__ = {
            "shape": (n,), "typestr": "|u1", "version": 3, "strides": None,
            "data": (int(lib().llk_packed_weights_device_data(pw.handle)), False)}
    dev = gpu.as_tensor(_View(), device="cuda")
    assert np.array_equal(dev.cpu().numpy(), host)


def test_mlp(llk, gpu, orc):
    """MLP block (config 5 structure) at a small ragged size."""
    print("case mlp", flush=True)
    for M in (1, 17, 255):
        K, N = 320, 448
        x, wg, wu = swiglu_inputs(M, K, N, seed=21)
        x = outliers(x, seed=21)
        wd = normal_bf16(21, 3, (N, K), 1.0 / np.sqrt(N))
        y_ref, z_ref = orc.mlp(x, wg, wu, wd)
        yf_ref, _ = orc.swiglu(x, wg, wu)
        pg, pu, pd = (llk.PackedWeights.from_host(w) for w in (wg, wu, wd))
        y, z = llk.mlp(to_dev(gpu, x), pg, pu, pd)
        y, z = from_dev(y), from_dev(z)
        assert_parity_bf16(y, yf_ref, f"mlp y M={M}")
        # each stage against the oracle applied to that stage's own input:
        # Z consumes the GPU's Y, so compare with the oracle GEMM of that Y
        zf_ref, _ = orc.gemm(y, wd)
        assert_parity_bf16(z, zf_ref, f"mlp z M={M}")
        # end to end against the oracle's own chain (Y rounding flips feed Z)
        p = parity(bf16_bits_to_f32(z), bf16_bits_to_f32(z_ref))
        assert p["rel_l2"] <= 1e-3, p


def test_errors(llk, gpu):
    """Shape and scratch errors come back as LLKError with a message."""
    print("case errors", flush=True)
    wg = llk.PackedWeights.from_host(normal_bf16(1, 1, (16, 32)))
    wu = llk.PackedWeights.from_host(normal_bf16(1, 2, (16, 48)))
    x = gpu.zeros((4, 16), dtype=gpu.bfloat16, device="cuda")
    with pytest.raises(llk.LLKError, match="N dimension mismatch"):
        llk.fused_swiglu(x, wg, wu, out=gpu.empty((4, 32), dtype=gpu.bfloat16, device="cuda"))
    x2 = gpu.zeros((4, 15), dtype=gpu.bfloat16, device="cuda")
    with pytest.raises(llk.LLKError, match="K dimension mismatch"):
        llk.fused_swiglu(x2, wg, wg)
    big = llk.PackedWeights.from_host(normal_bf16(1, 1, (1024, 32)))
    need = llk.swiglu_scratch_size(4, 32, 1024)
    assert need > 4
    with pytest.raises(llk.LLKError, match="LLK_ERR_SCRATCH"):
        llk.fused_swiglu(gpu.zeros((4, 1024), dtype=gpu.bfloat16, device="cuda"), big, big,
                         scratch=gpu.zeros(4, dtype=gpu.uint8, device="cuda"))
    # operand dtypes the kernels do not read or write are refused up front
    with pytest.raises(ValueError, match="x has dtype"):
        llk.fused_swiglu(x.float(), wg, wg)
    with pytest.raises(ValueError, match="out has dtype"):
        llk.fused_swiglu(x, wg, wg, out=gpu.empty((4, 32), dtype=gpu.float16, device="cuda"))
    with pytest.raises(ValueError, match="y has dtype"):
        llk.mlp(x, wg, wg, llk.PackedWeights.from_host(normal_bf16(1, 3, (32, 8))),
                y=gpu.empty((4, 32), dtype=gpu.float32, device="cuda"))


GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


@pytest.mark.parametrize("shape", [(32, 128, 256), (16, 512, 512), (32, 256, 127), (4, 8, 3)])
def test_golden_reference_inputs_on_gpu(llk, gpu, orc, shape):
    """The reference tests' own inputs (tests/golden, reproduced from their
    mt19937 streams): the kernel's fp32 result against the reference's own
    fp64 routine and against the oracle; bf16 result = RNE of it."""
    print(f"case golden {shape}", flush=True)
    g = np.load(GOLDEN / "ref_vectors.npz")
    M, N, K = shape
    t = f"vec_M{M}_N{N}_K{K}"
    x, wg, wu, y64 = g[t + "_x"], g[t + "_wg"], g[t + "_wu"], g[t + "_y_fp64"]
    yf = _run_swiglu(llk, gpu, x, wg, wu, gpu.float32)
    p = parity(yf, y64)
    assert p["rel_l2"] < 2e-6 and p["max_abs_over_rms"] < 2e-5, p
    yf_ref, _ = orc.swiglu(x, wg, wu)
    assert_parity(yf, yf_ref, f"golden {shape}")


def test_golden_config1_samples_on_gpu(llk, gpu):
    """BASELINE config 1 through the GPU against the committed oracle samples."""
    print("case golden config1", flush=True)
    s = np.load(GOLDEN / "config1_samples.npz")
    x, wg, wu = swiglu_inputs(64, 512, 1376, seed=42)
    yf = _run_swiglu(llk, gpu, x, wg, wu, gpu.float32).ravel()[s["index"]]
    yb = _run_swiglu(llk, gpu, x, wg, wu, gpu.bfloat16).ravel()[s["index"]]
    assert_parity(yf, s["y_fp32"], "config1 samples fp32")
    assert np.mean(yb == s["y_bf16"]) > 0.99


@pytest.mark.parametrize("M,splits", [(300, 0), (300, 3), (8, 0), (40, 2)])
def test_gemm_fp16_out(llk, gpu, orc, M, splits):
    """llk.matmul's f16 result type: the fp16 output is RNE of the same
    kernel's fp32 result (numpy's float32 -> float16 rounds to nearest even)
    and meets the bar against the oracle; overflow gives infinity."""
    print(f"case gemm fp16 M={M} splits={splits}", flush=True)
    K, N = 768, 520
    s = 1.0 / np.sqrt(K)
    a = normal_bf16(13, 0, (M, K), s * 8)
    b = normal_bf16(13, 1, (K, N), s)
    pb = llk.PackedWeights.from_host(b)
    ad = to_dev(gpu, a)
    knob = "tile_splits" if M > 64 else "decode_splits"
    with _Tunable(llk, knob, splits):
        cf = from_dev(llk.matmul(ad, pb, out_dtype=gpu.float32))
        ch = from_dev(llk.matmul(ad, pb, out_dtype=gpu.float16))
    assert ch.dtype == np.float16
    assert np.array_equal(ch.view(np.uint16), cf.astype(np.float16).view(np.uint16))
    cf_ref, _ = orc.gemm(a, b)
    assert_parity(ch.astype(np.float32), cf_ref, f"gemm fp16 M={M}")
    # overflow: exact integer products beyond fp16's 65504
    big = to_bf16_bits(np.full((M, 64), 64.0, np.float32))
    ones = to_bf16_bits(np.full((64, 128), 32.0, np.float32))  # 64*64*32 = 131072
    hb = from_dev(llk.matmul(to_dev(gpu, big), llk.PackedWeights.from_host(ones),
                             out_dtype=gpu.float16))
    assert np.all(np.isposinf(hb))
