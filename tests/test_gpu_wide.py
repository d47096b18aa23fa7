"""The wide SwiGLU tile kernel (kernels/swiglu_wide.hip: tiles of 16 B columns
per matrix, B = 7 or 11, bf16 output).

It runs the same MFMAs over the same 32-k stages as the 128-column tile
kernel and the same SiLU epilogue, so its output must equal that kernel's
unsplit output bit for bit -- and RNE of that kernel's unsplit fp32 output --
on every shape (a k split sums fp32 partial planes in split order, which
rounds differently); it is also held to the oracle
(FuseDoubleContraction.cpp:155-199 semantics) at the bar.
Shapes cover one 64-k step and odd step counts (the four-stage loop body
exits after two stages), ragged M and N (last tiles partly outside Y, weight
blocks past the payload), tiles starting at every 16-column offset inside
the packed 128-column blocks, more than 8 m-tiles (grouped tile order), a
padded X, misaligned outputs and exact-integer inputs."""
from __future__ import annotations

import contextlib
import os

import numpy as np
import pytest

from common import assert_parity_bf16, bf16_bits_to_f32, swiglu_inputs, to_bf16_bits
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu


@contextlib.contextmanager
def _tunables(llk, **kv):
    old = {k: llk.get_tunable(k) for k in kv}
    try:
        for k, v in kv.items():
            llk.set_tunable(k, v)
        yield
    finally:
        for k, v in old.items():
            llk.set_tunable(k, v)


def _threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


# (M, N, K)
SHAPES = [
    (65, 176, 64),      # one tile, one 64-k step, ragged M
    (256, 368, 128),    # last n tile 16 columns wide
    (300, 1000, 192),   # odd 64-k steps, ragged M and N
    (513, 1376, 320),   # three m tiles
    (777, 2200, 200),   # K % 64 != 0: padded X
    (1024, 11008, 256),  # config 3's N: tiles start at every 16-column offset of a block
    (2100, 600, 1024),  # 9 m tiles: a group of 8 and a short one
    (384, 1232, 4096),  # long K
]


def _wide_and_tile(llk, gpu, x, wg, wu, B, x_stride=None):
    M, K = x.shape
    N = wg.shape[1]
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x, x_stride)
    # midm_max_m = 64: rows 65..128 stay on the tile kernels
    with _tunables(llk, tile_wide=B, tile_splits=1, midm_max_m=64):
        plan = llk.describe_launch("fused_swiglu", M, N, K, x_aligned=x_stride is None and K % 64 == 0)
        assert (plan["kernel"], plan["tile_columns"], plan["splits"]) == ("wide_tile", 16 * B, 1), plan
        yw = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    with _tunables(llk, tile_wide=0, tile_splits=1, midm_max_m=64):
        plan = llk.describe_launch("fused_swiglu", M, N, K)
        assert (plan["kernel"], plan["splits"]) == ("tile", 1), plan
        yt = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
        yf = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.float32))  # fp32: 128-column
    gpu.cuda.synchronize()
    pg.free()
    pu.free()
    return yw, yt, yf


@pytest.mark.parametrize("B", [11, 7])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_wide_matches_tile_kernel_and_oracle(llk, gpu, orc, B, M, N, K):
    print(f"case wide B={B} M={M} N={N} K={K}", flush=True)
    x, wg, wu = swiglu_inputs(M, K, N, seed=B * 1000 + M)
    yw, yt, yf = _wide_and_tile(llk, gpu, x, wg, wu, B)
    assert np.array_equal(yw, yt), f"B={B} {M}x{N}x{K}: differs from the 128-column kernel"
    assert np.array_equal(yw, to_bf16_bits(yf)), f"B={B} {M}x{N}x{K}: != RNE(fp32)"
    _, yf_ref = orc.swiglu_avx2(x, wg, wu, _threads(), want_f32=True)
    assert_parity_bf16(yw, yf_ref, f"wide B={B} {M}x{N}x{K}")


@pytest.mark.parametrize("B", [11, 7])
def test_wide_strided_x(llk, gpu, orc, B):
    """X rows with a wider stride than K (aligned): read in place."""
    print(f"case wide strided x B={B}", flush=True)
    M, N, K = 300, 700, 256
    x, wg, wu = swiglu_inputs(M, K, N, seed=3 + B)
    yw, yt, _ = _wide_and_tile(llk, gpu, x, wg, wu, B, x_stride=K + 64)
    assert np.array_equal(yw, yt)
    _, yf_ref = orc.swiglu_avx2(x, wg, wu, _threads(), want_f32=True)
    assert_parity_bf16(yw, yf_ref, f"wide strided B={B}")


@pytest.mark.parametrize("B", [11, 7])
def test_wide_misaligned_y(llk, gpu, orc, B):
    """Y a view one element into its buffer with an odd row stride (no
    16-byte chunks): the element-wise copy-out; columns either side of the
    view stay untouched."""
    print(f"case wide misaligned y B={B}", flush=True)
    M, N, K = 300, 500, 128
    x, wg, wu = swiglu_inputs(M, K, N, seed=40 + B)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x)
    buf = gpu.full((M, N + 7), 7.0, dtype=gpu.bfloat16, device="cuda")
    y = buf[:, 1:N + 1]
    with _tunables(llk, tile_wide=B, tile_splits=1):
        assert llk.describe_launch("fused_swiglu", M, N, K)["kernel"] == "wide_tile"
        llk.fused_swiglu(xd, pg, pu, out=y)
    with _tunables(llk, tile_wide=0, tile_splits=1):
        yt = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    gpu.cuda.synchronize()
    host = from_dev(buf)
    edge = np.concatenate([host[:, :1], host[:, N + 1:]], axis=1)
    assert np.all(bf16_bits_to_f32(edge) == 7.0), "wrote outside the view"
    assert np.array_equal(host[:, 1:N + 1], yt)


@pytest.mark.parametrize("B", [11, 7])
def test_wide_exact_integers(llk, gpu, orc, B):
    """Small-integer inputs: gate and up are exact in fp32 in any order, so
    the result equals the oracle's bf16 but for the expf implementation (at
    most 1 ulp, on under 1% of the outputs)."""
    print(f"case wide exact integers B={B}", flush=True)
    rng = np.random.default_rng(B)
    M, K, N = 260, 192, 16 * B * 3 + 48
    x = to_bf16_bits(rng.integers(-3, 4, (M, K)).astype(np.float32))
    wg = to_bf16_bits(rng.integers(-2, 3, (K, N)).astype(np.float32) * 0.0625)
    wu = to_bf16_bits(rng.integers(-2, 3, (K, N)).astype(np.float32) * 0.125)
    yw, yt, _ = _wide_and_tile(llk, gpu, x, wg, wu, B)
    assert np.array_equal(yw, yt)
    _, yb_ref = orc.swiglu(x, wg, wu)
    d = np.abs(yw.astype(np.int32) - yb_ref.astype(np.int32))
    assert d.max() <= 1 and np.mean(d == 0) > 0.99


@pytest.mark.parametrize("B", [11, 7])
def test_wide_epilogue_every_bf16_gate(llk, gpu, B):
    """K = 1, X = 1, Wg = g, Wu = 1 over every finite bf16 g with |g| <= 80:
    the wide kernel's bf16 SiLU(g) equals RNE of the 128-column kernel's fp32
    one (whose accuracy against the fp64 closed form the parity tests pin)."""
    print(f"case wide epilogue B={B}", flush=True)
    bits = np.arange(1 << 16, dtype=np.uint32)
    gv = (bits << 16).view(np.float32)
    gv = np.unique(gv[np.isfinite(gv) & (np.abs(gv) <= 80.0)])
    M, N = 70, gv.size
    x = to_bf16_bits(np.ones((M, 1), np.float32))
    wg = to_bf16_bits(np.tile(gv.reshape(1, N), (1, 1)))
    wu = to_bf16_bits(np.ones((1, N), np.float32))
    yw, _, yf = _wide_and_tile(llk, gpu, x, wg, wu, B)
    assert np.array_equal(yw, to_bf16_bits(yf))


def test_wide_config3_whole_output(llk, gpu, orc):
    """Config 3 (M = 2048, K = 4096, N = 11008), where the dispatcher takes
    the wide kernel (B = 11, 504 tiles): every output equal to the 128-column
    kernel's, every row at the bar against the oracle, reruns bit-identical."""
    print("case wide config 3 whole output", flush=True)
    M, K, N = 2048, 4096, 11008
    plan = llk.describe_launch("fused_swiglu", M, N, K)
    assert (plan["kernel"], plan["tile_columns"], plan["workgroups"]) == ("wide_tile", 176, 504)
    x, wg, wu = swiglu_inputs(M, K, N, seed=42)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x)
    yw = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    yw2 = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    with _tunables(llk, tile_wide=0, tile_splits=1):
        yt = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    gpu.cuda.synchronize()
    assert np.array_equal(yw, yw2), "reruns differ"
    assert np.array_equal(yw, yt), "differs from the 128-column kernel"
    _, yf_ref = orc.swiglu_avx2(x, wg, wu, _threads(), want_f32=True)
    for m0 in range(0, M, 256):
        assert_parity_bf16(yw[m0:m0 + 256], yf_ref[m0:m0 + 256], f"config 3 rows {m0}..")


# (M, N, K, S): k splits of the wide kernel; config 5's SwiGLU at M = 255 is
# the dispatcher's own choice (B = 7, S = 2)
SPLIT_SHAPES = [
    (255, 13824, 5120, 2),
    (100, 1000, 1000, 3),   # padded X, ragged M and N, odd block count per split
    (300, 700, 640, 2),     # two m tiles, last n tile partial
    (513, 2200, 320, 3),    # three m tiles, 5 blocks over 3 splits
]


@pytest.mark.parametrize("B", [7, 11])
@pytest.mark.parametrize("M,N,K,S", SPLIT_SHAPES)
def test_wide_split_matches_tile_split_and_oracle(llk, gpu, orc, B, M, N, K, S):
    """The k split sums register-order partials in split order over the same
    k ranges as the 128-column kernel's split, so the two agree bit for bit;
    every output at the bar against the oracle."""
    print(f"case wide split B={B} M={M} N={N} K={K} S={S}", flush=True)
    x, wg, wu = swiglu_inputs(M, K, N, seed=7 * B + S)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x)
    with _tunables(llk, tile_wide=B, tile_splits=S):
        plan = llk.describe_launch("fused_swiglu", M, N, K, x_aligned=K % 64 == 0)
        assert (plan["kernel"], plan["tile_columns"], plan["splits"]) == ("wide_tile", 16 * B, S), plan
        yw = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    with _tunables(llk, tile_wide=0, tile_splits=S):
        plan = llk.describe_launch("fused_swiglu", M, N, K)
        assert (plan["kernel"], plan["splits"]) == ("tile", S), plan
        yt = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    gpu.cuda.synchronize()
    assert np.array_equal(yw, yt), f"B={B} S={S} {M}x{N}x{K}: differs from the 128-column split"
    _, yf_ref = orc.swiglu_avx2(x, wg, wu, _threads(), want_f32=True)
    assert_parity_bf16(yw, yf_ref, f"wide split B={B} S={S} {M}x{N}x{K}")


def test_wide_split_default_plan_config5(llk, gpu):
    """The dispatcher's plan for config 5's SwiGLU at M = 255 (B = 7, S = 2,
    248 workgroups, register-order partials in the workspace), run twice:
    reruns bit-identical."""
    M, N, K = 255, 13824, 5120
    plan = llk.describe_launch("fused_swiglu", M, N, K)
    assert (plan["kernel"], plan["tile_columns"], plan["splits"], plan["workgroups"]) == \
        ("wide_tile", 112, 2, 248), plan
    assert plan["workspace_bytes"] == 2 * 124 * 4 * 7 * 8 * 64 * 16
    x, wg, wu = swiglu_inputs(M, K, N, seed=5)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x)
    y1 = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    y2 = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    gpu.cuda.synchronize()
    assert np.array_equal(y1, y2)
