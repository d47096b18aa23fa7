"""The tile kernel's two-piece k split (SwiGLU's partial last wave, or all
of its tiles when there is no whole wave; knob tile_two_piece, off by
default): each tile's k range runs as a long and a short piece, and the
piece that arrives second finishes the tile from both pieces' raw fp32
accumulators.

- Parity with the oracle on every row, for shapes with ragged rows and
  columns and for a whole-wave head plus a two-piece tail.
- The same inputs without the two-piece form (knob tile_two_piece = 0)
  differ only by the order of the k sum: fp32 outputs within the bar, and
  bit-identical where the two-piece grid runs whole tiles (the head).
- Bit-identical reruns (the sum P0 + P1 does not depend on which piece
  arrives second: fp32 addition commutes).
- A caller scratch whose counter area holds garbage (the library clears it
  before the launch), and the library's workspace reused across shapes."""
from __future__ import annotations

import numpy as np
import pytest

from common import assert_parity, assert_parity_bf16, swiglu_inputs
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def two_piece_on(llk):
    """The form is off by default (measured slower on MI355X): these tests
    switch it on."""
    llk.set_tunable("tile_two_piece", 1)
    yield
    llk.set_tunable("tile_two_piece", 0)


SHAPES = [
    (300, 1000, 512),    # 2 x 8 tiles, ragged rows and columns, no whole wave
    (257, 1280, 768),    # one row into the second m-tile
    (1000, 2000, 1024),  # 4 x 16 tiles
]


def _plan(llk, M, N, K):
    return llk.describe_launch("fused_swiglu", M, N, K)


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_two_piece_parity(llk, gpu, orc, M, N, K):
    print(f"case two-piece parity M={M} N={N} K={K}", flush=True)
    assert _plan(llk, M, N, K)["two_piece_kb"] > 0
    x, wg, wu = swiglu_inputs(M, K, N, seed=31)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x)
    yf = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.float32))
    yb = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    yb2 = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    gpu.cuda.synchronize()
    assert np.array_equal(yb, yb2), "reruns differ"
    yf_ref, _ = orc.swiglu(x, wg, wu)
    assert_parity(yf, yf_ref, f"two-piece fp32 {M}x{N}x{K}")
    assert_parity_bf16(yb, yf_ref, f"two-piece bf16 {M}x{N}x{K}")
    old = llk.get_tunable("tile_two_piece")
    llk.set_tunable("tile_two_piece", 0)
    try:
        assert _plan(llk, M, N, K)["two_piece_kb"] == 0
        yf1 = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.float32))
    finally:
        llk.set_tunable("tile_two_piece", old)
    assert_parity(yf, yf1, "two-piece vs one piece (order of the k sum only)")


def test_two_piece_tail_after_whole_waves(llk, gpu, orc):
    """Config 5's SwiGLU at M = 1000: 256 whole tiles, then 176 as two
    pieces (cut at 61 of 80 blocks), in one grid; every row against the
    oracle, and the head's columns bit-identical to the one-launch form."""
    M, N, K = 1000, 13824, 5120
    print(f"case two-piece tail M={M}", flush=True)
    p = _plan(llk, M, N, K)
    assert (p["head_blocks_n"], p["two_piece_kb"]) == (64, 61)
    x, wg, wu = swiglu_inputs(M, K, N, seed=32)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x)
    yf = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.float32))
    _, yf_ref = orc.swiglu_avx2(x, wg, wu, 16, want_f32=True)
    assert_parity(yf, yf_ref, "M=1000 fp32 (all rows)")
    for n0 in range(64 * 128, N, 128):  # every tail column block on its own
        assert_parity(yf[:, n0:n0 + 128], yf_ref[:, n0:n0 + 128], f"tail columns {n0}..")
    # The head's whole tiles run in the two-piece grid with the plain
    # kernel's arithmetic: bit-identical to the one-launch form there.
    llk.set_tunable("tile_two_piece", 0)
    try:
        yf1 = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.float32))
    finally:
        llk.set_tunable("tile_two_piece", 1)
    head = 64 * 128
    assert np.array_equal(yf[:, :head].view(np.uint32), yf1[:, :head].view(np.uint32)), \
        "head columns differ from the one-launch form"
    assert_parity(yf[:, head:], yf1[:, head:], "tail vs one piece (order of the k sum only)")


def test_caller_scratch_with_garbage_counters(llk, gpu):
    M, N, K = 300, 1000, 512
    print("case two-piece caller scratch", flush=True)
    p = _plan(llk, M, N, K)
    assert p["two_piece_kb"] > 0
    x, wg, wu = swiglu_inputs(M, K, N, seed=33)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x)
    want = from_dev(llk.fused_swiglu(xd, pg, pu))
    scratch = gpu.full((p["workspace_bytes"],), 0xFF, dtype=gpu.uint8, device="cuda")
    for _ in range(2):  # the second call finds the counters it left
        got = from_dev(llk.fused_swiglu(xd, pg, pu, scratch=scratch))
        assert np.array_equal(got, want)


def test_workspace_reused_across_shapes(llk, gpu):
    """Calls of other shapes and kernels between two-piece calls on the
    library's workspace (padded X, k-split planes, small-M partials) leave
    its counter area untouched."""
    print("case two-piece workspace reuse", flush=True)
    cases = []
    for M, N, K in [(300, 1000, 512), (300, 640, 1000), (8, 4096, 2048), (1000, 2000, 1024)]:
        x, wg, wu = swiglu_inputs(M, K, N, seed=34)
        pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
        xd = to_dev(gpu, x)
        cases.append((xd, pg, pu, from_dev(llk.fused_swiglu(xd, pg, pu))))
    for _ in range(2):
        for xd, pg, pu, want in cases:
            assert np.array_equal(from_dev(llk.fused_swiglu(xd, pg, pu)), want)
