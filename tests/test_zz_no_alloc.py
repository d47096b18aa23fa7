"""llk_swiglu_bf16_noalloc (the entry point that allocates nothing: its
workspace is a fixed device array built into the library) against the
existing entry point llk_swiglu_bf16 on the same inputs, called through the
C ABI, to the north-star bar (bit-identical where both choose the same
launch plan); two calls in a row, the second with a smaller input, since the
fixed array keeps the previous call's contents."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from common import assert_parity, assert_parity_bf16, swiglu_inputs, to_bf16_bits
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu

NOALLOC_BYTES = 64 << 20


def _t2d(llk, t):
    return llk._lib.tensor2d(t.data_ptr(), t.shape[0], t.shape[1], t.stride(0), t.stride(1))


def _both(llk, torch, x, wg, wu, out_dtype, x_stride=None):
    """(existing entry's output, no-allocation entry's output) on the current stream."""
    L = llk.lib()
    M, K = x.shape
    N = wg.shape[1]
    xd = to_dev(torch, x, x_stride)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    code = llk._lib.LLK_BF16 if out_dtype == torch.bfloat16 else llk._lib.LLK_FP32
    stream = torch.cuda.current_stream().cuda_stream
    y_ref = torch.full((M, N), float("nan"), dtype=out_dtype, device="cuda")
    y_new = torch.full((M, N), float("nan"), dtype=out_dtype, device="cuda")
    ctx = llk._lib.KernelContext(None, 0, stream)
    llk._lib.check(L.llk_swiglu_bf16(C.byref(_t2d(llk, xd)), pg.handle, pu.handle,
                                C.byref(_t2d(llk, y_ref)), code, C.byref(ctx)))
    llk._lib.check(L.llk_swiglu_bf16_noalloc(C.byref(_t2d(llk, xd)), pg.handle, pu.handle,
                                        C.byref(_t2d(llk, y_new)), code, stream))
    torch.cuda.synchronize()
    return from_dev(y_ref), from_dev(y_new)


# (M, K, N, X row stride or None): each pair is a larger call then a smaller one.
PAIRS = [
    # k splits (bf16: the wide kernel's register-order partials, fp32: the
    # 128-column kernel's planes); then padded X
    ((255, 5120, 13824, None), (100, 1000, 500, 1003)),
    ((8, 13824, 5120, None), (3, 4096, 384, None)),       # small-M k split; then unsplit
    ((9000, 4000, 256, None), (300, 4000, 256, 4008)),    # padded X beyond the array: chunks
    ((128, 2048, 1000, None), (70, 1024, 600, None)),     # mid M (decode tile, 128 rows), k splits
]


@pytest.mark.parametrize("pair", PAIRS, ids=["tile-split", "small-m-split", "pad-chunks",
                                             "mid-m-split"])
def test_noalloc_matches_existing_entry(llk, gpu, orc, pair):
    for M, K, N, xs in pair:
        print(f"case noalloc M={M} K={K} N={N} x_stride={xs}", flush=True)
        x, wg, wu = swiglu_inputs(M, K, N, seed=M + K)
        plan = llk.describe_launch("fused_swiglu", M, N, K, x_aligned=xs is None)
        yb_ref, yb = _both(llk, gpu, x, wg, wu, gpu.bfloat16, xs)
        yf_ref, yf = _both(llk, gpu, x, wg, wu, gpu.float32, xs)
        assert not np.isnan(yf).any()
        assert np.array_equal(yb, to_bf16_bits(yf))
        if plan["workspace_bytes"] <= NOALLOC_BYTES:
            # same launch plan as the existing entry point: identical bits
            assert np.array_equal(yf.view(np.uint32), yf_ref.view(np.uint32))
            assert np.array_equal(yb, yb_ref)
        assert_parity(yf, yf_ref, f"noalloc vs existing M={M} fp32")
        assert_parity_bf16(yb, yf_ref, f"noalloc vs existing M={M} bf16")
        rows = sorted({0, M // 2, M - 1})
        ref, _ = orc.swiglu_rows(x, wg, wu, rows)
        assert_parity(yf[rows], ref, f"noalloc vs oracle M={M}")


def test_noalloc_rejects_what_cannot_fit(llk, gpu):
    """A padded X whose 256-row chunk alone exceeds the fixed array (K above
    ~65000) is refused with LLK_ERR_SCRATCH and a message, before any launch."""
    L = llk.lib()
    M, K, N = 300, 140_000, 128
    print(f"case noalloc reject M={M} K={K}", flush=True)
    x = gpu.zeros((M, K + 1), dtype=gpu.bfloat16, device="cuda")[:, :K]
    wg = np.zeros((K, N), np.uint16)
    pg = llk.PackedWeights.from_host(wg)
    y = gpu.empty((M, N), dtype=gpu.bfloat16, device="cuda")
    st = L.llk_swiglu_bf16_noalloc(C.byref(_t2d(llk, x)), pg.handle, pg.handle,
                                   C.byref(_t2d(llk, y)), llk._lib.LLK_BF16, None)
    assert st == llk._lib.LLK_ERR_SCRATCH, st
    assert b"workspace" in L.llk_last_error()
