"""Whole-output parity of the tile kernel where its grouped tile order is
active: more than 8 m-tiles (M > 2048) together with several n-tiles, a short
last group of m-tiles, with and without k splits, and with the tail split
(the columns of a partial last wave as a separate k-split launch).  The
wide SwiGLU kernel, which the dispatcher would take for some of these
shapes, is switched off here (tests/test_gpu_wide.py covers it).  Every
row is compared with the oracle, so a tile computed into the wrong place
fails wherever it lands."""
from __future__ import annotations

import contextlib
import os

import numpy as np
import pytest

from common import assert_parity, assert_parity_bf16, normal_bf16, swiglu_inputs, to_bf16_bits
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


# (forced k splits, workgroups per wave (0: the first of TAIL_WAVES whose
# plan has a tail-split launch), expect a tail-split launch)
VARIANTS = [(1, 256, False), (3, 256, False), (0, 0, True)]
TAIL_WAVES = (40, 24, 20, 12)
K_ORDER, N_ORDER = 1024, 600


def _per_wave(llk, op, M, per_wave):
    if per_wave:
        return per_wave
    for w in TAIL_WAVES:
        with _tunables(llk, tile_splits=0, tile_wgs_per_wave=w, tile_tail_split=1, tile_wide=0):
            if llk.describe_launch(op, M, N_ORDER, K_ORDER)["head_blocks_n"] > 0:
                return w
    raise AssertionError(f"no workgroups-per-wave value engages the tail split for {op} M={M}")


@pytest.mark.parametrize("M", [2305, 4097])
@pytest.mark.parametrize("splits,per_wave,tail", VARIANTS)
def test_swiglu_grouped_order_whole_output(llk, gpu, orc, M, splits, per_wave, tail):
    K, N = K_ORDER, N_ORDER
    per_wave = _per_wave(llk, "fused_swiglu", M, per_wave)
    print(f"case swiglu order M={M} S={splits} per_wave={per_wave}", flush=True)
    x, wg, wu = swiglu_inputs(M, K, N, seed=31)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    with _tunables(llk, tile_splits=splits, tile_wgs_per_wave=per_wave, tile_tail_split=1,
                   tile_wide=0):
        plan = llk.describe_launch("fused_swiglu", M, N, K)
        assert plan["kernel"] == "tile"
        assert (plan["head_blocks_n"] > 0) == tail, plan
        if splits:
            assert plan["splits"] == splits, plan
        xd = to_dev(gpu, x)
        yb = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
        yf = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.float32))
    gpu.cuda.synchronize()
    _, yf_ref = orc.swiglu_avx2(x, wg, wu, _threads(), want_f32=True)
    assert np.array_equal(yb, to_bf16_bits(yf))
    for m0 in range(0, M, 256):
        rs = slice(m0, m0 + 256)
        assert_parity(yf[rs], yf_ref[rs], f"swiglu M={M} rows {m0}..")
        assert_parity_bf16(yb[rs], yf_ref[rs], f"swiglu M={M} bf16 rows {m0}..")


@pytest.mark.parametrize("M", [2305, 4097])
@pytest.mark.parametrize("splits,per_wave,tail", VARIANTS)
def test_gemm_grouped_order_whole_output(llk, gpu, orc, M, splits, per_wave, tail):
    K, N = K_ORDER, N_ORDER
    per_wave = _per_wave(llk, "matmul", M, per_wave)
    print(f"case gemm order M={M} S={splits} per_wave={per_wave}", flush=True)
    a = normal_bf16(32, 0, (M, K))
    b = normal_bf16(32, 1, (K, N), 1.0 / np.sqrt(K))
    pb = llk.PackedWeights.from_host(b)
    with _tunables(llk, tile_splits=splits, tile_wgs_per_wave=per_wave, tile_tail_split=1):
        plan = llk.describe_launch("matmul", M, N, K)
        assert plan["kernel"] == "tile"
        assert (plan["head_blocks_n"] > 0) == tail, plan
        c = from_dev(llk.matmul(to_dev(gpu, a), pb, out_dtype=gpu.float32))
    gpu.cuda.synchronize()
    cf_ref, _ = orc.gemm_avx2(a, b, _threads(), want_bf16=False)
    for m0 in range(0, M, 256):
        rs = slice(m0, m0 + 256)
        assert_parity(c[rs], cf_ref[rs], f"gemm M={M} rows {m0}..")
