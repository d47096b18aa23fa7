"""The reference's KernelFn calling convention (JitCache.h:79-81):
llk_swiglu_kernel_fn(x, wg, wu, init, result) with five 56-byte MemRef2D
descriptors (JitCache.h:43-51) built here in ctypes, init == result as the
reference's callers pass them (swiglu_vector_avx2.cpp:278-285), raw
row-major weights resolved through the L4 weight level (a miss packs, the
next call with the same buffers hits), against the oracle; with device
operands and with host operands (the reference's callers' own buffers)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from common import assert_parity_bf16, swiglu_inputs
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _memref(ptr: int, rows: int, cols: int, stride0: int, offset: int = 0):
    from dslcompiler_amd._lib import MemRef2D
    return MemRef2D(ptr, ptr, offset, rows, cols, stride0, 1)


def _l4(llk):
    from dslcompiler_amd._lib import CacheStatsC
    st = CacheStatsC()
    cache = llk.lib().llk_kernel_fn_cache()
    assert cache
    llk._lib.check(llk.lib().llk_cache_get_stats(cache, C.byref(st)))
    return st.hits[3], st.misses[3]


def test_memref_is_56_bytes():
    from dslcompiler_amd._lib import MemRef2D
    assert C.sizeof(MemRef2D) == 56


@pytest.mark.parametrize("M,K,N", [(8, 1024, 768), (300, 576, 392)])
def test_kernel_fn_device_operands(llk, gpu, orc, M, K, N):
    print(f"case kernel_fn device M={M} K={K} N={N}", flush=True)
    L = llk.lib()
    x, wg, wu = swiglu_inputs(M, K, N, seed=M + 5)
    xd, wgd, wud = to_dev(gpu, x), to_dev(gpu, wg), to_dev(gpu, wu)
    y = gpu.full((M, N), float("nan"), dtype=gpu.bfloat16, device="cuda")
    mx = _memref(xd.data_ptr(), M, K, K)
    mg = _memref(wgd.data_ptr(), K, N, N)
    mu = _memref(wud.data_ptr(), K, N, N)
    my = _memref(y.data_ptr(), M, N, N)
    yf_ref, _ = orc.swiglu(x, wg, wu)
    L.llk_cache_clear(L.llk_kernel_fn_cache())  # no stale entry at a reused address
    hits0, miss0 = _l4(llk)
    L.llk_swiglu_kernel_fn(C.byref(mx), C.byref(mg), C.byref(mu), C.byref(my), C.byref(my))
    assert L.llk_kernel_fn_status() == 0, L.llk_last_error()
    hits1, miss1 = _l4(llk)
    assert (hits1 - hits0, miss1 - miss0) == (0, 2), "first call: both weights packed (L4 miss)"
    got1 = from_dev(y)
    assert_parity_bf16(got1, yf_ref, "KernelFn device, first call")
    y.fill_(float("nan"))
    L.llk_swiglu_kernel_fn(C.byref(mx), C.byref(mg), C.byref(mu), C.byref(my), C.byref(my))
    assert L.llk_kernel_fn_status() == 0, L.llk_last_error()
    hits2, miss2 = _l4(llk)
    assert (hits2 - hits1, miss2 - miss1) == (2, 0), "second call: both weights from L4"
    assert np.array_equal(from_dev(y), got1)


def test_kernel_fn_host_operands_with_offset(llk, gpu, orc):
    """Host buffers as the reference's tests pass them, with a non-zero
    memref offset on X and a padded result row stride."""
    print("case kernel_fn host", flush=True)
    L = llk.lib()
    M, K, N = 33, 200, 136
    x, wg, wu = swiglu_inputs(M, K, N, seed=77)
    xbuf = np.zeros(M * K + 5, np.uint16)
    xbuf[5:] = x.ravel()
    wg_h, wu_h = np.ascontiguousarray(wg), np.ascontiguousarray(wu)
    ybuf = np.full((M, N + 8), 0xFFFF, np.uint16)
    mx = _memref(xbuf.ctypes.data, M, K, K, offset=5)
    mg = _memref(wg_h.ctypes.data, K, N, N)
    mu = _memref(wu_h.ctypes.data, K, N, N)
    my = _memref(ybuf.ctypes.data, M, N, N + 8)
    L.llk_swiglu_kernel_fn(C.byref(mx), C.byref(mg), C.byref(mu), C.byref(my), C.byref(my))
    assert L.llk_kernel_fn_status() == 0, L.llk_last_error()
    yf_ref, _ = orc.swiglu(x, wg, wu)
    assert_parity_bf16(ybuf[:, :N], yf_ref, "KernelFn host operands")
    assert np.all(ybuf[:, N:] == 0xFFFF), "row padding written"


def test_kernel_fn_reports_errors(llk, gpu):
    """No return value: a shape error leaves the status and message."""
    L = llk.lib()
    a = gpu.zeros((4, 8), dtype=gpu.bfloat16, device="cuda")
    mx = _memref(a.data_ptr(), 4, 8, 8)
    mw = _memref(a.data_ptr(), 4, 8, 8)  # K = 4 != 8
    L.llk_swiglu_kernel_fn(C.byref(mx), C.byref(mw), C.byref(mw), C.byref(mx), C.byref(mx))
    assert L.llk_kernel_fn_status() == llk._lib.LLK_ERR_SHAPE
    assert b"K dimension mismatch" in L.llk_last_error()
