"""The reference's KernelFn calling convention (JitCache.h:79-81):
fn(x, wg, wu, init, result) with five 56-byte MemRef2D descriptors
(JitCache.h:43-51) built here in ctypes, init == result as the reference's
callers pass them (swiglu_vector_avx2.cpp:278-285), raw row-major weights,
against the oracle; with device operands and with host operands (the
reference's callers' own buffers).

Like the reference's JIT'd function, every call reads the weights as they
are at the call: a buffer rewritten in place gives the new result; two host
threads calling at once both get right results.  Reuse of packed weights
across calls is opt-in (llk_kernel_fn_assume_immutable_weights).  The
object-code level hands out entries of the same shape that run the kernels
of the key's loaded code object (JitCache.cpp:182-250), also by string key
(JitCache.h:103-105)."""
from __future__ import annotations

import ctypes as C
import threading

import numpy as np
import pytest

from common import assert_parity, assert_parity_bf16, normal_bf16, swiglu_inputs
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


def _call(llk, mx, mg, mu, my):
    L = llk.lib()
    L.llk_swiglu_kernel_fn(C.byref(mx), C.byref(mg), C.byref(mu), C.byref(my), C.byref(my))
    assert L.llk_kernel_fn_status() == 0, L.llk_last_error()


def test_memref_is_56_bytes():
    from dslcompiler_amd._lib import MemRef2D
    assert C.sizeof(MemRef2D) == 56


@pytest.mark.parametrize("M,K,N", [(8, 1024, 768), (300, 576, 392)])
def test_kernel_fn_device_operands(llk, gpu, orc, M, K, N):
    """Device operands used in place; by default the weights are read at
    every call (M = 8: straight from the row-major buffers; M = 300: packed
    per call), the L4 level is not consulted, and repeated calls give the
    same bits."""
    print(f"case kernel_fn device M={M} K={K} N={N}", flush=True)
    x, wg, wu = swiglu_inputs(M, K, N, seed=M + 5)
    xd, wgd, wud = to_dev(gpu, x), to_dev(gpu, wg), to_dev(gpu, wu)
    y = gpu.full((M, N), float("nan"), dtype=gpu.bfloat16, device="cuda")
    mx, mg = _memref(xd.data_ptr(), M, K, K), _memref(wgd.data_ptr(), K, N, N)
    mu, my = _memref(wud.data_ptr(), K, N, N), _memref(y.data_ptr(), M, N, N)
    yf_ref, _ = orc.swiglu(x, wg, wu)
    l4_0 = _l4(llk)
    _call(llk, mx, mg, mu, my)
    got1 = from_dev(y)
    assert_parity_bf16(got1, yf_ref, "KernelFn device, first call")
    y.fill_(float("nan"))
    _call(llk, mx, mg, mu, my)
    assert np.array_equal(from_dev(y), got1)
    assert _l4(llk) == l4_0, "weights read per call, not through L4"


def test_kernel_fn_sees_weights_rewritten_in_place(llk, gpu, orc):
    """The caller rewrites wg in place (same address, same shape) between
    two calls: the second result is that of the new weights, as the
    reference's JIT'd function, which reads its arguments every call, gives."""
    print("case kernel_fn in-place weight rewrite", flush=True)
    M, K, N = 200, 768, 640
    x, wg, wu = swiglu_inputs(M, K, N, seed=31)
    _, wg2, _ = swiglu_inputs(M, K, N, seed=32)
    xd, wgd, wud = to_dev(gpu, x), to_dev(gpu, wg), to_dev(gpu, wu)
    y = gpu.empty((M, N), dtype=gpu.bfloat16, device="cuda")
    mx, mg = _memref(xd.data_ptr(), M, K, K), _memref(wgd.data_ptr(), K, N, N)
    mu, my = _memref(wud.data_ptr(), K, N, N), _memref(y.data_ptr(), M, N, N)
    _call(llk, mx, mg, mu, my)
    assert_parity_bf16(from_dev(y), orc.swiglu(x, wg, wu)[0], "before the rewrite")
    wgd.copy_(to_dev(gpu, wg2))  # same buffer, new contents
    gpu.cuda.synchronize()
    _call(llk, mx, mg, mu, my)
    assert_parity_bf16(from_dev(y), orc.swiglu(x, wg2, wu)[0], "after the in-place rewrite")
    # host weights likewise
    wg_h = np.ascontiguousarray(wg)
    mg_h = _memref(wg_h.ctypes.data, K, N, N)
    _call(llk, mx, mg_h, mu, my)
    assert_parity_bf16(from_dev(y), orc.swiglu(x, wg, wu)[0], "host wg")
    wg_h[:] = wg2
    _call(llk, mx, mg_h, mu, my)
    assert_parity_bf16(from_dev(y), orc.swiglu(x, wg2, wu)[0], "host wg rewritten")


def test_kernel_fn_two_threads_same_weights(llk, gpu, orc):
    """Two host threads call the KernelFn at once on the same weight buffers
    (each with its own X and result), several times each: every result
    matches the oracle."""
    print("case kernel_fn two threads", flush=True)
    K, N = 1024, 1536
    _, wg, wu = swiglu_inputs(8, K, N, seed=41)
    wgd, wud = to_dev(gpu, wg), to_dev(gpu, wu)
    jobs = []
    for t, M in enumerate((8, 700)):  # one small-M and one tile-kernel shape
        x, _, _ = swiglu_inputs(M, K, N, seed=50 + t)
        xd = to_dev(gpu, x)
        y = gpu.empty((M, N), dtype=gpu.bfloat16, device="cuda")
        jobs.append((M, x, xd, y))
    gpu.cuda.synchronize()
    L = llk.lib()
    errors, outs = [], [[] for _ in jobs]
    start = threading.Barrier(len(jobs))

    def run(i):
        M, _, xd, y = jobs[i]
        mx, my = _memref(xd.data_ptr(), M, K, K), _memref(y.data_ptr(), M, N, N)
        mg, mu = _memref(wgd.data_ptr(), K, N, N), _memref(wud.data_ptr(), K, N, N)
        start.wait()
        for _ in range(4):
            L.llk_swiglu_kernel_fn(C.byref(mx), C.byref(mg), C.byref(mu), C.byref(my),
                                   C.byref(my))
            if L.llk_kernel_fn_status() != 0:
                errors.append(L.llk_last_error())
                return
            outs[i].append(from_dev(y))  # the call is synchronous: y is final here

    th = [threading.Thread(target=run, args=(i,)) for i in range(len(jobs))]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errors, errors
    for (M, x, _, _), got in zip(jobs, outs):
        ref = orc.swiglu(x, wg, wu)[0]
        assert len(got) == 4
        for g in got:
            assert_parity_bf16(g, ref, f"thread M={M}")
            assert np.array_equal(g, got[0])


def test_kernel_fn_opt_in_reuse(llk, gpu, orc):
    """With llk_kernel_fn_assume_immutable_weights(1) the weights resolve
    through the device cache's L4 level: the first call packs both (two
    misses), the next hits both, and the result is unchanged."""
    print("case kernel_fn immutable weights", flush=True)
    M, K, N = 96, 512, 384
    x, wg, wu = swiglu_inputs(M, K, N, seed=61)
    xd, wgd, wud = to_dev(gpu, x), to_dev(gpu, wg), to_dev(gpu, wu)
    y = gpu.empty((M, N), dtype=gpu.bfloat16, device="cuda")
    mx, mg = _memref(xd.data_ptr(), M, K, K), _memref(wgd.data_ptr(), K, N, N)
    mu, my = _memref(wud.data_ptr(), K, N, N), _memref(y.data_ptr(), M, N, N)
    L = llk.lib()
    assert L.llk_kernel_fn_assume_immutable_weights(1) == 0
    try:
        L.llk_cache_clear(L.llk_kernel_fn_cache())  # no entry at a reused address
        h0, m0 = _l4(llk)
        _call(llk, mx, mg, mu, my)
        h1, m1 = _l4(llk)
        assert (h1 - h0, m1 - m0) == (0, 2)
        got = from_dev(y)
        _call(llk, mx, mg, mu, my)
        h2, m2 = _l4(llk)
        assert (h2 - h1, m2 - m1) == (2, 0)
        assert np.array_equal(from_dev(y), got)
        assert_parity_bf16(got, orc.swiglu(x, wg, wu)[0], "KernelFn with L4 reuse")
    finally:
        assert L.llk_kernel_fn_assume_immutable_weights(0) == 1
        L.llk_cache_clear(L.llk_kernel_fn_cache())


def test_kernel_fn_host_operands_with_offset(llk, gpu, orc):
    """Host buffers as the reference's tests pass them, with a non-zero
    memref offset on X and a padded result row stride."""
    print("case kernel_fn host", flush=True)
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
    _call(llk, mx, mg, mu, my)
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


def test_object_code_kernel_fn_entries(llk, gpu, orc):
    """lookupOrCompile hands back the KernelFn of the key (JitCache.cpp:
    182-250): a MemRef2D-shaped entry that runs the kernels of the key's
    loaded code object, its pack kernel included.  SwiGLU: bit-equal to
    llk_swiglu_kernel_fn and to the oracle's bar; matmul (fp32 key):
    result = init + x wg (linalg.matmul's outs(init)), init != result."""
    print("case object-code KernelFn entries", flush=True)
    from dslcompiler_amd import cache as cmod
    M, K, N = 300, 1000, 640
    x, wg, wu = swiglu_inputs(M, K, N, seed=71)
    xd, wgd, wud = to_dev(gpu, x), to_dev(gpu, wg), to_dev(gpu, wu)
    jc = llk.JitCache()
    fn = jc.lookup_or_compile(llk.KernelKey(operation=0, isa=7, N=N, K=K, M_bucket=4,
                                            weight_layout=2))
    y = gpu.full((M, N), float("nan"), dtype=gpu.bfloat16, device="cuda")
    fn(xd, wgd, wud, y, y)
    y_lib = gpu.empty_like(y)
    cmod.swiglu_kernel_fn(xd, wgd, wud, y_lib, y_lib)
    assert np.array_equal(from_dev(y), from_dev(y_lib))
    assert_parity_bf16(from_dev(y), orc.swiglu(x, wg, wu)[0], "object-code KernelFn")
    # fp32 matmul entry with a separate init
    mm = jc.lookup_or_compile(llk.KernelKey(operation=3, isa=7, N=N, K=K, output_type=2))
    init = gpu.randn((M, N), dtype=gpu.float32, device="cuda")
    c = gpu.full((M, N), float("nan"), dtype=gpu.float32, device="cuda")
    mm(xd, wgd, None, init, c)
    ref, _ = orc.gemm(x, wg)
    assert_parity(from_dev(c), ref + from_dev(init), "object-code matmul KernelFn")
    # in place (init == result): accumulates again
    mm(xd, wgd, None, c, c)
    assert_parity(from_dev(c), 2 * ref + from_dev(init), "matmul KernelFn in place")
    jc.close()


def test_string_keyed_kernel_fn(llk, gpu, orc):
    """The string-keyed lookupOrCompile (JitCache.h:103-105) with a module in
    the reference's MLIR text: its KernelFn runs on the GPU."""
    print("case string-keyed KernelFn", flush=True)
    M, K, N = 64, 512, 1376
    module = f"""
func.func @swiglu(%x: tensor<{M}x{K}xbf16>, %wg: tensor<{K}x{N}xbf16>, %wu: tensor<{K}x{N}xbf16>,
                  %init: tensor<{M}x{N}xbf16>) -> tensor<{M}x{N}xbf16> {{
  %0 = llk.fused_swiglu ins(%x, %wg, %wu : tensor<{M}x{K}xbf16>, tensor<{K}x{N}xbf16>,
                            tensor<{K}x{N}xbf16>) outs(%init : tensor<{M}x{N}xbf16>)
       -> tensor<{M}x{N}xbf16>
  return %0 : tensor<{M}x{N}xbf16>
}}
"""
    x, wg, wu = swiglu_inputs(M, K, N, seed=81)
    xd, wgd, wud = to_dev(gpu, x), to_dev(gpu, wg), to_dev(gpu, wu)
    jc = llk.JitCache()
    fn = jc.lookup_or_compile_str(f"llk_{hash(module) & 0xffff}_M{M}_N{N}_K{K}", module)
    y = gpu.empty((M, N), dtype=gpu.bfloat16, device="cuda")
    fn(xd, wgd, wud, y, y)
    assert_parity_bf16(from_dev(y), orc.swiglu(x, wg, wu)[0], "string-keyed KernelFn")
    jc.close()


@pytest.mark.parametrize("M,K,N,ldw", [(1, 1024, 768, 768), (8, 2048, 1000, 1008),
                                       (33, 640, 600, 603), (64, 4096, 512, 512),
                                       (100, 1280, 1376, 1376), (128, 576, 392, 400),
                                       (129, 576, 392, 392)])
def test_kernel_fn_rowmajor_matches_packed(llk, gpu, orc, M, K, N, ldw):
    """Device weights and at most 128 rows of X: the KernelFn reads the
    caller's row-major weights (rows of ldw elements, ldw % 8 == 0) straight
    into the decode tile kernel, without a pack; its result equals
    llk_swiglu_bf16's on packed weights bit for bit (the same launch) and the
    oracle to the bar.  A stride the row-major loads cannot take (ldw % 8 !=
    0) and M > 128 pack first, with the same result."""
    print(f"case kernel_fn row-major M={M} K={K} N={N} ldw={ldw}", flush=True)
    x, wg, wu = swiglu_inputs(M, K, N, seed=M + K)
    xd = to_dev(gpu, x)
    wgd, wud = to_dev(gpu, wg, ldw), to_dev(gpu, wu, ldw)
    y = gpu.full((M, N), float("nan"), dtype=gpu.bfloat16, device="cuda")
    mx, my = _memref(xd.data_ptr(), M, K, K), _memref(y.data_ptr(), M, N, N)
    mg, mu = _memref(wgd.data_ptr(), K, N, ldw), _memref(wud.data_ptr(), K, N, ldw)
    _call(llk, mx, mg, mu, my)
    got = from_dev(y)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    packed = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    assert np.array_equal(got, packed), "KernelFn differs from the packed path"
    assert_parity_bf16(got, orc.swiglu(x, wg, wu)[0], f"KernelFn row-major M={M}")


@pytest.mark.parametrize("M,S", [(8, 0), (40, 3), (100, 0), (200, 0), (600, 0), (300, 5)])
def test_kernel_fn_rowmajor_matmul_entry(llk, gpu, orc, M, S):
    """The object-code level's matmul KernelFn (fp32 key, result = init + x
    wg) on device weights (row-major, no pack: the decode tile kernel's form
    up to 128 rows, the tile kernel's accumulating form above) and on host
    weights (packed per call): the same bits, on the oracle's bar; with a k
    split forced (S = 3 on the decode tile kernel, 5 on the tile kernel: the
    reduce adds init)."""
    print(f"case kernel_fn row-major matmul M={M} S={S}", flush=True)
    K, N = 1536, 700
    a = normal_bf16(91, M, (M, K))
    b = normal_bf16(91, K, (K, N), 1.0 / np.sqrt(K))
    ad, bd = to_dev(gpu, a), to_dev(gpu, b)
    b_host = np.ascontiguousarray(b)
    jc = llk.JitCache()
    mm = jc.lookup_or_compile(llk.KernelKey(operation=3, isa=7, N=N, K=K, output_type=2))
    init = gpu.randn((M, N), dtype=gpu.float32, device="cuda")
    knob = "decode_splits" if M <= 128 else "tile_splits"
    old = llk.get_tunable(knob)
    llk.set_tunable(knob, S)
    try:
        c_dev = gpu.full((M, N), float("nan"), dtype=gpu.float32, device="cuda")
        mm(ad, bd, None, init, c_dev)
        c_host = gpu.full((M, N), float("nan"), dtype=gpu.float32, device="cuda")
        mm(ad, b_host, None, init, c_host)
    finally:
        llk.set_tunable(knob, old)
        jc.close()
    assert np.array_equal(from_dev(c_dev), from_dev(c_host))
    ref, _ = orc.gemm(a, b)
    assert_parity(from_dev(c_dev), ref + from_dev(init), f"matmul KernelFn row-major M={M}")


@pytest.mark.parametrize("M,S", [(24, 5), (96, 3)])
def test_kernel_fn_rowmajor_split_matches_packed(llk, gpu, orc, M, S):
    """A forced k split on the row-major path (partial planes and the
    split-order reduce) gives the packed path's bits at the same split."""
    print(f"case kernel_fn row-major split M={M} S={S}", flush=True)
    K, N = 1280, 720
    x, wg, wu = swiglu_inputs(M, K, N, seed=M + S)
    xd, wgd, wud = to_dev(gpu, x), to_dev(gpu, wg), to_dev(gpu, wu)
    y = gpu.full((M, N), float("nan"), dtype=gpu.bfloat16, device="cuda")
    mx, my = _memref(xd.data_ptr(), M, K, K), _memref(y.data_ptr(), M, N, N)
    mg, mu = _memref(wgd.data_ptr(), K, N, N), _memref(wud.data_ptr(), K, N, N)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    old = llk.get_tunable("decode_splits")
    llk.set_tunable("decode_splits", S)
    try:
        assert llk.describe_launch("fused_swiglu", M, N, K)["splits"] == S
        _call(llk, mx, mg, mu, my)
        got = from_dev(y)
        packed = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    finally:
        llk.set_tunable("decode_splits", old)
    assert np.array_equal(got, packed)
    assert_parity_bf16(got, orc.swiglu(x, wg, wu)[0], f"KernelFn row-major M={M} S={S}")


@pytest.fixture
def tile_knobs(llk):
    """Sets dispatcher knobs for one test and restores them after it."""
    saved = {}

    def set_(**kw):
        for k, v in kw.items():
            saved.setdefault(k, llk.get_tunable(k))
            llk.set_tunable(k, v)
    yield set_
    for k, v in saved.items():
        llk.set_tunable(k, v)


@pytest.mark.parametrize("M,K,N,ldw,wide", [
    (129, 576, 392, 392, True), (200, 1024, 1000, 1000, True), (257, 640, 1400, 1400, True),
    (300, 2048, 1408, 1416, True), (600, 1024, 1000, 1000, False), (2304, 1024, 4096, 4096, False)])
def test_kernel_fn_rowmajor_tile_matches_packed(llk, gpu, orc, tile_knobs, M, K, N, ldw, wide):
    """Above 128 rows, device weights with K % 64 == 0 and N % 8 == 0: the
    KernelFn runs the 128-column tile kernel's row-major form on the
    caller's [K, N] weights (rows of ldw elements), with that kernel's plan
    -- k splits, and at M = 2304 x N = 4096 an unsplit head of 28 n-blocks
    and a 2-way split tail.  Its result equals llk_swiglu_bf16's on packed
    weights bit for bit: against the 128-column kernel's own plan, and (wide)
    against the default plan, whose wide tiles give the same bits at the
    same split count; and the oracle to the bar."""
    print(f"case kernel_fn row-major tile M={M} K={K} N={N} ldw={ldw}", flush=True)
    if not wide:
        tile_knobs(tile_wide=0)
    x, wg, wu = swiglu_inputs(M, K, N, seed=M + N)
    xd = to_dev(gpu, x)
    wgd, wud = to_dev(gpu, wg, ldw), to_dev(gpu, wu, ldw)
    y = gpu.full((M, N), float("nan"), dtype=gpu.bfloat16, device="cuda")
    mx, my = _memref(xd.data_ptr(), M, K, K), _memref(y.data_ptr(), M, N, N)
    mg, mu = _memref(wgd.data_ptr(), K, N, ldw), _memref(wud.data_ptr(), K, N, ldw)
    _call(llk, mx, mg, mu, my)
    got = from_dev(y)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    packed = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    assert np.array_equal(got, packed), "KernelFn differs from the packed path"
    if M * N <= 600 * 1408:
        assert_parity_bf16(got, orc.swiglu(x, wg, wu)[0], f"KernelFn row-major tile M={M}")


@pytest.mark.parametrize("M", [64, 300])
def test_kernel_fn_rowmajor_off_packs(llk, gpu, orc, tile_knobs, M):
    """kernel_fn_rowmajor = 0: the KernelFn packs the weights on every call
    instead, with the same bits as the row-major forms (the 128-column plan
    on both sides at M = 300)."""
    print(f"case kernel_fn row-major off M={M}", flush=True)
    K, N = 1024, 1000
    tile_knobs(tile_wide=0)
    x, wg, wu = swiglu_inputs(M, K, N, seed=M + 5)
    xd, wgd, wud = to_dev(gpu, x), to_dev(gpu, wg), to_dev(gpu, wu)
    mx, mg, mu = (_memref(xd.data_ptr(), M, K, K), _memref(wgd.data_ptr(), K, N, N),
                  _memref(wud.data_ptr(), K, N, N))
    outs = []
    for on in (1, 0):
        tile_knobs(kernel_fn_rowmajor=on)
        y = gpu.full((M, N), float("nan"), dtype=gpu.bfloat16, device="cuda")
        _call(llk, mx, mg, mu, _memref(y.data_ptr(), M, N, N))
        outs.append(from_dev(y))
    assert np.array_equal(outs[0], outs[1])
    assert_parity_bf16(outs[1], orc.swiglu(x, wg, wu)[0], f"KernelFn packed M={M}")


@pytest.mark.parametrize("M,S", [(300, 3), (520, 7)])
def test_kernel_fn_rowmajor_tile_split_matches_packed(llk, gpu, orc, tile_knobs, M, S):
    """A forced k split on the row-major tile path (partial planes, the
    split-order reduce) gives the packed 128-column kernel's bits at the
    same split."""
    print(f"case kernel_fn row-major tile split M={M} S={S}", flush=True)
    K, N = 1280, 720
    tile_knobs(tile_wide=0, tile_splits=S)
    assert llk.describe_launch("fused_swiglu", M, N, K)["splits"] == S
    x, wg, wu = swiglu_inputs(M, K, N, seed=M + S)
    xd, wgd, wud = to_dev(gpu, x), to_dev(gpu, wg), to_dev(gpu, wu)
    y = gpu.full((M, N), float("nan"), dtype=gpu.bfloat16, device="cuda")
    mx, my = _memref(xd.data_ptr(), M, K, K), _memref(y.data_ptr(), M, N, N)
    mg, mu = _memref(wgd.data_ptr(), K, N, N), _memref(wud.data_ptr(), K, N, N)
    _call(llk, mx, mg, mu, my)
    got = from_dev(y)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    packed = from_dev(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16))
    assert np.array_equal(got, packed)
    assert_parity_bf16(got, orc.swiglu(x, wg, wu)[0], f"KernelFn row-major tile M={M} S={S}")


def test_kernel_fn_rowmajor_tile_config3(llk, gpu):
    """Config 3 at full size (M = 2048, K = 4096, N = 11008) through the
    KernelFn on row-major device weights: bit for bit llk_swiglu_bf16's
    result on packed weights (the wide kernel, unsplit, whose bits are the
    128-column kernel's)."""
    print("case kernel_fn row-major tile config 3", flush=True)
    M, K, N = 2048, 4096, 11008
    g = gpu.Generator(device="cuda")
    g.manual_seed(3)
    xd = gpu.randn((M, K), generator=g, device="cuda").to(gpu.bfloat16)
    wgd = (gpu.randn((K, N), generator=g, device="cuda") / 64).to(gpu.bfloat16)
    wud = (gpu.randn((K, N), generator=g, device="cuda") / 64).to(gpu.bfloat16)
    y = gpu.full((M, N), float("nan"), dtype=gpu.bfloat16, device="cuda")
    mx, my = _memref(xd.data_ptr(), M, K, K), _memref(y.data_ptr(), M, N, N)
    mg, mu = _memref(wgd.data_ptr(), K, N, N), _memref(wud.data_ptr(), K, N, N)
    _call(llk, mx, mg, mu, my)
    pg, pu = llk.PackedWeights.from_device(wgd), llk.PackedWeights.from_device(wud)
    ref = llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.bfloat16)
    assert gpu.equal(y, ref)
    assert not gpu.isnan(y.float()).any()


@pytest.mark.parametrize("M", [100, 300])
def test_object_code_swiglu_fp32_rowmajor(llk, gpu, orc, M):
    """The object-code level's SwiGLU entry with an fp32 result key on device
    weights (row-major: the decode tile kernel's form at M = 100, the tile
    kernel's at M = 300) and on host weights (packed per call): the same
    bits, and the oracle's fp32 result to the bar."""
    print(f"case object-code SwiGLU fp32 row-major M={M}", flush=True)
    K, N = 1024, 720
    x, wg, wu = swiglu_inputs(M, K, N, seed=M + 11)
    xd, wgd, wud = to_dev(gpu, x), to_dev(gpu, wg), to_dev(gpu, wu)
    jc = llk.JitCache()
    try:
        fn = jc.lookup_or_compile(llk.KernelKey(operation=0, isa=7, N=N, K=K, output_type=2))
        y_dev = gpu.full((M, N), float("nan"), dtype=gpu.float32, device="cuda")
        fn(xd, wgd, wud, y_dev, y_dev)
        y_host = gpu.full((M, N), float("nan"), dtype=gpu.float32, device="cuda")
        fn(xd, np.ascontiguousarray(wg), np.ascontiguousarray(wu), y_host, y_host)
    finally:
        jc.close()
    assert np.array_equal(from_dev(y_dev), from_dev(y_host))
    assert_parity(from_dev(y_dev), orc.swiglu(x, wg, wu)[0], f"SwiGLU fp32 KernelFn M={M}")
