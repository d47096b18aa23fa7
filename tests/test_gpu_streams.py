"""Stream and graph behaviour: concurrent launches on two streams with their
own scratch buffers and with the library's workspace (one per stream), and
HIP-graph capture + replay of SwiGLU / MLP calls (every replay checked
against the eager result, with eager work between)."""
from __future__ import annotations

import numpy as np
import pytest

from common import assert_parity, assert_parity_bf16, bf16_bits_to_f32, normal_bf16, swiglu_inputs
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu


def test_two_streams_own_scratch(llk, gpu):
    print("case two streams", flush=True)
    cases = [(300, 2048, 1000), (8, 4096, 2000)]  # tile with splits; small-M with splits
    data = []
    for M, K, N in cases:
        x, wg, wu = swiglu_inputs(M, K, N, seed=M)
        pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
        xd = to_dev(gpu, x)
        ref = from_dev(llk.fused_swiglu(xd, pg, pu))
        data.append((xd, pg, pu, ref))
    gpu.cuda.synchronize()
    old = llk.get_tunable("tile_splits"), llk.get_tunable("decode_splits")
    llk.set_tunable("tile_splits", 3)
    llk.set_tunable("decode_splits", 3)
    try:
        streams = [gpu.cuda.Stream(), gpu.cuda.Stream()]
        outs = []
        for (xd, pg, pu, ref), s in zip(data, streams):
            need = max(llk.describe_launch("fused_swiglu", xd.shape[0], pg.N, pg.K)
                       ["workspace_bytes"], 256)
            scratch = gpu.empty(need, dtype=gpu.uint8, device="cuda")
            ys = []
            with gpu.cuda.stream(s):
                for _ in range(20):
                    ys.append(llk.fused_swiglu(xd, pg, pu, stream=s, scratch=scratch))
            outs.append((ys, ref, scratch))
        gpu.cuda.synchronize()
        for ys, ref, _ in outs:
            for y in ys:
                got = from_dev(y)
                # every run bit-identical; the forced split changes the
                # summation order, so against the unsplit result: the bar
                assert np.array_equal(got, from_dev(ys[0]))
                assert_parity(bf16_bits_to_f32(got), bf16_bits_to_f32(ref), "split vs unsplit")
    finally:
        llk.set_tunable("tile_splits", old[0])
        llk.set_tunable("decode_splits", old[1])


def test_two_streams_library_workspace(llk, gpu, orc):
    """No caller scratch: both streams' k-split launches take their workspace
    from the library, which keeps one per stream, so interleaved launches on
    two streams with different shapes never share partial planes."""
    print("case two streams, library workspace", flush=True)
    cases = [(300, 2048, 1000), (8, 4096, 2000), (255, 5120, 1536)]
    data = []
    for M, K, N in cases:
        x, wg, wu = swiglu_inputs(M, K, N, seed=M + 1)
        pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
        yf_ref, _ = orc.swiglu(x, wg, wu)
        data.append((to_dev(gpu, x), pg, pu, yf_ref))
    gpu.cuda.synchronize()
    old = llk.get_tunable("tile_splits"), llk.get_tunable("decode_splits")
    llk.set_tunable("tile_splits", 3)
    llk.set_tunable("decode_splits", 3)
    try:
        for xd, pg, pu, _ in data:
            assert llk.describe_launch("fused_swiglu", xd.shape[0], pg.N, pg.K)[
                "workspace_bytes"] > 0
        streams = [gpu.cuda.Stream() for _ in data]
        outs = [[] for _ in data]
        for _ in range(20):
            for i, ((xd, pg, pu, _), s) in enumerate(zip(data, streams)):
                with gpu.cuda.stream(s):
                    outs[i].append(llk.fused_swiglu(xd, pg, pu, out_dtype=gpu.float32,
                                                    stream=s))
        gpu.cuda.synchronize()
        for ys, (_, _, _, yf_ref) in zip(outs, data):
            first = from_dev(ys[0])
            assert_parity(first, yf_ref, "library workspace vs oracle")
            for y in ys[1:]:
                assert np.array_equal(from_dev(y).view(np.uint32), first.view(np.uint32))
    finally:
        llk.set_tunable("tile_splits", old[0])
        llk.set_tunable("decode_splits", old[1])


@pytest.mark.parametrize("M", [8, 300])
def test_graph_capture_replay(llk, gpu, M):
    """A captured SwiGLU + MLP call replays to the eager result each time."""
    print(f"case graph M={M}", flush=True)
    K, N = 1024, 768
    x, wg, wu = swiglu_inputs(M, K, N, seed=11)
    wd = normal_bf16(12, 3, (N, 512), 1.0 / np.sqrt(N))
    pg, pu, pd = (llk.PackedWeights.from_host(w) for w in (wg, wu, wd))
    xd = to_dev(gpu, x)
    y = gpu.empty((M, N), dtype=gpu.bfloat16, device="cuda")
    y2 = gpu.empty((M, N), dtype=gpu.bfloat16, device="cuda")
    z = gpu.empty((M, pd.N), dtype=gpu.bfloat16, device="cuda")
    s = gpu.cuda.Stream()
    with gpu.cuda.stream(s):  # warm-up on the capture stream: allocates the workspace
        llk.fused_swiglu(xd, pg, pu, out=y, stream=s)
        llk.mlp(xd, pg, pu, pd, y=y2, z=z, stream=s)
    s.synchronize()
    eager_y, eager_z = from_dev(y), from_dev(z)
    g = gpu.cuda.CUDAGraph()
    with gpu.cuda.graph(g, stream=s):
        llk.fused_swiglu(xd, pg, pu, out=y, stream=s)
        llk.mlp(xd, pg, pu, pd, y=y2, z=z, stream=s)
    for rep in range(4):
        y.zero_()
        z.zero_()
        gpu.cuda.synchronize()
        g.replay()
        gpu.cuda.synchronize()
        assert np.array_equal(from_dev(y), eager_y), rep
        assert np.array_equal(from_dev(z), eager_z), rep
        llk.fused_swiglu(xd, pg, pu, out=y2)  # eager work between replays
        gpu.cuda.synchronize()


def test_graph_survives_workspace_growth(llk, gpu):
    """A graph captured while the library's own workspace was in use still
    replays correctly after a later call outgrew that workspace (the library
    retires an outgrown buffer instead of freeing it)."""
    print("case graph + workspace growth", flush=True)
    M, K, N = 300, 1024, 768
    x, wg, wu = swiglu_inputs(M, K, N, seed=21)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x)
    y = gpu.empty((M, N), dtype=gpu.bfloat16, device="cuda")
    old = llk.get_tunable("tile_splits")
    llk.set_tunable("tile_splits", 3)
    try:
        assert llk.describe_launch("fused_swiglu", M, N, K)["workspace_bytes"] > 0
        s = gpu.cuda.Stream()
        with gpu.cuda.stream(s):
            llk.fused_swiglu(xd, pg, pu, out=y, stream=s)
        s.synchronize()
        eager = from_dev(y)
        g = gpu.cuda.CUDAGraph()
        with gpu.cuda.graph(g, stream=s):
            llk.fused_swiglu(xd, pg, pu, out=y, stream=s)
        # a split GEMM whose partial planes (8 x 4096 x 12288 fp32 = 1.6 GB)
        # exceed any earlier workspace by more than the 1.5x growth step
        llk.set_tunable("tile_splits", 8)
        Mb, Kb, Nb = 4096, 4096, 12288
        assert llk.describe_launch("matmul", Mb, Nb, Kb)["workspace_bytes"] >= 1_500_000_000
        a = gpu.randn((Mb, Kb), device="cuda").to(gpu.bfloat16)
        pb = llk.PackedWeights.from_device(gpu.randn((Kb, Nb), device="cuda").to(gpu.bfloat16) * 0.02)
        c = llk.matmul(a, pb)
        gpu.cuda.synchronize()
        assert bool(gpu.isfinite(c).all())
        del a, c, pb
        # memory freed by torch in between is handed out again: fill it
        junk = gpu.full((1 << 28,), 3.0, device="cuda")
        for rep in range(3):
            y.zero_()
            gpu.cuda.synchronize()
            g.replay()
            gpu.cuda.synchronize()
            assert np.array_equal(from_dev(y), eager), rep
        del junk
    finally:
        llk.set_tunable("tile_splits", old)


def test_workspaces_stay_bounded_per_thread_stream(llk, gpu, orc):
    """Threads launching on the per-thread default stream each get a library
    workspace of their own; the library keeps at most max_workspaces of
    them (least recently used freed once its calls are done), every result
    stays right, and llk_workspace_trim frees the idle ones.  Workspaces
    that graphs captured earlier in this process are pinned (never freed):
    the bound is set above what a trim leaves."""
    import ctypes as C
    import threading
    from dslcompiler_amd._lib import KernelContext, tensor2d
    print("case workspaces per thread bounded", flush=True)
    M, K, N = 300, 2048, 640
    x, wg, wu = swiglu_inputs(M, K, N, seed=91)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x)
    ref = orc.swiglu(x, wg, wu)[0]
    old = llk.get_tunable("tile_splits"), llk.get_tunable("max_workspaces")
    gpu.cuda.synchronize()
    llk.workspace_trim()
    pinned = llk.workspace_stats()[0]  # kept for graphs captured by earlier tests
    llk.set_tunable("tile_splits", 3)  # partial planes: a workspace per call
    llk.set_tunable("max_workspaces", pinned + 4)
    L = llk.lib()
    per_thread = 2  # hipStreamPerThread
    ys = [gpu.empty((M, N), dtype=gpu.bfloat16, device="cuda") for _ in range(12)]
    gpu.cuda.synchronize()
    errors, counts = [], []
    lock = threading.Lock()

    def run(i):
        ctx = KernelContext(None, 0, per_thread)
        xt = tensor2d(xd.data_ptr(), M, K)
        yt = tensor2d(ys[i].data_ptr(), M, N)
        for _ in range(3):
            rc = L.llk_swiglu_bf16(C.byref(xt), pg.handle, pu.handle, C.byref(yt), 0, C.byref(ctx))
            if rc:
                errors.append(L.llk_last_error())
                return
        with lock:
            counts.append(llk.workspace_stats()[0])

    try:
        for batch in range(3):  # 4 threads at a time, 12 distinct threads in all
            th = [threading.Thread(target=run, args=(4 * batch + i,)) for i in range(4)]
            for t in th:
                t.start()
            for t in th:
                t.join()
        gpu.cuda.synchronize()
        assert not errors, errors
        assert max(counts) <= pinned + 4, (pinned, counts)
        n, nbytes = llk.workspace_stats()
        assert n <= pinned + 4 and nbytes > 0
        for y in ys:
            assert_parity_bf16(from_dev(y), ref, "per-thread stream, split 3")
        llk.workspace_trim()
        assert llk.workspace_stats()[0] == pinned
    finally:
        llk.set_tunable("tile_splits", old[0])
        llk.set_tunable("max_workspaces", old[1])


def test_accumulate_scratch_sized_from_plan(llk, gpu, orc):
    """llk_describe_launch with LLK_PLAN_ACCUMULATE gives exactly the scratch
    the accumulating GEMM needs (its partial planes exist even unsplit): a
    caller buffer of that size works on the S = 1 tile case (M = 700, N =
    768, K = 384: the plain plan needs no workspace at all), a smaller one is
    LLK_ERR_SCRATCH, and the result equals the library-workspace call bit
    for bit."""
    print("case accumulate scratch from plan", flush=True)
    M, K, N = 700, 384, 768
    x, wb, _ = swiglu_inputs(M, K, N, seed=93)
    xd, pb = to_dev(gpu, x), llk.PackedWeights.from_host(wb)
    plan = llk.describe_launch("matmul", M, N, K, accumulate=True)
    assert plan["splits"] == 1 and plan["workspace_bytes"] >= M * N * 4
    assert llk.describe_launch("matmul", M, N, K)["workspace_bytes"] == 0
    c0 = gpu.randn((M, N), dtype=gpu.float32, device="cuda")
    c_lib = c0.clone()
    llk.matmul(xd, pb, out=c_lib, accumulate=True)
    c_own = c0.clone()
    scratch = gpu.empty(plan["workspace_bytes"], dtype=gpu.uint8, device="cuda")
    llk.matmul(xd, pb, out=c_own, accumulate=True, scratch=scratch)
    gpu.cuda.synchronize()
    assert np.array_equal(from_dev(c_own), from_dev(c_lib))
    ref, _ = orc.gemm(x, wb)
    assert_parity(from_dev(c_own), ref + from_dev(c0), "accumulate with plan-sized scratch")
    small = gpu.empty(plan["workspace_bytes"] - 256, dtype=gpu.uint8, device="cuda")
    with pytest.raises(llk.LLKError, match="SCRATCH"):
        llk.matmul(xd, pb, out=c0.clone(), accumulate=True, scratch=small)
