"""GPU side of the kernel / weight cache and the packed-weights blob: entry
points from lookupOrCompile launch the same kernels as the direct C-ABI
calls (bit-identical outputs), device-resident weights are cached by buffer,
and a blob restores a device handle whose results are bit-identical."""
from __future__ import annotations

import numpy as np
import pytest

from common import normal_bf16, swiglu_inputs
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu


def test_lookup_or_compile_entries_run_on_gpu(llk, gpu):
    print("case cache entry points", flush=True)
    M, K, N = 300, 512, 640
    x, wg, wu = swiglu_inputs(M, K, N, seed=5)
    pg, pu = llk.PackedWeights.from_host(wg), llk.PackedWeights.from_host(wu)
    xd = to_dev(gpu, x)
    cache = llk.JitCache()
    sw = cache.lookup_or_compile_packed(llk.KernelKey(operation=0, isa=7, N=N, K=K, M_bucket=4,
                                                      weight_layout=2))
    mm = cache.lookup_or_compile_packed(llk.KernelKey(operation=3, isa=7, N=N, K=K, M_bucket=4,
                                                      weight_layout=2, output_type=2))
    y = gpu.empty((M, N), dtype=gpu.bfloat16, device="cuda")
    sw(xd, pg, pu, y)
    c = gpu.empty((M, N), dtype=gpu.float32, device="cuda")
    mm(xd, pg, None, c)
    gpu.cuda.synchronize()
    assert np.array_equal(from_dev(y), from_dev(llk.fused_swiglu(xd, pg, pu)))
    assert np.array_equal(from_dev(c), from_dev(llk.matmul(xd, pg, out_dtype=gpu.float32)))


def test_device_weights_cached_by_buffer(llk, gpu):
    print("case cache device weights", flush=True)
    K, N = 256, 384
    w = to_dev(gpu, normal_bf16(6, 1, (K, N), 1 / 16))
    cache = llk.JitCache()
    a = cache.get_packed_weights(w, 64)
    b = cache.get_packed_weights(w, 64)
    assert a.handle.value == b.handle.value
    assert cache.stats()["hits"][3] == 1
    fresh = llk.PackedWeights.from_device(w)
    x = to_dev(gpu, normal_bf16(6, 0, (70, K)))
    assert np.array_equal(from_dev(llk.matmul(x, a, out_dtype=gpu.float32)),
                          from_dev(llk.matmul(x, fresh, out_dtype=gpu.float32)))
    cache.close()  # frees the cached handle


@pytest.mark.parametrize("keep_host", [False, True])
def test_blob_restores_device_handle(llk, gpu, tmp_path, keep_host):
    print(f"case blob device keep_host={keep_host}", flush=True)
    M, K, N = 40, 1000, 333
    x, wg, wu = swiglu_inputs(M, K, N, seed=8)
    pg = llk.PackedWeights.from_host(wg, keep_host=True)
    pu = llk.PackedWeights.from_device(to_dev(gpu, wu))
    blob = pg.serialize()  # payload copied back from the GPU
    assert np.array_equal(np.frombuffer(blob[96:], np.uint8), llk.pack_device_layout(wg))
    pu.save(tmp_path / "wu.llkpw")
    pg2 = llk.PackedWeights.from_blob(blob, keep_host=keep_host)
    pu2 = llk.PackedWeights.load(tmp_path / "wu.llkpw", keep_host=keep_host)
    if keep_host:
        assert np.array_equal(pg2.host_data(), pg.host_data())
    xd = to_dev(gpu, x)
    y1 = from_dev(llk.fused_swiglu(xd, pg, pu))
    y2 = from_dev(llk.fused_swiglu(xd, pg2, pu2))
    assert np.array_equal(y1, y2)
