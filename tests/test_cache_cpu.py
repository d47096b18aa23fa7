"""Kernel / weight cache and the serialized packed-weights format, on the CPU.

The LRU cases restate the reference's own cache tests
(test/Execution/cache_eviction.cpp:16-116, jit_cache_hit.cpp:74-140,
jit_cache_miss.cpp:15-70) against llk_cache_*; packed-weight handles are
host-only (no GPU)."""
from __future__ import annotations

import ctypes as C
import struct
import threading

import numpy as np
import pytest

import dslcompiler_amd as llk
from dslcompiler_amd import JitCache, KernelKey, WeightKey
from dslcompiler_amd._lib import lib

from common import normal_bf16


def _host_pw(K=70, N=150, bk=64, seed=1):
    w = normal_bf16(seed, 1, (K, N))
    return w, llk.PackedWeights.from_host(w, bk, host_only=True)


# ---- cache_eviction.cpp -----------------------------------------------------

def test_l1_hit_and_miss():
    c = JitCache()
    c.insert_ir("key1", "ir_module_string_1")
    c.insert_ir("key2", "ir_module_string_2")
    assert c.lookup_ir("key1") == "ir_module_string_1"
    assert c.lookup_ir("key2") == "ir_module_string_2"
    assert c.lookup_ir("key3") is None


def test_lru_eviction_beyond_capacity():
    c = JitCache()
    c.set_max_entries(1, 2)
    for k in "abc":
        c.insert_ir(k, "value_" + k)
    assert c.lookup_ir("a") is None
    assert c.lookup_ir("b") == "value_b"
    assert c.lookup_ir("c") == "value_c"


def test_lru_access_updates_recency():
    c = JitCache()
    c.set_max_entries(1, 2)
    c.insert_ir("a", "value_a")
    c.insert_ir("b", "value_b")
    c.lookup_ir("a")  # a becomes most recently used
    c.insert_ir("c", "value_c")  # evicts b
    assert c.lookup_ir("a") == "value_a"
    assert c.lookup_ir("b") is None
    assert c.lookup_ir("c") == "value_c"


def test_l2_optimized():
    c = JitCache()
    c.insert_optimized_mlir("opt_key", "optimized_mlir_module")
    assert c.lookup_optimized_mlir("opt_key") == "optimized_mlir_module"
    assert c.lookup_ir("opt_key") is None  # levels are separate


def test_l4_packed_weight_cache():
    c = JitCache()
    _, pw = _host_pw()
    raw = pw.handle.value
    key = WeightKey(0xDEADBEEF, 12345, 64, 64)
    c.insert_packed_weights(key, pw)
    got = c.lookup_packed_weights(key)
    assert got is not None and got.handle.value == raw
    assert (got.N, got.K_blocks, got.BK) == (150, 2, 64)
    assert c.lookup_packed_weights(WeightKey(0xDEADBEEF, 12345, 64, 128)) is None


def test_l4_reinsert_same_handle_refreshes():
    """Inserting the handle a key already holds (C ABI, raw handle) only
    refreshes the entry: the handle stays valid, and clearing the cache
    frees it once (a second owner would free it twice)."""
    c = JitCache()
    _, pw = _host_pw()
    raw = pw.release()
    key = WeightKey(0x5150, 7, 64, 128)
    for _ in range(3):
        assert lib().llk_cache_insert_packed_weights(c._c, C.byref(key.c()), raw) == 0
    got = c.lookup_packed_weights(key)
    assert got is not None and got.handle.value == raw.value and got.N == 150
    assert c.size() == 1
    c.clear()
    assert c.size() == 0 and c.lookup_packed_weights(key) is None


def test_stats_accumulate():
    c = JitCache()
    c.lookup_ir("nonexistent")
    c.insert_ir("stats_key", "data")
    c.lookup_ir("stats_key")
    s = c.stats()
    assert s["hits"][0] == 1 and s["misses"][0] == 1
    assert s["hits"][1:] == [0, 0, 0] and s["misses"][1:] == [0, 0, 0]


def test_clear_removes_all_entries():
    c = JitCache()
    c.insert_ir("k1", "v1")
    c.insert_optimized_mlir("k2", "v2")
    _, pw = _host_pw()
    c.insert_packed_weights(WeightKey(1, 2, 3, 4), pw)
    assert c.size() == 3
    c.clear()
    assert c.lookup_ir("k1") is None and c.lookup_optimized_mlir("k2") is None
    assert c.size() == 0


# ---- jit_cache_hit.cpp / jit_cache_miss.cpp --------------------------------

def test_object_code_miss_then_sentinel_hit():
    c = JitCache()
    key = KernelKey(M_bucket=0, N=4096, K=4096)
    assert c.lookup_object_code(key) is None
    c.insert_object_code(key, 0xDEADBEEF)
    for _ in range(2):
        got = c.lookup_object_code(key)
        assert got is not None and got.address == 0xDEADBEEF


def test_different_kernel_keys_are_separate():
    c = JitCache()
    ka = KernelKey(M_bucket=0, N=4096, K=4096)
    kb = KernelKey(M_bucket=4, N=4096, K=4096)
    c.insert_object_code(ka, 0xAAA)
    c.insert_object_code(kb, 0xBBB)
    assert c.lookup_object_code(ka).address == 0xAAA
    assert c.lookup_object_code(kb).address == 0xBBB
    assert ka.hash() != kb.hash()


def test_l1_miss_on_new_key():
    c = JitCache()
    assert c.lookup_ir("new_module_v1") is None
    c.insert_ir("new_module_v1", "module_content_v1")
    assert c.lookup_ir("new_module_v1") == "module_content_v1"
    assert c.lookup_ir("new_module_v2") is None


# ---- LRU details of the reference CacheLevel (JitCache.cpp:41-88, 332-363) --

def test_replace_existing_refreshes_without_eviction():
    c = JitCache()
    c.set_max_entries(1, 2)
    c.insert_ir("a", "1")
    c.insert_ir("b", "2")
    c.insert_ir("a", "3")  # replace: a is now most recent, nothing evicted
    assert c.stats()["evictions"][0] == 0
    c.insert_ir("c", "4")  # evicts b
    assert c.lookup_ir("a") == "3" and c.lookup_ir("b") is None
    assert c.stats()["evictions"][0] == 1


def test_evict_lru_trims_and_sets_capacity():
    c = JitCache()
    for i in range(10):
        c.insert_optimized_mlir(f"k{i}", str(i))
    c.evict_lru(2, 3)  # keeps the 3 most recent
    assert [c.lookup_optimized_mlir(f"k{i}") for i in range(10)] == [None] * 7 + ["7", "8", "9"]
    assert c.stats()["evictions"][1] == 7
    c.insert_optimized_mlir("x", "x")  # capacity is now 3
    assert c.size() == 3
    c.set_max_entries(2, 0)  # capacity 0: an insert still leaves one entry
    c.insert_optimized_mlir("y", "y")
    assert c.size() == 1 and c.lookup_optimized_mlir("y") == "y"


def test_bad_level_is_an_error():
    c = JitCache()
    with pytest.raises(llk.LLKError, match="INVALID_ARGUMENT"):
        c.evict_lru(5, 1)
    with pytest.raises(llk.LLKError, match="INVALID_ARGUMENT"):
        c._insert(3, "k", "v")


def test_l4_eviction_frees_and_misses():
    c = JitCache()
    c.set_max_entries(4, 2)
    for i in range(3):
        _, pw = _host_pw(seed=i + 1)
        c.insert_packed_weights(WeightKey(0x1000 + i, i, 64, 128), pw)
    assert c.lookup_packed_weights(WeightKey(0x1000, 0, 64, 128)) is None
    assert c.lookup_packed_weights(WeightKey(0x1002, 2, 64, 128)) is not None
    assert c.stats()["evictions"][3] == 1


def test_get_packed_weights_host_hits_on_same_buffer():
    c = JitCache()
    w = normal_bf16(3, 1, (130, 200))
    a = c.get_packed_weights(w, 64, host_only=True)
    b = c.get_packed_weights(w, 64, host_only=True)
    assert a.handle.value == b.handle.value
    d = c.get_packed_weights(w, 32, host_only=True)  # BK is part of the key
    assert d.handle.value != a.handle.value and d.BK == 32
    s = c.stats()
    assert (s["hits"][3], s["misses"][3]) == (1, 2)
    ref = llk.PackedWeights.from_host(w, 64, host_only=True)
    assert np.array_equal(a.host_data(), ref.host_data())


# ---- lookupOrCompile -------------------------------------------------------

def test_lookup_or_compile_selects_entries():
    """gfx950 keys resolve to entries of their operation's code object (read
    and checked here; loaded on a device at first call), one per (object,
    output type), cached in L3: the KernelFn shape (MemRef2D) from
    lookup_or_compile, the packed-handle shape of the same L3 entry from
    lookup_or_compile_packed."""
    c = JitCache()
    sw = KernelKey(operation=0, isa=7, N=11008, K=4096, M_bucket=4, weight_layout=2)
    mm = KernelKey(operation=3, isa=7, N=4096, K=4096, M_bucket=4, output_type=2)
    f1 = c.lookup_or_compile(sw)
    f2 = c.lookup_or_compile(mm)
    p1 = c.lookup_or_compile_packed(sw)
    lib_fn = C.cast(lib().llk_swiglu_kernel_fn, C.c_void_p).value
    swiglu_addr = C.cast(lib().llk_swiglu_bf16, C.c_void_p).value
    assert len({f1.address, f2.address, p1.address, lib_fn, swiglu_addr, 0}) == 6
    assert c.lookup_or_compile(sw).address == f1.address  # L3 hit
    assert c.lookup_object_code(sw).address == p1.address
    s = c.stats()
    assert (s["hits"][2], s["misses"][2]) == (3, 2)
    # another key of the same object and output type shares the entry
    assert JitCache().lookup_or_compile(KernelKey(operation=0, isa=7, N=64, K=64)).address == \
        f1.address
    # a matmul key may ask for f16 (llk.matmul's result types); SwiGLU may not
    assert c.lookup_or_compile(KernelKey(operation=3, isa=7, N=64, K=64, output_type=1)).address
    with pytest.raises(llk.LLKError, match="DTYPE"):
        c.lookup_or_compile(KernelKey(operation=0, isa=7, N=64, K=64, output_type=1))


SWIGLU_MODULE = """
func.func @swiglu(%x: tensor<4x8xbf16>, %wg: tensor<8x16xbf16>, %wu: tensor<8x16xbf16>,
                  %init: tensor<4x16xbf16>) -> tensor<4x16xbf16> {
  %0 = llk.fused_swiglu ins(%x, %wg, %wu : tensor<4x8xbf16>, tensor<8x16xbf16>,
                            tensor<8x16xbf16>) outs(%init : tensor<4x16xbf16>)
       -> tensor<4x16xbf16>
  return %0 : tensor<4x16xbf16>
}
"""
MATMUL_F32_MODULE = """
func.func @mm(%a: tensor<4x8xbf16>, %b: tensor<8x16xbf16>, %c: tensor<4x16xf32>) -> tensor<4x16xf32> {
  %0 = llk.matmul ins(%a, %b : tensor<4x8xbf16>, tensor<8x16xbf16>) outs(%c : tensor<4x16xf32>)
       -> tensor<4x16xf32>
  return %0 : tensor<4x16xf32>
}
"""


def test_lookup_or_compile_string_key():
    """The string-keyed overload (JitCache.h:103-105) that llk-compile uses:
    the module's first llk op picks the code object and output type, the
    entry is cached under the caller's key, a repeat of the key hits L3
    without reading the module, and a module with no llk op is the
    reference's "No exported kernel entry point" error (JitCache.cpp:
    214-220) with nothing inserted."""
    c = JitCache()
    sw_key = KernelKey(operation=0, isa=7, N=16, K=8)
    f_sw = c.lookup_or_compile_str("llk_1_M4_N16_K8", SWIGLU_MODULE)
    assert f_sw.address == c.lookup_or_compile(sw_key).address  # same (object, bf16) entry
    f_mm = c.lookup_or_compile_str("llk_2_M4_N16_K8", MATMUL_F32_MODULE)
    assert f_mm.address == c.lookup_or_compile(KernelKey(operation=3, isa=7, N=16, K=8,
                                                         output_type=2)).address
    assert f_mm.address != f_sw.address
    n = c.size()
    assert c.lookup_or_compile_str("llk_1_M4_N16_K8", "not read on a hit").address == f_sw.address
    assert c.stats()["hits"][2] >= 1 and c.size() == n
    with pytest.raises(llk.LLKError, match="No exported kernel entry point found in module"):
        c.lookup_or_compile_str("llk_3", "func.func @f() { return }")
    with pytest.raises(llk.LLKError, match="DTYPE"):
        c.lookup_or_compile_str("llk_4", SWIGLU_MODULE.replace("x8xbf16>, tensor<8x16", "x8xf32>, tensor<8x16", 1))
    assert c.size() == n


def test_get_packed_weights_single_flight_threads():
    """8 threads miss on one key at once (host-only packs of a 2048 x 2048
    matrix, ~10 ms each, the GIL released in the C call): one pack, one
    handle for all, one L4 entry; counted references survive a clear."""
    w = normal_bf16(91, 1, (2048, 2048))
    c = JitCache()
    got, start = [None] * 8, threading.Barrier(8)

    def run(i):
        start.wait()
        got[i] = c.get_packed_weights(w, 64, host_only=True).handle.value

    th = [threading.Thread(target=run, args=(i,)) for i in range(8)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert len(set(got)) == 1 and got[0]
    assert c.size() == 1 and c.stats()["evictions"][3] == 0
    ref = c.acquire_packed_weights(w, 64, host_only=True)
    assert ref.handle.value == got[0]
    c.clear()
    assert c.size() == 0
    assert np.array_equal(ref.host_data(),
                          llk.PackedWeights.from_host(w, 64, host_only=True).host_data())
    c.release_packed_weights(ref)
    with pytest.raises(llk.LLKError, match="no reference"):
        c.release_packed_weights(ref)


@pytest.mark.parametrize("kw,match", [
    (dict(isa=0), "UNSUPPORTED_ARCH"),
    (dict(isa=7, operation=1), "INVALID_ARGUMENT"),
    (dict(isa=7, operation=2), "INVALID_ARGUMENT"),
    (dict(isa=7, input_type=2), "DTYPE"),
    (dict(isa=7, output_type=1), "DTYPE"),
    (dict(isa=7, N=0), "INVALID_ARGUMENT"),
])
def test_lookup_or_compile_rejects(kw, match):
    c = JitCache()
    key = KernelKey(N=64, K=64)
    for k, v in kw.items():
        setattr(key, k, v)
    with pytest.raises(llk.LLKError, match=match):
        c.lookup_or_compile(key)
    assert c.size() == 0


def test_concurrent_use_is_consistent():
    """Threads hammer one level (ctypes releases the GIL during calls)."""
    c = JitCache()
    c.set_max_entries(1, 64)
    n_threads, per = 8, 400

    def work(t):
        for i in range(per):
            k = f"k{(t * 7 + i) % 100}"
            if c.lookup_ir(k) is None:
                c.insert_ir(k, k * 3)
            else:
                assert c.lookup_ir(k) in (None, k * 3)

    th = [threading.Thread(target=work, args=(t,)) for t in range(n_threads)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    s = c.stats()
    assert c.size() <= 64
    assert s["hits"][0] + s["misses"][0] >= n_threads * per


# ---- serialized packed weights ---------------------------------------------

@pytest.mark.parametrize("K,N,bk", [(70, 150, 64), (4096, 256, 64), (1, 1, 32), (200, 129, 48)])
def test_blob_roundtrip_host(K, N, bk):
    w, pw = _host_pw(K, N, bk, seed=K + N)
    blob = pw.serialize()
    magic, version, dtype, k, n, bk2, kblk, bsz, KB, NB, nbytes, csum, res = struct.unpack(
        "<8sIIqqqqqqqQQQ", blob[:96])
    assert magic == b"LLKPW950" and version == 1 and dtype == 0 and res == 0
    assert (k, n, bk2, kblk, bsz) == (K, N, bk, -(-K // bk), bk * N * 2)
    assert (KB, NB) == (-(-K // 64), -(-N // 128)) and nbytes == len(blob) - 96
    assert np.array_equal(np.frombuffer(blob[96:], np.uint8), llk.pack_device_layout(w))
    back = llk.PackedWeights.from_blob(blob, host_only=True)
    assert (back.K, back.N, back.BK, back.K_blocks, back.block_size) == (
        pw.K, pw.N, pw.BK, pw.K_blocks, pw.block_size)
    assert np.array_equal(back.host_data(), pw.host_data())
    assert back.serialize() == blob


def test_blob_file_roundtrip(tmp_path):
    w, pw = _host_pw(300, 260, 64, seed=9)
    p = tmp_path / "w.llkpw"
    pw.save(p)
    back = llk.PackedWeights.load(p, host_only=True)
    assert np.array_equal(back.host_data(), pw.host_data())
    assert p.stat().st_size == 96 + llk.lib().llk_pack_device_bytes(300, 260)


def test_blob_empty_matrix():
    pw = llk.PackedWeights.from_host(np.zeros((0, 5), np.uint16), 64, host_only=True)
    blob = pw.serialize()
    assert len(blob) == 96
    back = llk.PackedWeights.from_blob(blob, host_only=True)
    assert (back.K, back.N, back.K_blocks) == (0, 5, 0)


def test_blob_rejects_corruption(tmp_path):
    _, pw = _host_pw()
    blob = bytearray(pw.serialize())
    bad = bytearray(blob)
    bad[200] ^= 1
    with pytest.raises(llk.LLKError, match="checksum"):
        llk.PackedWeights.from_blob(bytes(bad), host_only=True)
    with pytest.raises(llk.LLKError, match="truncated"):
        llk.PackedWeights.from_blob(bytes(blob[:-1]), host_only=True)
    bad = bytearray(blob)
    bad[0:8] = b"XXXXXXXX"
    with pytest.raises(llk.LLKError, match="version-1"):
        llk.PackedWeights.from_blob(bytes(bad), host_only=True)
    bad = bytearray(blob)
    bad[48:56] = struct.pack("<q", 3)  # K_blocks inconsistent with K, BK
    with pytest.raises(llk.LLKError, match="inconsistent"):
        llk.PackedWeights.from_blob(bytes(bad), host_only=True)
    with pytest.raises(llk.LLKError, match="NOT_FOUND"):
        llk.PackedWeights.load(tmp_path / "missing.llkpw", host_only=True)
