"""Python view of the four-level kernel / weight cache (llk_cache_* in
include/llk/llk_abi.h), the counterpart of the reference's JitCache
(include/LLK/Runtime/JitCache.h:67-218)."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, fields

import numpy as np

from . import _lib
from ._lib import (KERNEL_FN, MEMREF_FN, CacheStatsC, KernelContext, KernelKeyC, MemRef2D,
                   WeightKeyC, check, lib, tensor2d)
from .ops import PackedWeights, _check_operand, _ctx, _out_dtype_code, _t2d, _torch

# Enum values (KernelKey.h:22-38, plus this backend's additions).
OP_FUSED_SWIGLU, OP_ROPE, OP_ATTENTION, OP_MATMUL = 0, 1, 2, 3
LAYOUT_ROW_MAJOR, LAYOUT_PACKED_KN, LAYOUT_DEVICE = 0, 1, 2
ISA_AVX2, ISA_UNKNOWN, ISA_GFX950 = 0, 6, 7
MATH_STRICT, MATH_BOUNDED_FAST, MATH_UNSAFE_FAST = 0, 1, 2


@dataclass
class KernelKey:
    """KernelKey (KernelKey.h:45-57) with the reference's default values."""
    operation: int = OP_FUSED_SWIGLU
    input_type: int = 0
    output_type: int = 0
    M_bucket: int = 0
    N: int = 0
    K: int = 0
    weight_layout: int = LAYOUT_ROW_MAJOR
    isa: int = ISA_AVX2
    math_mode: int = MATH_BOUNDED_FAST
    thread_count: int = 1
    compiler_version: int = 0
    schedule_version: int = 0

    def c(self) -> KernelKeyC:
        return KernelKeyC(*(getattr(self, f.name) for f in fields(self)))

    def hash(self) -> int:
        return lib().llk_kernel_key_hash(*(getattr(self, f.name) for f in fields(self)))


@dataclass
class WeightKey:
    """WeightKey (KernelKey.h:114-124)."""
    weight_ptr: int = 0
    shape_hash: int = 0
    BK: int = 0
    BN: int = 0

    def c(self) -> WeightKeyC:
        return WeightKeyC(self.weight_ptr or None, self.shape_hash, self.BK, self.BN)


class PackedEntry:
    """An object-code entry in its packed-handle shape (llk_kernel_fn: the
    signature of llk_swiglu_bf16)."""

    def __init__(self, fn: KERNEL_FN):
        self._fn = fn

    @property
    def address(self) -> int:
        return C.cast(self._fn, C.c_void_p).value or 0

    def __call__(self, x, w0: PackedWeights, w1: PackedWeights | None, y, stream=None,
                 scratch=None) -> None:
        torch = _torch()
        _check_operand(x, "x", (torch.bfloat16,))
        _check_operand(y, "y", (torch.bfloat16, torch.float16, torch.float32))
        ctx = _ctx(stream, scratch)
        check(self._fn(C.byref(_t2d(x)), w0.handle, w1.handle if w1 is not None else None,
                       C.byref(_t2d(y)), _out_dtype_code(y.dtype), C.byref(ctx)))


def memref(t) -> MemRef2D:
    """MemRef2D (JitCache.h:43-51) over a 2-D torch tensor (any device) or
    numpy array; strides in elements, offset 0."""
    if isinstance(t, np.ndarray):
        if t.ndim != 2:
            raise ValueError("memref operands are 2-D")
        ptr, (d0, d1) = t.ctypes.data, t.shape
        s0, s1 = (st // t.itemsize for st in t.strides)
    else:
        if t.dim() != 2:
            raise ValueError("memref operands are 2-D")
        ptr, (d0, d1), (s0, s1) = t.data_ptr(), t.shape, t.stride()
    return MemRef2D(ptr, ptr, 0, d0, d1, s0, s1)


def kernel_fn_status() -> int:
    """Status of the calling thread's last KernelFn-shaped call."""
    return int(lib().llk_kernel_fn_status())


def _check_kernel_fn() -> None:
    st = kernel_fn_status()
    if st != _lib.LLK_OK:
        check(st)


class KernelFn:
    """JitCache::KernelFn (JitCache.h:79-81): fn(x, wg, wu, init, result)
    over five MemRef2D, no return value (status: llk_kernel_fn_status)."""

    def __init__(self, fn: MEMREF_FN):
        self._fn = fn

    @property
    def address(self) -> int:
        return C.cast(self._fn, C.c_void_p).value or 0

    def __call__(self, x, wg, wu, init, result) -> None:
        """Operands: 2-D torch tensors or numpy arrays (wu None for a
        matmul entry); raises LLKError on a failed call."""
        m = [memref(t) if t is not None else None for t in (x, wg, wu, init, result)]
        if result is init:
            m[4] = m[3]
        self._fn(*(C.byref(v) if v is not None else None for v in m))
        _check_kernel_fn()


def swiglu_kernel_fn(x, wg, wu, init, result) -> None:
    """llk_swiglu_kernel_fn (the library's KernelFn for the fused SwiGLU)."""
    KernelFn(C.cast(lib().llk_swiglu_kernel_fn, MEMREF_FN))(x, wg, wu, init, result)


def kernel_fn_assume_immutable_weights(on: bool) -> bool:
    """Opt-in reuse of packed weights by KernelFn calls; returns the previous
    setting."""
    return bool(lib().llk_kernel_fn_assume_immutable_weights(int(on)))


def code_object_path(operation: int, directory: str | None = None) -> str:
    """Path of the gfx950 code object of `operation` (OP_FUSED_SWIGLU or
    OP_MATMUL) in `directory` (None: the default directory)."""
    n = lib().llk_code_object_path(operation, directory.encode() if directory else None, None, 0)
    if n < 0:
        check(n)
    buf = C.create_string_buffer(n + 1)
    lib().llk_code_object_path(operation, directory.encode() if directory else None, buf, n + 1)
    return buf.value.decode()


def code_object_info(path: str) -> list[str]:
    """Reads and checks a code object without loading it: its kernel symbols."""
    count, n = C.c_int(), C.c_size_t()
    check(lib().llk_code_object_info(path.encode(), C.byref(count), None, 0, C.byref(n)))
    buf = C.create_string_buffer(n.value + 1)
    check(lib().llk_code_object_info(path.encode(), C.byref(count), buf, n.value + 1, C.byref(n)))
    names = buf.value.decode().split()
    assert len(names) == count.value
    return names


class JitCache:
    """Four LRU levels: L1 IR text, L2 optimized text, L3 KernelKey -> entry
    point, L4 WeightKey -> packed weights (owned by the cache)."""

    def __init__(self):
        self._c = C.c_void_p()
        check(lib().llk_cache_create(C.byref(self._c)))

    def close(self) -> None:
        if self._c is not None and self._c.value:
            lib().llk_cache_destroy(self._c)
        self._c = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- L3 -------------------------------------------------------------------
    def set_object_dir(self, path: str | None) -> None:
        """Directory the code objects are read from (None: the default)."""
        check(lib().llk_cache_set_object_dir(self._c, path.encode() if path else None))

    def lookup_or_compile(self, key: KernelKey) -> KernelFn:
        """lookupOrCompile(KernelKey): the key's KernelFn (MemRef2D shape)."""
        fn = MEMREF_FN()
        check(lib().llk_cache_lookup_or_compile(self._c, C.byref(key.c()), C.byref(fn)))
        return KernelFn(fn)

    def lookup_or_compile_packed(self, key: KernelKey) -> PackedEntry:
        """The same L3 entry in its packed-handle shape."""
        fn = KERNEL_FN()
        check(lib().llk_cache_lookup_or_compile_packed(self._c, C.byref(key.c()), C.byref(fn)))
        return PackedEntry(fn)

    def lookup_or_compile_str(self, cache_key: str, module: str) -> KernelFn:
        """lookupOrCompile(std::string, ModuleOp): the KernelFn of the
        module's first llk op, cached under `cache_key`."""
        fn = MEMREF_FN()
        text = module.encode()
        check(lib().llk_cache_lookup_or_compile_str(self._c, cache_key.encode(), text, len(text),
                                                    C.byref(fn)))
        return KernelFn(fn)

    def lookup_object_code(self, key: KernelKey) -> PackedEntry | None:
        fn = KERNEL_FN()
        r = lib().llk_cache_lookup_object_code(self._c, C.byref(key.c()), C.byref(fn))
        if r < 0:
            check(r)
        return PackedEntry(fn) if r == 1 else None

    def insert_object_code(self, key: KernelKey, fn: PackedEntry | int) -> None:
        f = fn._fn if isinstance(fn, PackedEntry) else KERNEL_FN(fn)
        check(lib().llk_cache_insert_object_code(self._c, C.byref(key.c()), f))

    # -- L1 / L2 --------------------------------------------------------------
    def _insert(self, level: int, key: str | bytes, value: str | bytes) -> None:
        k = key.encode() if isinstance(key, str) else key
        v = value.encode() if isinstance(value, str) else value
        check(lib().llk_cache_insert_blob(self._c, level, k, len(k), v, len(v)))

    def _lookup(self, level: int, key: str | bytes) -> str | None:
        k = key.encode() if isinstance(key, str) else key
        n = C.c_size_t()
        cap = 1 << 16
        buf = C.create_string_buffer(cap)
        r = lib().llk_cache_lookup_blob(self._c, level, k, len(k), buf, cap, C.byref(n))
        if r < 0:
            check(r)
        if r == 0:
            return None
        if n.value > cap:  # rare: a second lookup (counted as another hit)
            buf = C.create_string_buffer(n.value)
            lib().llk_cache_lookup_blob(self._c, level, k, len(k), buf, n.value, C.byref(n))
        return buf.raw[:n.value].decode()

    def insert_ir(self, key, value) -> None:
        self._insert(1, key, value)

    def lookup_ir(self, key) -> str | None:
        return self._lookup(1, key)

    def insert_optimized_mlir(self, key, value) -> None:
        self._insert(2, key, value)

    def lookup_optimized_mlir(self, key) -> str | None:
        return self._lookup(2, key)

    # -- L4 -------------------------------------------------------------------
    def insert_packed_weights(self, key: WeightKey, pw: PackedWeights) -> None:
        """Transfers ownership of `pw` to the cache."""
        check(lib().llk_cache_insert_packed_weights(self._c, C.byref(key.c()), pw.release()))

    def lookup_packed_weights(self, key: WeightKey) -> PackedWeights | None:
        out = C.c_void_p()
        r = lib().llk_cache_lookup_packed_weights(self._c, C.byref(key.c()), C.byref(out))
        if r < 0:
            check(r)
        return PackedWeights(out.value, owned=False) if r == 1 else None

    def get_packed_weights(self, w, bk: int = 64, host_only: bool = False) -> PackedWeights:
        """L4 lookup by (data pointer, shape, BK), packing on a miss: `w` is a
        host uint16 ndarray (bf16 bits) or a CUDA bfloat16 tensor.  The
        result is borrowed from the cache."""
        out = C.c_void_p()
        t, on_device, flags = self._weight_args(w, host_only)
        check(lib().llk_cache_get_packed_weights(self._c, C.byref(t), bk, on_device, flags,
                                                  C.byref(out)))
        return PackedWeights(out.value, owned=False)

    def acquire_packed_weights(self, w, bk: int = 64, host_only: bool = False) -> PackedWeights:
        """get_packed_weights with a counted reference: valid whatever the
        level does until release_packed_weights."""
        out = C.c_void_p()
        t, on_device, flags = self._weight_args(w, host_only)
        check(lib().llk_cache_acquire_packed_weights(self._c, C.byref(t), bk, on_device, flags,
                                                      C.byref(out)))
        return PackedWeights(out.value, owned=False)

    def release_packed_weights(self, pw: PackedWeights) -> None:
        check(lib().llk_cache_release_packed_weights(self._c, pw.handle))

    @staticmethod
    def _weight_args(w, host_only: bool):
        if isinstance(w, np.ndarray):
            if w.dtype != np.uint16 or w.ndim != 2 or w.strides[1] != 2:
                raise ValueError("w must be a 2-D uint16 array with unit inner stride")
            t = tensor2d(w.ctypes.data, w.shape[0], w.shape[1], w.strides[0] // 2)
            return t, 0, _lib.LLK_PACK_HOST_ONLY if host_only else 0
        _check_operand(w, "w", (_torch().bfloat16,))
        return _t2d(w), 1, 0

    # -- management -----------------------------------------------------------
    def evict_lru(self, level: int, max_entries: int) -> None:
        check(lib().llk_cache_evict_lru(self._c, level, max_entries))

    def set_max_entries(self, level: int, max_entries: int) -> None:
        check(lib().llk_cache_set_max_entries(self._c, level, max_entries))

    def stats(self) -> dict:
        s = CacheStatsC()
        check(lib().llk_cache_get_stats(self._c, C.byref(s)))
        return {"hits": list(s.hits), "misses": list(s.misses), "evictions": list(s.evictions)}

    def clear(self) -> None:
        lib().llk_cache_clear(self._c)

    def size(self) -> int:
        return lib().llk_cache_size(self._c)
