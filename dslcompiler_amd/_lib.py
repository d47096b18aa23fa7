"""ctypes binding of the C ABI in include/llk/llk_abi.h.

Loads ``dslcompiler_amd/libllk_gfx950.so`` from the package directory.  There
is no fallback: if the library is missing, :func:`lib` raises, so nothing can
silently run a CPU path instead of the HIP kernels.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libllk_gfx950.so"

LLK_OK = 0
LLK_ERR_INVALID_ARGUMENT = -1
LLK_ERR_SHAPE = -2
LLK_ERR_DTYPE = -3
LLK_ERR_LAYOUT = -4
LLK_ERR_HIP = -5
LLK_ERR_NO_DEVICE = -6
LLK_ERR_UNSUPPORTED_ARCH = -7
LLK_ERR_OUT_OF_MEMORY = -8
LLK_ERR_SCRATCH = -9
LLK_ERR_DEVICE_MISMATCH = -10
LLK_ERR_NOT_FOUND = -11

LLK_BF16, LLK_FP16, LLK_FP32 = 0, 1, 2
LLK_PACK_KEEP_HOST = 1
LLK_PACK_HOST_ONLY = 2
LLK_PLAN_X_ALIGNED = 1
LLK_PLAN_ACCUMULATE = 2
LLK_PLAN_OUT_F32 = 4

STATUS_NAMES = {
    0: "LLK_OK", -1: "LLK_ERR_INVALID_ARGUMENT", -2: "LLK_ERR_SHAPE", -3: "LLK_ERR_DTYPE",
    -4: "LLK_ERR_LAYOUT", -5: "LLK_ERR_HIP", -6: "LLK_ERR_NO_DEVICE",
    -7: "LLK_ERR_UNSUPPORTED_ARCH", -8: "LLK_ERR_OUT_OF_MEMORY", -9: "LLK_ERR_SCRATCH",
    -10: "LLK_ERR_DEVICE_MISMATCH", -11: "LLK_ERR_NOT_FOUND",
}


class Tensor2D(C.Structure):
    """Tensor2D (JitCache.h:30-36)."""
    _fields_ = [("data", C.c_void_p), ("dim0", C.c_int64), ("dim1", C.c_int64),
                ("stride0", C.c_int64), ("stride1", C.c_int64)]


class KernelContext(C.Structure):
    """KernelContext (JitCache.h:59-62) plus the HIP stream."""
    _fields_ = [("scratch", C.c_void_p), ("scratch_size", C.c_size_t), ("stream", C.c_void_p)]


class ScheduleEntry(C.Structure):
    """ScheduleEntry (ScheduleLoader.h:23-31)."""
    _fields_ = [("BM", C.c_int64), ("BN", C.c_int64), ("BK", C.c_int64), ("VM", C.c_int64),
                ("VN", C.c_int64), ("vector_width", C.c_int64), ("num_threads", C.c_int64),
                ("grain_size", C.c_int64), ("parallel_axis", C.c_char * 8)]


class KernelKeyC(C.Structure):
    """KernelKey (KernelKey.h:45-57): same fields, types and order."""
    _fields_ = [("operation", C.c_uint8), ("input_type", C.c_uint8), ("output_type", C.c_uint8),
                ("M_bucket", C.c_int64), ("N", C.c_int64), ("K", C.c_int64),
                ("weight_layout", C.c_uint8), ("isa", C.c_uint8), ("math_mode", C.c_uint8),
                ("thread_count", C.c_uint16), ("compiler_version", C.c_uint64),
                ("schedule_version", C.c_uint64)]


class WeightKeyC(C.Structure):
    """WeightKey (KernelKey.h:114-124)."""
    _fields_ = [("weight_ptr", C.c_void_p), ("shape_hash", C.c_uint64), ("BK", C.c_int64),
                ("BN", C.c_int64)]


class CacheStatsC(C.Structure):
    """CacheStats (JitCache.h:67-71)."""
    _fields_ = [("hits", C.c_size_t * 4), ("misses", C.c_size_t * 4),
                ("evictions", C.c_size_t * 4)]


class LaunchPlan(C.Structure):
    """llk_launch_plan: the dispatcher's choice for one call."""
    _fields_ = [("kernel", C.c_int), ("splits", C.c_int), ("group_width", C.c_int),
                ("pad_x", C.c_int), ("workgroups", C.c_int64),
                ("threads_per_workgroup", C.c_int64), ("launches", C.c_int64),
                ("workspace_bytes", C.c_size_t), ("head_blocks_n", C.c_int64),
                ("tile_columns", C.c_int64)]


class MemRef2D(C.Structure):
    """MemRef2D (JitCache.h:43-51): 56 bytes."""
    _fields_ = [("allocated", C.c_void_p), ("aligned", C.c_void_p), ("offset", C.c_int64),
                ("size0", C.c_int64), ("size1", C.c_int64), ("stride0", C.c_int64),
                ("stride1", C.c_int64)]


class LLKError(RuntimeError):
    """A negative llk_status, with the library's message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


P = C.c_void_p
PP = C.POINTER(C.c_void_p)
T2 = C.POINTER(Tensor2D)
CTX = C.POINTER(KernelContext)
KKP = C.POINTER(KernelKeyC)
WKP = C.POINTER(WeightKeyC)
# llk_kernel_fn: the shape of llk_swiglu_bf16
KERNEL_FN = C.CFUNCTYPE(C.c_int, T2, P, P, T2, C.c_int, CTX)

MR = C.POINTER(MemRef2D)
# llk_memref_kernel_fn: JitCache::KernelFn (JitCache.h:79-81)
MEMREF_FN = C.CFUNCTYPE(None, MR, MR, MR, MR, MR)

# name -> (restype, argtypes); every function declared in include/llk/llk_abi.h.
SIGNATURES = {
    "llk_last_error": (C.c_char_p, []),
    "llk_abi_version": (C.c_int, []),
    "llk_device_info": (C.c_int, [C.c_char_p, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                  C.POINTER(C.c_int)]),
    "llk_pack_weights": (C.c_int, [T2, C.c_int64, C.c_uint, PP]),
    "llk_pack_weights_device": (C.c_int, [T2, C.c_int64, P, PP]),
    "llk_repack": (C.c_int, [P, T2]),
    "llk_packed_weights_free": (None, [P]),
    "llk_packed_weights_k_blocks": (C.c_int64, [P]),
    "llk_packed_weights_n": (C.c_int64, [P]),
    "llk_packed_weights_block_size": (C.c_int64, [P]),
    "llk_packed_weights_bk": (C.c_int64, [P]),
    "llk_packed_weights_dtype": (C.c_int, [P]),
    "llk_packed_weights_k": (C.c_int64, [P]),
    "llk_packed_weights_host_data": (C.c_void_p, [P]),
    "llk_packed_weights_device_data": (C.c_void_p, [P]),
    "llk_packed_weights_device_bytes": (C.c_size_t, [P]),
    "llk_pack_device_bytes": (C.c_size_t, [C.c_int64, C.c_int64]),
    "llk_pack_device_layout": (C.c_int, [T2, P]),
    "llk_swiglu_bf16": (C.c_int, [T2, P, P, T2, C.c_int, CTX]),
    "llk_swiglu_bf16_noalloc": (C.c_int, [T2, P, P, T2, C.c_int, P]),
    "llk_swiglu_scratch_size": (C.c_size_t, [C.c_int64, C.c_int64, C.c_int64]),
    "llk_verify_fused_swiglu": (C.c_int, [C.c_int64] * 8),
    "llk_verify_matmul": (C.c_int, [C.c_int64, C.c_int64]),
    "llk_describe_launch": (C.c_int, [C.c_int, C.c_int64, C.c_int64, C.c_int64, C.c_uint,
                                      C.POINTER(LaunchPlan)]),
    "llk_workspace_stats": (C.c_int, [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "llk_workspace_trim": (C.c_int, []),
    "llk_gemm_bf16": (C.c_int, [T2, P, T2, C.c_int, CTX]),
    "llk_gemm_bf16_accumulate": (C.c_int, [T2, P, T2, C.c_int, CTX]),
    "llk_mlp_bf16": (C.c_int, [T2, P, P, P, T2, T2, CTX]),
    "llk_classify_m": (C.c_int, [C.c_int64]),
    "llk_num_tiles": (C.c_int64, [C.c_int64, C.c_int64]),
    "llk_tile_size": (C.c_int64, [C.c_int64, C.c_int64, C.c_int64]),
    "llk_num_inner_tiles": (C.c_int64, [C.c_int64, C.c_int64]),
    "llk_kernel_key_hash": (C.c_uint64, [C.c_uint8, C.c_uint8, C.c_uint8, C.c_int64, C.c_int64,
                                         C.c_int64, C.c_uint8, C.c_uint8, C.c_uint8, C.c_uint16,
                                         C.c_uint64, C.c_uint64]),
    "llk_set_schedule_db": (C.c_int, [C.c_char_p]),
    "llk_select_schedule": (C.c_int, [C.c_char_p, C.c_char_p, C.c_int,
                                      C.POINTER(ScheduleEntry), C.POINTER(C.c_int)]),
    "llk_fill_normal_bf16": (C.c_int, [C.c_uint64, C.c_uint64, C.c_float, P, C.c_int64,
                                       C.c_int]),
    "llk_set_tunable": (C.c_int, [C.c_char_p, C.c_int64]),
    "llk_get_tunable": (C.c_int, [C.c_char_p, C.POINTER(C.c_int64)]),
    "llk_packed_weights_serialize": (C.c_int, [P, P, C.c_size_t, C.POINTER(C.c_size_t)]),
    "llk_packed_weights_deserialize": (C.c_int, [P, C.c_size_t, C.c_uint, PP]),
    "llk_packed_weights_save": (C.c_int, [P, C.c_char_p]),
    "llk_packed_weights_load": (C.c_int, [C.c_char_p, C.c_uint, PP]),
    "llk_swiglu_kernel_fn": (None, [MR, MR, MR, MR, MR]),
    "llk_kernel_fn_status": (C.c_int, []),
    "llk_kernel_fn_cache": (C.c_void_p, []),
    "llk_kernel_fn_assume_immutable_weights": (C.c_int, [C.c_int]),
    "llk_cache_create": (C.c_int, [PP]),
    "llk_cache_destroy": (None, [P]),
    "llk_cache_lookup_or_compile": (C.c_int, [P, KKP, C.POINTER(MEMREF_FN)]),
    "llk_cache_lookup_or_compile_packed": (C.c_int, [P, KKP, C.POINTER(KERNEL_FN)]),
    "llk_cache_lookup_or_compile_str": (C.c_int, [P, C.c_char_p, C.c_char_p, C.c_size_t,
                                                  C.POINTER(MEMREF_FN)]),
    "llk_cache_set_object_dir": (C.c_int, [P, C.c_char_p]),
    "llk_code_object_path": (C.c_int, [C.c_int, C.c_char_p, C.c_char_p, C.c_size_t]),
    "llk_code_object_info": (C.c_int, [C.c_char_p, C.POINTER(C.c_int), C.c_char_p, C.c_size_t,
                                       C.POINTER(C.c_size_t)]),
    "llk_cache_lookup_object_code": (C.c_int, [P, KKP, C.POINTER(KERNEL_FN)]),
    "llk_cache_insert_object_code": (C.c_int, [P, KKP, KERNEL_FN]),
    "llk_cache_insert_blob": (C.c_int, [P, C.c_int, C.c_char_p, C.c_size_t, C.c_char_p,
                                        C.c_size_t]),
    "llk_cache_lookup_blob": (C.c_int, [P, C.c_int, C.c_char_p, C.c_size_t, P, C.c_size_t,
                                        C.POINTER(C.c_size_t)]),
    "llk_cache_insert_packed_weights": (C.c_int, [P, WKP, P]),
    "llk_cache_lookup_packed_weights": (C.c_int, [P, WKP, PP]),
    "llk_cache_get_packed_weights": (C.c_int, [P, T2, C.c_int64, C.c_int, C.c_uint, PP]),
    "llk_cache_acquire_packed_weights": (C.c_int, [P, T2, C.c_int64, C.c_int, C.c_uint, PP]),
    "llk_cache_release_packed_weights": (C.c_int, [P, P]),
    "llk_cache_evict_lru": (C.c_int, [P, C.c_int, C.c_size_t]),
    "llk_cache_set_max_entries": (C.c_int, [P, C.c_int, C.c_size_t]),
    "llk_cache_get_stats": (C.c_int, [P, C.POINTER(CacheStatsC)]),
    "llk_cache_clear": (None, [P]),
    "llk_cache_size": (C.c_size_t, [P]),
}

_LIB: C.CDLL | None = None


def lib() -> C.CDLL:
    """The loaded library (raises FileNotFoundError if it was never built)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `python -m dslcompiler_amd.build` "
                "(there is no CPU fallback)")
        # torch ships its own HIP runtime under the same SONAME
        # (libamdhip64.so.7).  Loading torch first makes this library bind to
        # that one copy, so both share device memory, streams and events.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        l = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _LIB = l
    return _LIB


def check(status: int) -> None:
    """Raises LLKError for a negative status."""
    if status != LLK_OK:
        msg = lib().llk_last_error()
        raise LLKError(status, msg.decode() if msg else "")


def tensor2d(ptr: int, dim0: int, dim1: int, stride0: int | None = None,
             stride1: int = 1) -> Tensor2D:
    return Tensor2D(ptr, dim0, dim1, dim1 if stride0 is None else stride0, stride1)
