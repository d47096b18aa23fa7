"""ctypes binding of the CPU oracle (oracle/oracle.cpp) and of oracle/_ref.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker.  The product library
never loads it.

Pinning status per function is listed in the header of oracle.cpp; the one
unpinned item is the exact bit pattern of the reference's JIT'd AVX2 output
(reduction order, LLVM expf), which needs an MLIR/LLVM 22 build.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libref.so"

_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i64 = C.c_int64


def build(ref: bool = True) -> None:
    """make liboracle.so (and oracle/_ref when the reference tree exists)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all" if ref else "oracle"], check=True)


_ORC = None
_REF = None


def orc() -> C.CDLL:
    global _ORC
    if _ORC is None:
        if not LIB_PATH.exists():
            build(ref=False)
        l = C.CDLL(str(LIB_PATH))
        l.orc_bf16_to_f32.restype = C.c_float
        l.orc_bf16_to_f32.argtypes = [C.c_uint16]
        l.orc_f32_to_bf16_rne.restype = C.c_uint16
        l.orc_f32_to_bf16_rne.argtypes = [C.c_float]
        l.orc_f32_to_bf16_testhelper.restype = C.c_uint16
        l.orc_f32_to_bf16_testhelper.argtypes = [C.c_float]
        l.orc_bf16_to_f32_array.argtypes = [_u16p, _f32p, _i64]
        l.orc_f32_to_bf16_rne_array.argtypes = [_f32p, _u16p, _i64]
        l.orc_swiglu_epilogue.restype = C.c_float
        l.orc_swiglu_epilogue.argtypes = [C.c_float, C.c_float]
        l.orc_swiglu_fused.argtypes = [C.c_void_p, _i64, C.c_void_p, C.c_void_p, _i64, _i64, _i64,
                                       _i64, C.c_void_p, C.c_void_p, _i64]
        l.orc_swiglu_accumulators.argtypes = [C.c_void_p, _i64, C.c_void_p, C.c_void_p, _i64,
                                              _i64, _i64, _i64, C.c_void_p, C.c_void_p]
        l.orc_swiglu_fp64.argtypes = [_f64p, _f64p, _f64p, _f64p, _i64, _i64, _i64]
        l.orc_gemm.argtypes = [C.c_void_p, _i64, C.c_void_p, _i64, _i64, _i64, _i64, C.c_void_p,
                               C.c_void_p, _i64]
        l.orc_gemm_init.argtypes = [C.c_void_p, _i64, C.c_void_p, _i64, _i64, _i64, _i64,
                                    C.c_void_p, _i64, C.c_void_p, C.c_void_p, _i64]
        l.orc_gemm_avx2_mt.argtypes = [C.c_void_p, _i64, C.c_void_p, _i64, _i64, _i64, _i64,
                                       C.c_void_p, _i64, C.c_void_p, C.c_void_p, _i64, C.c_int]
        l.orc_gemm_fp64.argtypes = [_u16p, _u16p, _f64p, _i64, _i64, _i64]
        l.orc_mlp.argtypes = [_u16p, _u16p, _u16p, _u16p, _i64, _i64, _i64, _u16p, _u16p]
        l.orc_classify_m.restype = C.c_int
        l.orc_classify_m.argtypes = [_i64]
        for n in ("orc_num_tiles", "orc_num_inner_tiles"):
            getattr(l, n).restype = _i64
            getattr(l, n).argtypes = [_i64, _i64]
        l.orc_tile_size.restype = _i64
        l.orc_tile_size.argtypes = [_i64, _i64, _i64]
        l.orc_kernel_key_hash.restype = C.c_uint64
        l.orc_kernel_key_hash.argtypes = [C.c_uint8, C.c_uint8, C.c_uint8, _i64, _i64, _i64,
                                          C.c_uint8, C.c_uint8, C.c_uint8, C.c_uint16, C.c_uint64,
                                          C.c_uint64]
        l.orc_pack_weight_meta.argtypes = [_i64, _i64, _i64, _i64p]
        l.orc_pack_weight_matrix.argtypes = [_u16p, _i64, _i64, _i64, _i64, _u16p]
        l.orc_swiglu_avx2_mt.argtypes = [C.c_void_p, _i64, C.c_void_p, C.c_void_p, _i64, _i64,
                                         _i64, _i64, C.c_void_p, C.c_void_p, _i64, C.c_int, _i64]
        l.orc_cpu_has_avx2_fma.restype = C.c_int
        _ORC = l
    return _ORC


def ref() -> C.CDLL | None:
    """The reference's own routines compiled from source, or None if absent."""
    global _REF
    if _REF is None:
        if not REF_PATH.exists():
            return None
        l = C.CDLL(str(REF_PATH))
        l.ref_swiglu_fp32.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64]
        l.ref_swiglu_fp64.argtypes = [_f64p, _f64p, _f64p, _f64p, _i64, _i64, _i64]
        l.ref_edge_swiglu_fp64.argtypes = [_f64p, _f64p, _f64p, _f64p, _i64, _i64, _i64]
        l.ref_f32_to_bf16.restype = C.c_uint16
        l.ref_f32_to_bf16.argtypes = [C.c_float]
        l.ref_bf16_to_f32.restype = C.c_float
        l.ref_bf16_to_f32.argtypes = [C.c_uint16]
        l.ref_kernel_key_hash.restype = C.c_uint64
        l.ref_kernel_key_hash.argtypes = [C.c_uint8, C.c_uint8, C.c_uint8, _i64, _i64, _i64,
                                          C.c_uint8, C.c_uint8, C.c_uint8, C.c_uint16, C.c_uint64,
                                          C.c_uint64]
        l.ref_kernel_key_default_hash.restype = C.c_uint64
        l.ref_kernel_key_sizeof.restype = C.c_int
        l.ref_kernel_key_to_string.restype = C.c_int
        l.ref_kernel_key_to_string.argtypes = [C.c_uint64, _i64, _i64, C.c_char_p, C.c_int]
        _REF = l
    return _REF


# ---------------------------------------------------------------------------
# numpy-level wrappers
# ---------------------------------------------------------------------------

def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    orc().orc_bf16_to_f32_array(h.ravel(), out.ravel(), h.size)
    return out


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    orc().orc_f32_to_bf16_rne_array(f.ravel(), out.ravel(), f.size)
    return out


def swiglu(x: np.ndarray, wg: np.ndarray, wu: np.ndarray, want_f32: bool = True,
           want_bf16: bool = True):
    """Fused-path SwiGLU of bf16 bits: returns (y_f32, y_bf16)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    wg = np.ascontiguousarray(wg, dtype=np.uint16)
    wu = np.ascontiguousarray(wu, dtype=np.uint16)
    M, K = x.shape
    N = wg.shape[1]
    yf = np.empty((M, N), np.float32) if want_f32 else None
    yb = np.empty((M, N), np.uint16) if want_bf16 else None
    orc().orc_swiglu_fused(_p(x), K, _p(wg), _p(wu), N, M, N, K, _p(yf), _p(yb), N)
    return yf, yb


def swiglu_rows(x: np.ndarray, wg: np.ndarray, wu: np.ndarray, rows) -> tuple:
    """Fused-path SwiGLU of selected rows only (for full-size spot checks)."""
    xs = np.ascontiguousarray(x[np.asarray(rows)], dtype=np.uint16)
    return swiglu(xs, wg, wu)


def swiglu_accumulators(x, wg, wu):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    wg = np.ascontiguousarray(wg, dtype=np.uint16)
    wu = np.ascontiguousarray(wu, dtype=np.uint16)
    M, K = x.shape
    N = wg.shape[1]
    g = np.empty((M, N), np.float32)
    u = np.empty((M, N), np.float32)
    orc().orc_swiglu_accumulators(_p(x), K, _p(wg), _p(wu), N, M, N, K, _p(g), _p(u))
    return g, u


def swiglu_fp64(x: np.ndarray, wg: np.ndarray, wu: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    wg = np.ascontiguousarray(wg, dtype=np.float64)
    wu = np.ascontiguousarray(wu, dtype=np.float64)
    M, K = x.shape
    N = wg.shape[1]
    y = np.empty((M, N), np.float64)
    orc().orc_swiglu_fp64(x, wg, wu, y, M, N, K)
    return y


def gemm(a: np.ndarray, b: np.ndarray, want_f32: bool = True, want_bf16: bool = True):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    M, K = a.shape
    N = b.shape[1]
    cf = np.empty((M, N), np.float32) if want_f32 else None
    cb = np.empty((M, N), np.uint16) if want_bf16 else None
    orc().orc_gemm(_p(a), K, _p(b), N, M, N, K, _p(cf), _p(cb), N)
    return cf, cb


def gemm_init(a: np.ndarray, b: np.ndarray, c_init: np.ndarray | None, want_f32: bool = True,
              want_bf16: bool = True):
    """C = C0 + A B with the fp32 accumulator starting at c_init (fp32
    [M, N], or None for 0) and the products added in k order."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    M, K = a.shape
    N = b.shape[1]
    ci = None if c_init is None else np.ascontiguousarray(c_init, dtype=np.float32)
    cf = np.empty((M, N), np.float32) if want_f32 else None
    cb = np.empty((M, N), np.uint16) if want_bf16 else None
    orc().orc_gemm_init(_p(a), K, _p(b), N, M, N, K, _p(ci), N, _p(cf), _p(cb), N)
    return cf, cb


def gemm_avx2(a: np.ndarray, b: np.ndarray, threads: int, c_init: np.ndarray | None = None,
              want_f32: bool = True, want_bf16: bool = True):
    """gemm_init on `threads` host threads (bit-equal to it): for full-size checks."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    M, K = a.shape
    N = b.shape[1]
    ci = None if c_init is None else np.ascontiguousarray(c_init, dtype=np.float32)
    cf = np.empty((M, N), np.float32) if want_f32 else None
    cb = np.empty((M, N), np.uint16) if want_bf16 else None
    orc().orc_gemm_avx2_mt(_p(a), K, _p(b), N, M, N, K, _p(ci), N, _p(cf), _p(cb), N, threads)
    return cf, cb


def gemm_fp64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    M, K = a.shape
    N = b.shape[1]
    c = np.empty((M, N), np.float64)
    orc().orc_gemm_fp64(a, b, c, M, N, K)
    return c


def mlp(x, wg, wu, wd):
    """(y_bf16, z_bf16) of the MLP block; wd is [N, K_out]."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    M, K = x.shape
    N = wg.shape[1]
    assert wd.shape == (N, K), "this oracle's MLP takes Wd [N, K] (output width = K)"
    y = np.empty((M, N), np.uint16)
    z = np.empty((M, K), np.uint16)
    orc().orc_mlp(x, np.ascontiguousarray(wg, np.uint16), np.ascontiguousarray(wu, np.uint16),
                  np.ascontiguousarray(wd, np.uint16), M, N, K, y, z)
    return y, z


def swiglu_avx2(x, wg, wu, threads: int, grain: int = 1, want_f32: bool = False):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    wg = np.ascontiguousarray(wg, dtype=np.uint16)
    wu = np.ascontiguousarray(wu, dtype=np.uint16)
    M, K = x.shape
    N = wg.shape[1]
    yb = np.empty((M, N), np.uint16)
    yf = np.empty((M, N), np.float32) if want_f32 else None
    orc().orc_swiglu_avx2_mt(_p(x), K, _p(wg), _p(wu), N, M, N, K, _p(yb), _p(yf), N, threads,
                             grain)
    return yb, yf


def pack_weight_matrix(w: np.ndarray, bk: int) -> tuple[np.ndarray, list[int]]:
    """Reference host layout [K_blocks][BK][N] and metadata list."""
    w = np.ascontiguousarray(w, dtype=np.uint16)
    K, N = w.shape
    meta = np.zeros(5, np.int64)
    orc().orc_pack_weight_meta(K, N, bk, meta)
    out = np.empty(int(meta[0] * bk * N), np.uint16)
    orc().orc_pack_weight_matrix(w, K, N, N, bk, out)
    return out.reshape(int(meta[0]), bk, N), [int(v) for v in meta]
