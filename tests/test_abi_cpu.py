"""CPU tests of the C ABI surface: the library loads, exports every function
include/llk/llk_abi.h declares, and validates arguments (FusedSwiGLUOp /
micro.mma verifier rules) before any device work."""
from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from common import normal_bf16

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "llk" / "llk_abi.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(llk_[a-z0-9_]+)\s*\(", text))


def test_header_is_plain_c():
    """The boundary header compiles as C (no C++ or torch types)."""
    r = subprocess.run(["gcc", "-std=c99", "-fsyntax-only", "-x", "c", str(HEADER)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_library_exports_every_declared_symbol(llk):
    from dslcompiler_amd._lib import LIB_PATH, SIGNATURES
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    decl = declared_functions()
    assert decl, "no declarations parsed"
    assert decl <= exported, sorted(decl - exported)
    assert decl == set(SIGNATURES), (sorted(decl - set(SIGNATURES)), sorted(set(SIGNATURES) - decl))


def test_abi_version(llk):
    assert llk.lib().llk_abi_version() == 4


def _t(arr, rows=None, cols=None, stride0=None, stride1=1):
    from dslcompiler_amd._lib import Tensor2D
    r = arr.shape[0] if rows is None else rows
    c = arr.shape[1] if cols is None else cols
    return Tensor2D(arr.ctypes.data, r, c, c if stride0 is None else stride0, stride1)


def test_swiglu_validation_errors(llk):
    """LLKOps.cpp:42-83 checks (and message wording) come back as status
    codes with a readable last-error string, before any device work."""
    L = llk.lib()
    wg = llk.PackedWeights.from_host(normal_bf16(1, 1, (16, 32)), host_only=True)
    wu = llk.PackedWeights.from_host(normal_bf16(1, 2, (16, 48)), host_only=True)
    wk = llk.PackedWeights.from_host(normal_bf16(1, 3, (15, 32)), host_only=True)
    x = np.zeros((4, 16), np.uint16)
    y = np.zeros((4, 32), np.uint16)
    ctx = llk.ops._lib.KernelContext(None, 0, None)

    def call(xt, a, b, yt, dtype=0):
        return L.llk_swiglu_bf16(C.byref(xt), a.handle, b.handle, C.byref(yt), dtype, C.byref(ctx))

    assert call(_t(x), wg, wu, _t(y)) == -2
    assert b"N dimension mismatch between Wg=32 and Wu=48" in L.llk_last_error()
    assert call(_t(x), wk, wg, _t(y)) == -2
    assert b"K dimension mismatch between X=16 and Wg=15" in L.llk_last_error()
    assert call(_t(x), wg, wg, _t(np.zeros((5, 32), np.uint16))) == -2
    assert b"M dimension mismatch" in L.llk_last_error()
    assert call(_t(x), wg, wg, _t(np.zeros((4, 31), np.uint16))) == -2
    assert call(_t(x), wg, wg, _t(y), dtype=1) == -3               # fp16 output unsupported
    assert call(_t(x, stride1=2), wg, wg, _t(y)) == -4             # non-unit inner stride
    assert call(_t(x, stride0=8), wg, wg, _t(y)) == -4             # stride0 < dim1
    assert L.llk_swiglu_bf16(None, wg.handle, wg.handle, C.byref(_t(y)), 0, None) == -1
    assert L.llk_swiglu_bf16(C.byref(_t(x)), None, wg.handle, C.byref(_t(y)), 0, None) == -1
    # M = 0 is valid: nothing to do (edge_cases.cpp:84-97)
    x0 = np.zeros((0, 16), np.uint16)
    y0 = np.zeros((0, 32), np.uint16)
    assert call(_t(x0), wg, wg, _t(y0)) == 0


def test_gemm_validation_errors(llk):
    L = llk.lib()
    b = llk.PackedWeights.from_host(normal_bf16(1, 1, (16, 32)), host_only=True)
    a = np.zeros((4, 16), np.uint16)
    c = np.zeros((4, 32), np.float32)
    assert L.llk_gemm_bf16(C.byref(_t(np.zeros((4, 17), np.uint16))), b.handle, C.byref(_t(c)),
                           2, None) == -2
    assert L.llk_gemm_bf16(C.byref(_t(a)), b.handle, C.byref(_t(np.zeros((4, 33), np.float32))),
                           2, None) == -2
    assert L.llk_gemm_bf16(C.byref(_t(a)), b.handle, C.byref(_t(c)), 7, None) == -3
    # the accumulating form checks the same contract before touching a device
    for fn in (L.llk_gemm_bf16, L.llk_gemm_bf16_accumulate):
        assert fn(C.byref(_t(np.zeros((4, 17), np.uint16))), b.handle, C.byref(_t(c)), 2,
                  None) == -2
        assert fn(C.byref(_t(a)), b.handle, C.byref(_t(c)), 7, None) == -3
        assert fn(C.byref(_t(a)), None, C.byref(_t(c)), 2, None) == -1


def test_pack_validation(llk):
    L = llk.lib()
    w = normal_bf16(1, 1, (8, 8))
    out = C.c_void_p()
    assert L.llk_pack_weights(C.byref(_t(w)), 0, 2, C.byref(out)) == -1   # BK must be > 0
    assert L.llk_pack_weights(C.byref(_t(w, stride1=3)), 64, 2, C.byref(out)) == -4
    assert L.llk_pack_weights(None, 64, 2, C.byref(out)) == -1
    assert L.llk_pack_weights(C.byref(_t(w)), 64, 2, None) == -1
    pw = llk.PackedWeights.from_host(w, host_only=True)
    with pytest.raises(llk.LLKError, match="repack shape"):
        pw.repack(normal_bf16(1, 1, (9, 8)))
    L.llk_packed_weights_free(None)  # no-op


def test_host_only_handle_is_rejected_by_kernels(llk):
    """A host-only handle has no device payload: a launch reports it (or the
    missing device on a CPU-only machine) instead of touching memory."""
    L = llk.lib()
    wg = llk.PackedWeights.from_host(normal_bf16(1, 1, (16, 32)), host_only=True)
    x = np.zeros((4, 16), np.uint16)
    y = np.zeros((4, 32), np.uint16)
    st = L.llk_swiglu_bf16(C.byref(_t(x)), wg.handle, wg.handle, C.byref(_t(y)), 0, None)
    assert st in (-1, -6, -7)
    assert L.llk_packed_weights_device_data(wg.handle) is None


def test_python_wrappers_reject_host_tensors(llk):
    """The torch wrappers refuse operands that are not CUDA tensors of the
    accepted dtype before calling the C ABI (which takes raw pointers: a
    host pointer would reach a kernel)."""
    import torch
    wg = llk.PackedWeights.from_host(normal_bf16(1, 1, (16, 32)), host_only=True)
    x = torch.zeros((4, 16), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="x must be a CUDA tensor"):
        llk.fused_swiglu(x, wg, wg)
    with pytest.raises(ValueError, match="a must be a CUDA tensor"):
        llk.matmul(x, wg)
    with pytest.raises(ValueError, match="x must be a CUDA tensor"):
        llk.mlp(x, wg, wg, wg)
    with pytest.raises(ValueError, match="w must be a CUDA tensor"):
        llk.PackedWeights.from_device(torch.zeros((16, 32), dtype=torch.bfloat16))


def test_cache_and_scratch_paths_reject_host_tensors(llk):
    """The entry point handed out by the cache's object-code level, the L4
    device-pack path and a caller workspace are checked like the wrappers'
    operands, before any C call (a host or fp32 tensor would otherwise reach
    a kernel as a raw pointer)."""
    import torch
    from dslcompiler_amd import cache, ops
    jc = cache.JitCache()
    fn = jc.lookup_or_compile_packed(cache.KernelKey(operation=cache.OP_FUSED_SWIGLU, N=32,
                                                     K=16, isa=cache.ISA_GFX950))
    wg = llk.PackedWeights.from_host(normal_bf16(1, 1, (16, 32)), host_only=True)
    x = torch.zeros((4, 16), dtype=torch.bfloat16)
    y = torch.zeros((4, 32), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="x must be a CUDA tensor"):
        fn(x, wg, wg, y)
    with pytest.raises(ValueError, match="w must be a CUDA tensor"):
        jc.get_packed_weights(torch.zeros((16, 32), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="w must be a CUDA tensor"):
        jc.get_packed_weights(torch.zeros((16, 32), dtype=torch.float32))
    with pytest.raises(ValueError, match="scratch must be a CUDA tensor"):
        ops._ctx(None, torch.zeros(1024, dtype=torch.uint8))
    assert jc.stats()["misses"][3] == 0  # nothing reached the L4 level
    jc.close()


def test_tunables(llk):
    assert llk.get_tunable("decode_max_m") == 64
    llk.set_tunable("decode_splits", 3)
    assert llk.get_tunable("decode_splits") == 3
    llk.set_tunable("decode_splits", 0)
    # the header's knobs, at their documented defaults
    assert [llk.get_tunable(k) for k in ("midm_max_m", "tile_tail_split", "tile_wide",
                                         "kernel_fn_rowmajor", "max_workspaces")] == [128, 1, 1, 1, 16]
    with pytest.raises(llk.LLKError, match="unknown tunable"):
        llk.set_tunable("no_such_knob", 1)
    with pytest.raises(llk.LLKError):
        llk.get_tunable("no_such_knob")


def test_scratch_size_query(llk):
    """Decode-sized problems that split K across workgroups need a workspace;
    whole-tile problems with aligned X need none."""
    assert llk.swiglu_scratch_size(0, 10, 10) == 0
    assert llk.swiglu_scratch_size(8, 5120, 13824 * 4) >= 0
    assert llk.swiglu_scratch_size(2048, 11008, 4096) > 0  # worst case: X needs padding


def test_kernel_fn_shape_errors_before_any_device_call(llk):
    """llk_swiglu_kernel_fn (JitCache::KernelFn shape) verifies the memrefs
    with the op's verifier before touching a device; its status and message
    are the calling thread's."""
    import ctypes as C
    from dslcompiler_amd._lib import MemRef2D
    L = llk.lib()
    buf = (C.c_uint16 * 64)()
    x = MemRef2D(C.addressof(buf), C.addressof(buf), 0, 4, 8, 8, 1)
    w = MemRef2D(C.addressof(buf), C.addressof(buf), 0, 4, 8, 8, 1)  # K = 4 != 8
    L.llk_swiglu_kernel_fn(C.byref(x), C.byref(w), C.byref(w), C.byref(x), C.byref(x))
    assert L.llk_kernel_fn_status() == llk._lib.LLK_ERR_SHAPE
    assert b"K dimension mismatch between X=8 and Wg=4" in L.llk_last_error()
    y = MemRef2D(C.addressof(buf), C.addressof(buf), 0, 4, 5, 5, 1)
    w8 = MemRef2D(C.addressof(buf), C.addressof(buf), 0, 8, 4, 4, 1)
    init = MemRef2D(C.addressof(buf), C.addressof(buf), 0, 4, 4, 4, 1)
    L.llk_swiglu_kernel_fn(C.byref(x), C.byref(w8), C.byref(w8), C.byref(init), C.byref(y))
    assert L.llk_kernel_fn_status() == llk._lib.LLK_ERR_SHAPE
    assert b"result shape differs from init" in L.llk_last_error()
    assert C.sizeof(MemRef2D) == 56
