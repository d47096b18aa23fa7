"""Host-side mirror of the reference operator surface for this path.

- :class:`PackedWeights` mirrors ``PackedWeights`` / ``packWeightMatrix`` /
  ``repack`` (PackedWeights.h:13-49) over the C ABI handle.
- :func:`fused_swiglu` is ``llk.fused_swiglu`` (LLKOps.td:13-67) executed by
  the gfx950 kernels: X[M,K] bf16, packed Wg/Wu [K,N], result bf16 (the
  reference op's result type) or fp32 (the pre-truncf value).
- :func:`matmul` is the micro.mma / llk.matmul contract (MicroOps.td:196-222,
  LLKOps.td:210-255) with fp32 accumulation.
- :func:`mlp` composes SwiGLU and the down projection.

torch tensors only carry device memory and the current stream; all compute
goes through ``libllk_gfx950.so``.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import (LLK_BF16, LLK_FP32, LLK_PACK_HOST_ONLY, LLK_PACK_KEEP_HOST, KernelContext,
                   check, lib, tensor2d)


def _torch():
    import torch
    return torch


def _stream_handle(stream=None) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _ctx(stream=None, scratch=None) -> KernelContext:
    if scratch is not None:
        _check_scratch(scratch)
    ctx = KernelContext(None, 0, _stream_handle(stream))
    if scratch is not None:
        ctx.scratch = scratch.data_ptr()
        ctx.scratch_size = scratch.numel() * scratch.element_size()
    return ctx


def _check_scratch(t) -> None:
    """A caller workspace must be contiguous device memory of the current
    device: the kernels write partial sums into it through a raw pointer."""
    torch = _torch()
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError("scratch must be a CUDA tensor")
    cur = torch.cuda.current_device()
    if t.device.index != cur:
        raise ValueError(f"scratch is on cuda:{t.device.index}, the current device is cuda:{cur}")
    if not t.is_contiguous():
        raise ValueError("scratch must be contiguous")


def _check_operand(t, name: str, dtypes) -> None:
    """A kernel operand must be a 2-D tensor of an accepted dtype on the
    current CUDA device: the C ABI takes raw pointers and cannot tell host
    memory (a GPU memory fault when a kernel reads it) or another device's
    memory from the current device's."""
    torch = _torch()
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA tensor")
    if t.dtype not in dtypes:
        raise ValueError(f"{name} has dtype {t.dtype}; expected one of {tuple(dtypes)}")
    cur = torch.cuda.current_device()
    if t.device.index != cur:
        raise ValueError(f"{name} is on cuda:{t.device.index}, the current device is cuda:{cur}")


def _t2d(t) -> _lib.Tensor2D:
    if t.dim() != 2:
        raise ValueError("expected a 2-D tensor")
    return tensor2d(t.data_ptr(), t.shape[0], t.shape[1], t.stride(0), t.stride(1))


def _out_dtype_code(dtype) -> int:
    torch = _torch()
    if dtype == torch.bfloat16:
        return LLK_BF16
    if dtype == torch.float32:
        return LLK_FP32
    if dtype == torch.float16:
        return _lib.LLK_FP16
    raise ValueError(f"unsupported output dtype {dtype}")


class PackedWeights:
    """Packed bf16 weight matrix [K, N] resident on the current device.

    Metadata (``K_blocks``, ``N``, ``block_size``, ``BK``, ``dtype``) equals the
    reference's packWeightMatrix exactly (PackedWeights.cpp:5-15).
    """

    def __init__(self, handle: int, owned: bool = True):
        self._h = C.c_void_p(handle)
        self._owned = owned  # False: borrowed from a cache, never freed here

    # -- construction -------------------------------------------------------
    @classmethod
    def from_host(cls, w: np.ndarray, bk: int = 64, keep_host: bool = False,
                  host_only: bool = False) -> "PackedWeights":
        """packWeightMatrix from a host bf16 matrix given as uint16 bits.
        host_only: the reference's host packer alone (no device payload)."""
        w = np.asarray(w, dtype=np.uint16)
        if w.ndim != 2:
            raise ValueError("w must be 2-D")
        if w.strides[1] != 2:
            w = np.ascontiguousarray(w)
        t = tensor2d(w.ctypes.data, w.shape[0], w.shape[1], w.strides[0] // 2)
        flags = (LLK_PACK_KEEP_HOST if keep_host else 0) | (LLK_PACK_HOST_ONLY if host_only else 0)
        out = C.c_void_p()
        check(lib().llk_pack_weights(C.byref(t), bk, flags, C.byref(out)))
        return cls(out.value)

    @classmethod
    def from_device(cls, w, bk: int = 64, stream=None) -> "PackedWeights":
        """Packs a torch bf16 [K, N] CUDA tensor with the device pack kernel."""
        torch = _torch()
        _check_operand(w, "w", (torch.bfloat16,))
        out = C.c_void_p()
        check(lib().llk_pack_weights_device(C.byref(_t2d(w)), bk, _stream_handle(stream),
                                            C.byref(out)))
        return cls(out.value)

    def repack(self, w: np.ndarray) -> None:
        """repack (PackedWeights.cpp:35-37) with new host contents."""
        w = np.ascontiguousarray(w, dtype=np.uint16)
        t = tensor2d(w.ctypes.data, w.shape[0], w.shape[1])
        check(lib().llk_repack(self._h, C.byref(t)))

    # -- serialized form ----------------------------------------------------
    def serialize(self) -> bytes:
        """The versioned blob (96-byte header + device-layout payload)."""
        n = C.c_size_t()
        check(lib().llk_packed_weights_serialize(self.handle, None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value)
        check(lib().llk_packed_weights_serialize(self.handle, buf, n.value, C.byref(n)))
        return buf.raw[:n.value]

    @classmethod
    def from_blob(cls, blob: bytes, keep_host: bool = False,
                  host_only: bool = False) -> "PackedWeights":
        flags = (LLK_PACK_KEEP_HOST if keep_host else 0) | (LLK_PACK_HOST_ONLY if host_only else 0)
        out = C.c_void_p()
        check(lib().llk_packed_weights_deserialize(blob, len(blob), flags, C.byref(out)))
        return cls(out.value)

    def save(self, path) -> None:
        check(lib().llk_packed_weights_save(self.handle, str(path).encode()))

    @classmethod
    def load(cls, path, keep_host: bool = False, host_only: bool = False) -> "PackedWeights":
        flags = (LLK_PACK_KEEP_HOST if keep_host else 0) | (LLK_PACK_HOST_ONLY if host_only else 0)
        out = C.c_void_p()
        check(lib().llk_packed_weights_load(str(path).encode(), flags, C.byref(out)))
        return cls(out.value)

    def release(self) -> C.c_void_p:
        """Gives up ownership (e.g. to a cache) and returns the raw handle."""
        h = self.handle
        self._owned = False
        return h

    def free(self) -> None:
        if self._h is not None and self._h.value and self._owned:
            lib().llk_packed_weights_free(self._h)
        self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()

    # -- metadata -----------------------------------------------------------
    @property
    def handle(self) -> C.c_void_p:
        if self._h is None:
            raise ValueError("packed weights were freed")
        return self._h

    @property
    def K_blocks(self) -> int:
        return lib().llk_packed_weights_k_blocks(self.handle)

    @property
    def N(self) -> int:
        return lib().llk_packed_weights_n(self.handle)

    @property
    def K(self) -> int:
        return lib().llk_packed_weights_k(self.handle)

    @property
    def block_size(self) -> int:
        return lib().llk_packed_weights_block_size(self.handle)

    @property
    def BK(self) -> int:
        return lib().llk_packed_weights_bk(self.handle)

    @property
    def dtype(self) -> int:
        return lib().llk_packed_weights_dtype(self.handle)

    @property
    def device_bytes(self) -> int:
        return lib().llk_packed_weights_device_bytes(self.handle)

    def host_data(self) -> np.ndarray | None:
        """The reference host layout [K_blocks][BK][N] (uint16), if kept."""
        p = lib().llk_packed_weights_host_data(self.handle)
        if not p:
            return None
        n = self.K_blocks * self.BK * self.N
        buf = (C.c_uint16 * n).from_address(p)
        return np.frombuffer(buf, dtype=np.uint16).reshape(self.K_blocks, self.BK, self.N).copy()


def pack_device_layout(w: np.ndarray) -> np.ndarray:
    """Host computation of the device payload bytes for bf16 bits ``w`` [K, N]."""
    w = np.ascontiguousarray(w, dtype=np.uint16)
    nbytes = lib().llk_pack_device_bytes(w.shape[0], w.shape[1])
    out = np.zeros(nbytes, dtype=np.uint8)
    t = tensor2d(w.ctypes.data, w.shape[0], w.shape[1])
    check(lib().llk_pack_device_layout(C.byref(t), out.ctypes.data))
    return out


def fused_swiglu(x, wg: PackedWeights, wu: PackedWeights, out=None, out_dtype=None,
                 stream=None, scratch=None):
    """Y = SiLU(X Wg) * (X Wu) on the current device (asynchronous)."""
    torch = _torch()
    _check_operand(x, "x", (torch.bfloat16,))
    if out is None:
        out = torch.empty((x.shape[0], wg.N), dtype=out_dtype or torch.bfloat16, device=x.device)
    _check_operand(out, "out", (torch.bfloat16, torch.float32))
    check(lib().llk_swiglu_bf16(C.byref(_t2d(x)), wg.handle, wu.handle, C.byref(_t2d(out)),
                                _out_dtype_code(out.dtype), C.byref(_ctx(stream, scratch))))
    return out


def matmul(a, b: PackedWeights, out=None, out_dtype=None, stream=None, scratch=None,
           accumulate: bool = False):
    """C = A B (micro.mma, fp32 accumulation) on the current device; with
    accumulate=True, out += A B (micro.mma's acc += lhs * rhs: `out` is
    required and read in place)."""
    torch = _torch()
    _check_operand(a, "a", (torch.bfloat16,))
    if out is None:
        if accumulate:
            raise ValueError("accumulate=True needs `out`, the accumulator")
        out = torch.empty((a.shape[0], b.N), dtype=out_dtype or torch.float32, device=a.device)
    _check_operand(out, "out", (torch.bfloat16, torch.float16, torch.float32))
    fn = lib().llk_gemm_bf16_accumulate if accumulate else lib().llk_gemm_bf16
    check(fn(C.byref(_t2d(a)), b.handle, C.byref(_t2d(out)), _out_dtype_code(out.dtype),
             C.byref(_ctx(stream, scratch))))
    return out


def mlp(x, wg: PackedWeights, wu: PackedWeights, wd: PackedWeights, y=None, z=None,
        stream=None, scratch=None):
    """Y = SwiGLU(X) (bf16), Z = Y Wd (bf16); returns (y, z)."""
    torch = _torch()
    _check_operand(x, "x", (torch.bfloat16,))
    if y is None:
        y = torch.empty((x.shape[0], wg.N), dtype=torch.bfloat16, device=x.device)
    if z is None:
        z = torch.empty((x.shape[0], wd.N), dtype=torch.bfloat16, device=x.device)
    _check_operand(y, "y", (torch.bfloat16,))
    _check_operand(z, "z", (torch.bfloat16,))
    check(lib().llk_mlp_bf16(C.byref(_t2d(x)), wg.handle, wu.handle, wd.handle,
                             C.byref(_t2d(y)), C.byref(_t2d(z)), C.byref(_ctx(stream, scratch))))
    return y, z


def fill_normal_bf16(seed: int, stream: int, shape, sigma: float = 1.0,
                     threads: int = 0) -> np.ndarray:
    """Deterministic bf16 bits of sigma * N(0, 1) (splitmix64 + Box-Muller)."""
    out = np.empty(shape, dtype=np.uint16)
    check(lib().llk_fill_normal_bf16(seed, stream, sigma, out.ctypes.data, out.size, threads))
    return out


def swiglu_scratch_size(M: int, N: int, K: int) -> int:
    return int(lib().llk_swiglu_scratch_size(M, N, K))


def describe_launch(op: str, M: int, N: int, K: int, x_aligned: bool = True,
                    accumulate: bool = False, out_f32: bool = False) -> dict:
    """The dispatcher's launch for op 'fused_swiglu' or 'matmul' (host only);
    accumulate: the plan of the C += A B matmul; out_f32: SwiGLU with an fp32
    result instead of bf16."""
    code = {"fused_swiglu": 0, "matmul": 3}[op]
    flags = (_lib.LLK_PLAN_X_ALIGNED if x_aligned else 0) | (
        _lib.LLK_PLAN_ACCUMULATE if accumulate else 0) | (_lib.LLK_PLAN_OUT_F32 if out_f32 else 0)
    p = _lib.LaunchPlan()
    check(lib().llk_describe_launch(code, M, N, K, flags, C.byref(p)))
    return {"kernel": ("small_m", "tile", "wide_tile", "decode_tile")[p.kernel], "splits": p.splits,
            "group_width": p.group_width, "pad_x": bool(p.pad_x), "workgroups": p.workgroups,
            "threads_per_workgroup": p.threads_per_workgroup, "launches": p.launches,
            "workspace_bytes": p.workspace_bytes, "head_blocks_n": p.head_blocks_n,
            "tile_columns": p.tile_columns}


def workspace_stats() -> tuple[int, int]:
    """(count, bytes) of the library-owned workspaces on the current device."""
    n, b = C.c_size_t(), C.c_size_t()
    check(lib().llk_workspace_stats(C.byref(n), C.byref(b)))
    return n.value, b.value


def workspace_trim() -> None:
    """Frees every idle, uncaptured library workspace of the current device."""
    check(lib().llk_workspace_trim())


def classify_m(M: int) -> int:
    return int(lib().llk_classify_m(M))


def set_tunable(name: str, value: int) -> None:
    check(lib().llk_set_tunable(name.encode(), value))


def get_tunable(name: str) -> int:
    v = C.c_int64()
    check(lib().llk_get_tunable(name.encode(), C.byref(v)))
    return v.value


def set_schedule_db(path: str | None) -> None:
    """Makes `path` the dispatcher's active schedule DB (None clears it)."""
    check(lib().llk_set_schedule_db(str(path).encode() if path else None))


def select_schedule(db_path: str, op_name: str, m_bucket: int):
    """(entry, n_matches, status) of the reference lookup semantics."""
    e = _lib.ScheduleEntry()
    n = C.c_int()
    st = lib().llk_select_schedule(db_path.encode(), op_name.encode(), m_bucket, C.byref(e),
                                   C.byref(n))
    return e, n.value, st


def device_info():
    name = C.create_string_buffer(64)
    cu, lds, clk = C.c_int(), C.c_int(), C.c_int()
    st = lib().llk_device_info(name, 64, C.byref(cu), C.byref(lds), C.byref(clk))
    return {"status": st, "arch": name.value.decode(), "cu_count": cu.value,
            "lds_bytes": lds.value, "clock_khz": clk.value}
