"""MI355X (gfx950) backend for DSLCompiler's fused SwiGLU / micro.mma path.

The product is ``libllk_gfx950.so`` (HIP kernels + C ABI, declared in
``include/llk/llk_abi.h``); this package builds it and binds it.
"""
from ._lib import LLKError, lib  # noqa: F401
from .ops import (PackedWeights, classify_m, device_info, fill_normal_bf16,  # noqa: F401
                  fused_swiglu,
                  get_tunable, matmul, mlp, pack_device_layout, select_schedule, set_tunable,
                  swiglu_scratch_size)

__all__ = ["LLKError", "PackedWeights", "classify_m", "device_info", "fill_normal_bf16", "fused_swiglu",
           "get_tunable", "lib", "matmul", "mlp", "pack_device_layout", "select_schedule",
           "set_tunable", "swiglu_scratch_size"]
