"""MI355X (gfx950) backend for DSLCompiler's fused SwiGLU / micro.mma path.

The product is ``libllk_gfx950.so`` (HIP kernels + C ABI, declared in
``include/llk/llk_abi.h``); this package builds it and binds it.
"""
from ._lib import LLKError, lib  # noqa: F401
from .cache import JitCache, KernelKey, WeightKey  # noqa: F401
from .ops import (PackedWeights, classify_m, describe_launch, device_info,  # noqa: F401
                  fill_normal_bf16, fused_swiglu, get_tunable, matmul, mlp, pack_device_layout,
                  select_schedule, set_schedule_db, set_tunable, swiglu_scratch_size,
                  workspace_stats, workspace_trim)

__all__ = ["JitCache", "KernelKey", "LLKError", "PackedWeights", "WeightKey", "classify_m",
           "describe_launch", "device_info", "fill_normal_bf16", "fused_swiglu", "get_tunable",
           "lib", "matmul", "mlp", "pack_device_layout", "select_schedule", "set_schedule_db",
           "set_tunable", "swiglu_scratch_size", "workspace_stats", "workspace_trim"]
