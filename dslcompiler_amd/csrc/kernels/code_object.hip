// code_object.hip -- one operation's gfx950 code object (built by
// dslcompiler_amd/build.py with hipcc --genco and LLK_CO_OP = 1 for the
// fused SwiGLU, 0 for the GEMM): the same kernel sources as the library,
// whose launchers, compiled here for the device only, instantiate the
// kernels of that operation.  Loaded at run time by code_object.cpp.
#ifndef LLK_CO_OP
#error "LLK_CO_OP must be 0 (GEMM) or 1 (fused SwiGLU)"
#endif
#include "mfma_tile.hip"
#include "swiglu_wide.hip"
#include "pack.hip"
#include "swiglu_decode.hip"
