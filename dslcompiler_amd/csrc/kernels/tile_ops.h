// tile_ops.h -- device building blocks shared by the MFMA kernels
// (mfma_tile.hip, swiglu_wide.hip, the decode tile kernel of
// swiglu_decode.hip): wait counters, buffer resources, the LDS-DMA loads, the
// in-place MFMA and the padding around it.
#pragma once

#include "common.h"

namespace llk_gfx950 {

// s_waitcnt with vmcnt(n) (n < 64) and the other counters left alone.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Raw buffer resource (stride 0) over [base, base + bytes), wave-uniform.
__device__ __forceinline__ u32x4 buffer_rsrc(const void* base, int bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  u32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((uint32_t)b);
  r.y = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32) & 0xffffu);  // stride 0
  r.z = __builtin_amdgcn_readfirstlane((uint32_t)bytes);
  r.w = kBufferWord3;
  return r;
}

// One buffer_load_dwordx4 ... lds: 16 bytes per lane from the resource at
// voff (per lane, range-checked: out of range reads zero) + soff (uniform)
// into LDS at lds + 16 * lane.  Issued from inline assembly so that the
// compiler's LDS-DMA alias tracking, which cannot tell ring slots indexed
// at run time apart, adds no waits of its own: the kernels' explicit vmcnt
// waits order every DMA against the LDS reads of its stage.
// M0 is clobbered explicitly; the compiler uses M0 for nothing else in these
// kernels (checked on the code object by tests/test_isa_cpu.py), so its
// warning about clobbering a reserved register is silenced here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const u32x4& rsrc, int voff, int soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voff), "s"(rsrc), "s"(soff) : "memory", "m0");
}
// The same load, non-temporal (`nt`): for data each workgroup reads once
// and no other workgroup reads again (weights when there is one m tile), so
// that it streams past L2 rather than evicting what is reused there (X).
// Measured per kernel: faster for the decode tile kernel and the wide SwiGLU
// kernel's gathered 256-byte runs, slower for mfma_tile_kernel's 8 KiB
// weight stages (k-split GEMM M = 200 / 255, SwiGLU M = 100: 6-16%), which
// keep ordinary loads.
__device__ __forceinline__ void dma16_nt(const u32x4& rsrc, int voff, int soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
               :: "s"(lds), "v"(voff), "s"(rsrc), "s"(soff) : "memory", "m0");
}
// The same load in two statements, for the K loops: set_m0 writes the LDS
// address and dma16_m0 issues the load that reads it.  The caller puts at
// least one instruction (an MFMA) between them -- the wait state M0 needs
// before an LDS-DMA load -- so that no s_nop is needed and the instructions
// of a refill (offset add, M0 write, load) never queue up between two
// MFMAs: a wave issues at most one instruction per 4 cycles, so only three
// others fit in the 16 cycles of one MFMA.  Nothing else in these kernels
// writes M0 between the two (checked by tests/test_isa_cpu.py).
__device__ __forceinline__ void set_m0(uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0" :: "s"(lds) : "m0");
}
__device__ __forceinline__ void dma16_m0(const u32x4& rsrc, int voff, int soff) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" :: "v"(voff), "s"(rsrc), "s"(soff)
               : "memory");
}
__device__ __forceinline__ void dma16_m0_nt(const u32x4& rsrc, int voff, int soff) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen nt lds" :: "v"(voff), "s"(rsrc), "s"(soff)
               : "memory");
}
#pragma clang diagnostic pop

// LDS byte address of a pointer into the kernel's dynamic shared memory.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  return (uint32_t)(uintptr_t)(lds_ptr_t)(const_cast<uint8_t*>(p));
}

// acc += A B on v_mfma_f32_16x16x32_bf16, accumulating in place in the
// accumulator's AGPRs: through the builtin the register allocator routes a
// varying set of the accumulators through temporary AGPRs every stage (up to
// 4 AGPR moves and s_nops per MFMA).  Lane l supplies A row l%16 / B column
// l%16 with k values 8*(l/16) .. +8 and receives D column l%16, rows
// 4*(l/16) + 0..3.
__device__ __forceinline__ void mfma16(const bf16x8& a, const bf16x8& b, f32x4& acc) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// The same with the accumulator in VGPRs (tiles with more accumulators than
// the 256 AGPRs of a wave).
__device__ __forceinline__ void mfma16_v(const bf16x8& a, const bf16x8& b, f32x4& acc) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}

// 64 wait states: more than a 16x16x32 MFMA needs before a VALU instruction
// may read its result (or before an MFMA may read an AGPR a VALU wrote).
__device__ __forceinline__ void mfma_drain() {
  asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15");
}

}  // namespace llk_gfx950
