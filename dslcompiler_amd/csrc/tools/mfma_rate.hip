// llk-mfma-rate -- register-only throughput of the two bf16 MFMA forms on
// gfx950, v_mfma_f32_32x32x16_bf16 and v_mfma_f32_16x16x32_bf16, with the
// tile kernel's register budget (one wave per SIMD, 256 accumulators per
// lane in AGPRs, 16 operand registers) and two operand fills: bf16 N(0,1)
// and one constant value.  The operand values set the board's power draw
// and so its clock, which is why the 16x16x32 form (half the accumulator
// register traffic per flop) sustains more on random data.
//
//   llk-mfma-rate [iterations]
//
// Every MFMA is issued from inline assembly with its accumulator tied in
// place (through the builtin the register allocator routes accumulators of
// the 16x16x32 loop through temporaries, which would measure the copies).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "kernels/common.h"
#include "tools/fill_normal.h"

namespace {

using llk_gfx950::bf16x8;
using llk_gfx950::f32x16;
using llk_gfx950::f32x4;

constexpr int kWorkgroups = 1024;  // 4 per CU
constexpr int kThreads = 256;

// One loop iteration: 32 MFMAs of 32x32x16 or 64 of 16x16x32 (both 2^20
// flops per wave), alternating between two operand sets.
template <bool K16>
__global__ __launch_bounds__(kThreads, 1) void mfma_rate_kernel(const bf16x8* src, float* out,
                                                               int iters) {
  const size_t base = ((size_t)blockIdx.x * kThreads + threadIdx.x) * 16;
  bf16x8 a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = src[base + i];
    b[i] = src[base + 8 + i];
  }
  float s = 0.0f;
  if constexpr (!K16) {
    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                         : "+a"(acc[i][j]) : "v"(a[4 * h + i]), "v"(b[4 * h + j]));
    asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15");
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        asm volatile("" : "+a"(acc[i][j]));
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[i][j][r];
      }
  } else {
    f32x4 acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{};
    for (int it = 0; it < iters; ++it)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                         : "+a"(acc[i][4 * h + j]) : "v"(a[i]), "v"(b[4 * h + j]));
    asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15");
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        asm volatile("" : "+a"(acc[i][j]));
#pragma unroll
        for (int r = 0; r < 4; ++r) s += acc[i][j][r];
      }
  }
  out[(size_t)blockIdx.x * kThreads + threadIdx.x] = s;
}

__global__ void fill_const_kernel(uint16_t* p, size_t n, uint16_t v) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

bool check(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
  return false;
}

template <bool K16>
bool run(const char* name, const bf16x8* src, float* out, int iters) {
  hipEvent_t e0, e1;
  if (!check(hipEventCreate(&e0), "event") || !check(hipEventCreate(&e1), "event")) return false;
  // warm-up past the clock ramp, then timed launches
  for (int i = 0; i < 30; ++i)
    hipLaunchKernelGGL(mfma_rate_kernel<K16>, dim3(kWorkgroups), dim3(kThreads), 0, 0, src, out, iters);
  if (!check(hipDeviceSynchronize(), "warm-up")) return false;
  const int reps = 20;
  if (!check(hipEventRecord(e0, 0), "event record")) return false;
  for (int i = 0; i < reps; ++i)
    hipLaunchKernelGGL(mfma_rate_kernel<K16>, dim3(kWorkgroups), dim3(kThreads), 0, 0, src, out, iters);
  if (!check(hipEventRecord(e1, 0), "event record") ||
      !check(hipEventSynchronize(e1), "timed launches"))
    return false;
  float ms = 0.0f;
  if (!check(hipEventElapsedTime(&ms, e0, e1), "elapsed time")) return false;
  const double flop = (double)kWorkgroups * (kThreads / 64) * iters * 32 * 32768.0;
  const double us = ms * 1e3 / reps;
  std::printf("%-28s %9.1f us per launch  %7.1f TFLOP/s\n", name, us, flop / (us * 1e-6) / 1e12);
  std::fflush(stdout);
  return check(hipEventDestroy(e0), "event") && check(hipEventDestroy(e1), "event");
}

}  // namespace

int main(int argc, char** argv) {
  const int iters = argc > 1 ? std::atoi(argv[1]) : 2000;
  if (iters < 1 || iters > 100000) {
    std::fprintf(stderr, "iterations must be in 1..100000\n");
    return 2;
  }
  const size_t n = (size_t)kWorkgroups * kThreads * 16 * 8;  // bf16 operands, 16 per lane
  uint16_t* src = nullptr;
  float* out = nullptr;
  if (!check(hipMalloc(&src, n * 2), "hipMalloc") ||
      !check(hipMalloc(&out, (size_t)kWorkgroups * kThreads * sizeof(float)), "hipMalloc"))
    return 1;
  const bf16x8* ops = reinterpret_cast<const bf16x8*>(src);
  hipLaunchKernelGGL(llk_tools::fill_normal_kernel, dim3(2048), dim3(256), 0, 0, src, n, 7ull, 1.0f);
  if (!check(hipDeviceSynchronize(), "fill")) return 1;
  if (!run<false>("32x32x16 bf16, N(0,1)", ops, out, iters)) return 1;
  if (!run<true>("16x16x32 bf16, N(0,1)", ops, out, iters)) return 1;
  hipLaunchKernelGGL(fill_const_kernel, dim3(2048), dim3(256), 0, 0, src, n, (uint16_t)0x3C3C);
  if (!check(hipDeviceSynchronize(), "fill")) return 1;
  if (!run<false>("32x32x16 bf16, constant", ops, out, iters)) return 1;
  if (!run<true>("16x16x32 bf16, constant", ops, out, iters)) return 1;
  return check(hipFree(src), "hipFree") && check(hipFree(out), "hipFree") ? 0 : 1;
}
