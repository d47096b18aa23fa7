// fill_normal.h -- device-side bf16 N(0, sigma^2) fill for the HIP tools
// (their operands must look like the bench's, because the operand values
// set the board's power draw and so its clock).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels/common.h"

namespace llk_tools {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

// bf16 N(0, sigma^2) by Box-Muller on a hash of the element index.
__global__ void fill_normal_kernel(uint16_t* p, size_t n, uint64_t seed, float sigma) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint64_t h = mix64(seed + 0x9e3779b97f4a7c15ULL * (i + 1));
    const float u1 = ((float)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);
    const float u2 = (float)(h & 0xffffff) * (1.0f / 16777216.0f);
    const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.2831853f * u2) * sigma;
    p[i] = llk_gfx950::f32_to_bf16_rne(z);
  }
}

}  // namespace llk_tools
