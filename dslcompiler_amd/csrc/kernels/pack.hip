// pack.hip -- repack a row-major bf16 W[K, N] (device memory) into the
// MFMA-ordered packed payload described in common.h.  One thread produces
// one 16-byte lane slot (8 consecutive k of one n); entries outside [K, N]
// are written as zero, so the whole payload is defined.
#include "common.h"
#include "launch.h"

namespace llk_gfx950 {

__global__ __launch_bounds__(256) void pack_weights_kernel(const uint16_t* __restrict__ w,
                                                           int64_t ld, int K, int N, int KB,
                                                           int64_t slots, uint4* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= slots) return;
  // slot index = ((nb*KB + kb)*16 + s)*64 + l
  const int l = (int)(idx & 63);
  const int s = (int)((idx >> 6) & 15);
  const int64_t blk = idx >> 10;
  const int kb = (int)(blk % KB);
  const int nb = (int)(blk / KB);
  const int kq = s >> 2, n32 = s & 3;
  const int n = nb * kPackN + n32 * 32 + (l & 31);
  const int k0 = kb * kPackK + kq * 16 + (l >> 5) * 8;
  uint16_t e[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int k = k0 + t;
    e[t] = (n < N && k < K) ? w[(int64_t)k * ld + n] : (uint16_t)0;
  }
  uint4 v;
  v.x = e[0] | ((uint32_t)e[1] << 16);
  v.y = e[2] | ((uint32_t)e[3] << 16);
  v.z = e[4] | ((uint32_t)e[5] << 16);
  v.w = e[6] | ((uint32_t)e[7] << 16);
  out[idx] = v;
}

}  // namespace llk_gfx950

hipError_t llk_launch_pack(const uint16_t* w, int64_t ld, int K, int N, int KB, int NB,
                           void* out, hipStream_t s) {
  using namespace llk_gfx950;
  const int64_t slots = (int64_t)NB * KB * 1024;
  const int64_t blocks = (slots + 255) / 256;
  hipLaunchKernelGGL(pack_weights_kernel, dim3((unsigned)blocks), dim3(256), 0, s, w, ld, K, N,
                     KB, slots, static_cast<uint4*>(out));
  return hipGetLastError();
}

// Copies X[M, K] (any row stride, any alignment) into a dense [M, ldo]
// buffer, ldo a multiple of 64, zero-filling columns K .. ldo-1: the layout
// the direct-to-LDS tile kernel reads.  One thread per 8 output columns.
__global__ __launch_bounds__(256) void pad_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                       int M, int K, uint16_t* __restrict__ out,
                                                       int64_t ldo) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_row = ldo / 8;
  if (idx >= (int64_t)M * per_row) return;
  const int64_t m = idx / per_row;
  const int c0 = (int)(idx % per_row) * 8;
  uint16_t e[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) e[t] = (c0 + t < K) ? x[m * ldx + c0 + t] : (uint16_t)0;
  uint4 v;
  v.x = e[0] | ((uint32_t)e[1] << 16);
  v.y = e[2] | ((uint32_t)e[3] << 16);
  v.z = e[4] | ((uint32_t)e[5] << 16);
  v.w = e[6] | ((uint32_t)e[7] << 16);
  *reinterpret_cast<uint4*>(out + m * ldo + c0) = v;
}

static const char* pad_rows_symbol() { return "_Z15pad_rows_kernelPKtliiPtl"; }

// mod: a loaded per-operation code object, or null for the library's own
// kernels (likewise llk_launch_zero_rows).
hipError_t llk_launch_pad_rows(const uint16_t* x, int64_t ldx, int M, int K, uint16_t* out,
                               int64_t ldo, const llk::ModuleFns* mod, hipStream_t s) {
  const int64_t threads = (int64_t)M * (ldo / 8);
  if (threads == 0) return hipSuccess;
  return llk_gfx950::launch_kernel(mod, reinterpret_cast<const void*>(pad_rows_kernel),
                                   &pad_rows_symbol, dim3((unsigned)((threads + 255) / 256)),
                                   dim3(256), 0, s, x, ldx, M, K, out, ldo);
}

// Writes zero to every element of a strided [M, N] matrix of 2- or 4-byte
// elements (an empty reduction, K == 0: SiLU(0) * 0 = +0 and C = 0), as a
// kernel rather than hipMemset2DAsync so that the call is safe inside
// captured HIP graphs.  One thread per element.
__global__ __launch_bounds__(256) void zero_rows_kernel(uint8_t* __restrict__ y, int64_t ld_bytes,
                                                        int64_t N, int elem_bytes, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int64_t m = idx / N, n = idx - m * N;
  uint8_t* p = y + m * ld_bytes + n * elem_bytes;
  if (elem_bytes == 4)
    *reinterpret_cast<uint32_t*>(p) = 0u;
  else
    *reinterpret_cast<uint16_t*>(p) = 0;
}

static const char* zero_rows_symbol() { return "_Z16zero_rows_kernelPhllil"; }

hipError_t llk_launch_zero_rows(void* y, int64_t ld_elems, int64_t M, int64_t N, int elem_bytes,
                                const llk::ModuleFns* mod, hipStream_t s) {
  const int64_t total = M * N;
  if (total <= 0) return hipSuccess;
  return llk_gfx950::launch_kernel(mod, reinterpret_cast<const void*>(zero_rows_kernel),
                                   &zero_rows_symbol, dim3((unsigned)((total + 255) / 256)),
                                   dim3(256), 0, s, static_cast<uint8_t*>(y),
                                   (int64_t)(ld_elems * elem_bytes), N, elem_bytes, total);
}

// Zeroes `words` 32-bit words (the two-piece k split's arrival counters in
// a caller's scratch), as a kernel so that the call can be captured in a
// HIP graph.
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* __restrict__ p, int64_t words) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < words) p[i] = 0u;
}

static const char* zero_words_symbol() { return "_Z17zero_words_kernelPjl"; }

hipError_t llk_launch_zero(void* p, size_t bytes, const llk::ModuleFns* mod, hipStream_t s) {
  const int64_t words = (int64_t)(bytes / 4);
  if (words <= 0) return hipSuccess;
  return llk_gfx950::launch_kernel(mod, reinterpret_cast<const void*>(zero_words_kernel),
                                   &zero_words_symbol, dim3((unsigned)((words + 255) / 256)),
                                   dim3(256), 0, s, static_cast<uint32_t*>(p), words);
}
