// pack.hip -- repack a row-major bf16 W[K, N] (device memory) into the
// MFMA-ordered packed payload described in common.h.  One thread produces
// one 16-byte lane slot (8 consecutive k of one n); entries outside [K, N]
// are written as zero, so the whole payload is defined.
#include "common.h"
#include "launch.h"

namespace llk_gfx950 {

// One workgroup per packed 16 KiB block (nb, kb): the 64 x 128 source tile
// W[64 kb .. +64, 128 nb .. +128] is read row by row (16 lanes per row, 16
// bytes each: 256 contiguous bytes of one k), staged in LDS, and written as
// the block's 1024 lane slots (8 consecutive k of one n, 16 bytes) in slot
// order, so both the reads and the writes stream whole cache lines.
// Entries outside [K, N] are zero.  vec: W's rows allow 16-byte loads
// (aligned base, ld % 8 == 0).
__global__ __launch_bounds__(256) void pack_tile_kernel(const uint16_t* __restrict__ w,
                                                        int64_t ld, int K, int N, int KB,
                                                        int vec, uint32_t* __restrict__ out) {
  constexpr int kPitch = kPackN + 8;  // padded LDS row (u16): spreads a column over banks
  __shared__ uint16_t tile[kPackK * kPitch];
  const int kb = (int)(blockIdx.x % (unsigned)KB);
  const int nb = (int)(blockIdx.x / (unsigned)KB);
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int c = (int)threadIdx.x + it * 256;  // 16-byte chunk: row c / 16, 8 n at 8 (c % 16)
    const int r = c >> 4, n = nb * kPackN + (c & 15) * 8, k = kb * kPackK + r;
    uint16_t* dst = tile + r * kPitch + (c & 15) * 8;
    const uint16_t* src = w + (int64_t)k * ld + n;
    if (vec && k < K && n + 8 <= N) {
      *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) dst[t] = (k < K && n + t < N) ? src[t] : (uint16_t)0;
    }
  }
  __syncthreads();
  uint4* const ob = reinterpret_cast<uint4*>(out) + (size_t)blockIdx.x * 1024;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    // slot = sub-block s (k quarter s / 4, 32-n group s % 4) * 64 + lane l
    const int slot = (int)threadIdx.x + it * 256;
    const int s = slot >> 6, l = slot & 63;
    const int nn = (s & 3) * 32 + (l & 31), kk = (s >> 2) * 16 + (l >> 5) * 8;
    uint32_t v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      v[q] = (uint32_t)tile[(kk + 2 * q) * kPitch + nn] |
             ((uint32_t)tile[(kk + 2 * q + 1) * kPitch + nn] << 16);
    ob[slot] = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

static const char* pack_tile_symbol() { return "_ZN10llk_gfx95016pack_tile_kernelEPKtliiiiPj"; }

}  // namespace llk_gfx950

// W: bf16 [K, N] in device memory, row stride ld; out: KB * NB * 16 KiB.
hipError_t llk_launch_pack(const uint16_t* w, int64_t ld, int K, int N, int KB, int NB,
                           void* out, const llk::ModuleFns* mod, hipStream_t s) {
  using namespace llk_gfx950;
  const int64_t blocks = (int64_t)NB * KB;
  if (blocks <= 0) return hipSuccess;
  const int vec = (reinterpret_cast<uintptr_t>(w) % 16 == 0 && ld % 8 == 0) ? 1 : 0;
  return launch_kernel(mod, reinterpret_cast<const void*>(pack_tile_kernel), &pack_tile_symbol,
                       dim3((unsigned)blocks), dim3(256), 0, s, w, ld, K, N, KB, vec,
                       static_cast<uint32_t*>(out));
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
