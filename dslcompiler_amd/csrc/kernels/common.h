// common.h -- shared device definitions for the gfx950 kernels.
//
// Packed weight layout on the device ("MFMA operand order")
// ---------------------------------------------------------
// A bf16 weight matrix W[K, N] (row-major in the reference: PackedWeights.cpp
// copies rows k of length N) is stored transposed into 16 KiB blocks:
//
//   N_pad = ceil(N / 128) * 128,  K_pad = ceil(K / 64) * 64
//   block (nb, kb), nb < N_pad/128, kb < K_pad/64, at byte (nb*KB + kb)*16384
//   inside a block: 16 sub-blocks of 1 KiB, sub-block s = kq*4 + n32
//       (kq in 0..3 selects k quarter [16*kq, 16*kq+16), n32 in 0..3)
//   inside a sub-block: 64 lane slots of 16 bytes, slot l holds the 8 bf16
//       W[k][n] for n = nb*128 + n32*32 + (l % 32),
//                   k = kb*64 + kq*16 + (l / 32)*8 + t,  t = 0..7
//   entries outside [K, N] are zero.
//
// A 1 KiB sub-block is exactly the A operand of one v_mfma_f32_32x32x16_bf16
// (32 rows n x 16 k) in lane order, so one contiguous 1 KiB wave load (global
// or LDS) yields a ready operand with no bank conflicts, and a 16 KiB block
// streams contiguously from HBM.  A v_mfma_f32_16x16x32_bf16 A operand (16
// rows x 32 k) is two 256-byte halves of two such sub-blocks (k quarters q,
// q+1), so the same layout serves both MFMA forms (the small-M kernel uses
// the 32x32x16 form, the tile kernel the 16x16x32 one).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace llk_gfx950 {

constexpr int kPackN = 128;           // n per packed block
constexpr int kPackK = 64;            // k per packed block
constexpr int kSubBytes = 1024;       // one MFMA operand
constexpr int kBlockBytes = 16384;    // kPackN * kPackK * 2

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Buffer resource word 3 for raw (untyped) buffer access on gfx950.
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// IEEE round-to-nearest-even f32 -> bf16 (what arith.truncf produces);
// NaN stays a quiet NaN with its upper payload bits.  gfx950 does this in
// hardware (v_cvt_pk_bf16_f32, two values per instruction); on MI355X it
// equals the integer formulation  b += 0x7fff + ((b >> 16) & 1), NaN ->
// (b >> 16) | 0x40  for all 2^32 inputs.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_rne(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// SwiGLU epilogue of the fused reference path: g * (1 / (1 + exp(-g))) * u
// (FuseDoubleContraction.cpp:175-199, math.exp).  exp(-g) = 2^t with
// t = -g log2(e): v_exp_f32 on the rounded t, times 2^err for the rounding
// errors of the product and of log2(e) in fp32 (err < 2^-20, so 2^err =
// 1 + err ln2 to fp32 precision); the reciprocal is v_rcp_f32.  Eight VALU
// operations and two transcendentals against ~22 for expf and an IEEE
// divide, and on MI355X the same bound: at most 3 ulp from the correctly
// rounded result for every finite bf16 g with |g| <= 100 and 2^20 random
// fp32 g in [-20, 20].  Results below ~1e-36 (g < -87.3, where
// 1 / (1 + e) is subnormal) flush to +-0; g = +-inf, NaN give what the
// exact formula gives.  The exponent is computed from g clamped to
// [-88.75, 88.75] (one v_med3_f32): beyond it 2^t is already +inf or below
// 2^-128, so 1 / (1 + e) is exactly 0 or 1 as for the unclamped g, and t
// stays finite, so the error terms never meet inf - inf (the clamp replaced
// a test of t for infinity, one VALU operation more, with the same results).
__device__ __forceinline__ float swiglu_act(float g, float u) {
  constexpr float kL2E = 1.44269502162933349609375f;  // log2(e) rounded to fp32
  constexpr float kL2ELo = 1.925963033500011079e-8f;  // log2(e) - kL2E
  constexpr float kLn2 = 0.693147180559945309f;
  const float gc = __builtin_amdgcn_fmed3f(g, -88.75f, 88.75f);
  const float t = gc * -kL2E;
  float err = __builtin_fmaf(gc, -kL2E, -t);  // the product's rounding error
  err = __builtin_fmaf(gc, -kL2ELo, err);
  const float e = __builtin_amdgcn_exp2f(t) * __builtin_fmaf(err, kLn2, 1.0f);
  const float sig = __builtin_amdgcn_rcpf(1.0f + e);
  return (g * sig) * u;
}

// D[32x32] += A[32x16] B[16x32].  Lane l supplies A row l%32 / B column
// l%32, k values 8*(l/32) .. +8; it receives D column l%32, rows
// 8*(r/4) + 4*(l/32) + r%4 for r = 0..15.
__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Maps a linear workgroup id to a tile id so that the tiles processed
// concurrently on one XCD are contiguous in tile order.  Workgroups are
// dispatched round-robin over the 8 XCDs (bid % 8 picks the XCD), so
// bid -> (xcd = bid % 8, local = bid / 8) -> xcd's contiguous range.
__device__ __forceinline__ int xcd_remap(int bid, int total) {
  constexpr int kXcd = 8;
  int xcd = bid % kXcd;
  int local = bid / kXcd;
  int base = total / kXcd, extra = total % kXcd;
  return xcd * base + (xcd < extra ? xcd : extra) + local;
}

// Output element types (values of llk_dtype).
constexpr int kOutBF16 = 0, kOutF16 = 1, kOutF32 = 2;

__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  const _Float16 h = static_cast<_Float16>(f);  // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}

// Stores 4 consecutive n of output row m (OUT: bf16, fp16 or fp32; both
// 16-bit types rounded to nearest even), bounds-checked.
template <int OUT>
__device__ __forceinline__ void store4(void* y, int64_t ldy, int M, int N, int m, int n,
                                       const float (&v)[4], bool vec_ok) {
  if (m >= M || n >= N) return;
  if (OUT == kOutF16) {
    uint16_t* dst = reinterpret_cast<uint16_t*>(y) + (size_t)m * ldy + n;
    if (vec_ok && n + 4 <= N) {
      u16x4 h = {f32_to_f16_rne(v[0]), f32_to_f16_rne(v[1]), f32_to_f16_rne(v[2]),
                 f32_to_f16_rne(v[3])};
      *reinterpret_cast<u16x4*>(dst) = h;
    } else {
      for (int r = 0; r < 4; ++r)
        if (n + r < N) dst[r] = f32_to_f16_rne(v[r]);
    }
  } else if (OUT == kOutBF16) {
    uint16_t* dst = reinterpret_cast<uint16_t*>(y) + (size_t)m * ldy + n;
    if (vec_ok && n + 4 <= N) {
      *reinterpret_cast<uint2*>(dst) =
          make_uint2(f32x2_to_bf16x2_rne(v[0], v[1]), f32x2_to_bf16x2_rne(v[2], v[3]));
    } else {
      for (int r = 0; r < 4; ++r)
        if (n + r < N) dst[r] = f32_to_bf16_rne(v[r]);
    }
  } else {
    float* dst = reinterpret_cast<float*>(y) + (size_t)m * ldy + n;
    if (vec_ok && n + 4 <= N) {
      *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
    } else {
      for (int r = 0; r < 4; ++r)
        if (n + r < N) dst[r] = v[r];
    }
  }
}

// Accumulate mode of the GEMM (C += A B, the micro.mma / linalg.matmul
// contract): adds the output's existing values at the 4 consecutive n of row
// m, read in the output type, to v (fp32), before the store rounds it.
// Bounds and the vector condition as store4.
template <int OUT>
__device__ __forceinline__ void add_existing4(const void* y, int64_t ldy, int M, int N, int m,
                                              int n, float (&v)[4], bool vec_ok) {
  if (m >= M || n >= N) return;
  if (OUT == kOutF32) {
    const float* src = reinterpret_cast<const float*>(y) + (size_t)m * ldy + n;
    if (vec_ok && n + 4 <= N) {
      const f32x4 c = *reinterpret_cast<const f32x4*>(src);
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] += c[r];
    } else {
      for (int r = 0; r < 4; ++r)
        if (n + r < N) v[r] += src[r];
    }
  } else {
    auto widen = [](uint16_t h) {
      if constexpr (OUT == kOutF16) return static_cast<float>(__builtin_bit_cast(_Float16, h));
      else return bf16_bits_to_f32(h);
    };
    const uint16_t* src = reinterpret_cast<const uint16_t*>(y) + (size_t)m * ldy + n;
    if (vec_ok && n + 4 <= N) {
      const uint2 c = *reinterpret_cast<const uint2*>(src);
      v[0] += widen((uint16_t)(c.x & 0xffffu));
      v[1] += widen((uint16_t)(c.x >> 16));
      v[2] += widen((uint16_t)(c.y & 0xffffu));
      v[3] += widen((uint16_t)(c.y >> 16));
    } else {
      for (int r = 0; r < 4; ++r)
        if (n + r < N) v[r] += widen(src[r]);
    }
  }
}

// Raises the dynamic-LDS limit of kernel `fn` to `bytes`, once per device
// (the attribute belongs to the current device); `done` is the caller's
// per-kernel bit set of devices already configured.
inline hipError_t ensure_dynamic_lds(const void* fn, int bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = (dev >= 0 && dev < 64) ? (uint64_t)1 << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
  return e;
}

}  // namespace llk_gfx950
