// mfma_tile.hip -- bf16 MFMA tile kernels for gfx950: the fused SwiGLU
// prefill kernel and the micro.mma GEMM.
//
// Computes  D^T = W^T X^T  on v_mfma_f32_16x16x32_bf16: the packed weight
// (n rows, k contiguous) is the MFMA A operand and the activation X (m rows,
// k contiguous) is the B operand, so each lane's four accumulator values are
// four consecutive n of one output row m (one 8- or 16-byte store).
//
// Workgroup: 256 threads (4 waves, 2 x 2).  Workgroup tile 256 m x 256
// MFMA rows:  GEMM -> 256 n;  SwiGLU -> 128 n of Wg + the same 128 n of Wu,
// so each wave holds the gate and up accumulators of the same (m, n) pairs
// and the SiLU(g)*u epilogue runs from registers (the reference's
// FuseDoubleContraction.cpp:175-199 epilogue, fused after the contraction of
// FuseDoubleContraction.cpp:155-173).  Wave tile: 128 m x 128 MFMA rows =
// 8 x 8 MFMA tiles, 256 fp32 accumulators per lane.
//
// K loop: 64 k per step, two LDS stages of 64 KiB (32 KiB weights + 32 KiB
// X), global loads for step kb+1 in flight during the MFMAs of step kb.
// LDS holds every operand as 1 KiB MFMA-ordered sub-blocks, so all LDS
// reads and writes are contiguous 1 KiB wave accesses.
#include "common.h"

namespace llk_gfx950 {

struct TileArgs {
  const uint16_t* x;   // [M, K] bf16, row stride ldx
  const uint8_t* w0;   // packed payload: Wg (swiglu) or B (gemm)
  const uint8_t* w1;   // packed payload: Wu (swiglu); unused for gemm
  void* y;             // [M, N] output, row stride ldy
  int64_t ldx, ldy;
  int M, N, K;
  int KB;              // K_pad / 64
  int NB;              // N_pad / 128 (packed n-blocks)
  int tiles_m, tiles_n;
};

constexpr int kThreads = 256;
constexpr int kTileM = 256;
constexpr int kStageBytes = 65536;
constexpr int kXOff = 32768;  // X sub-blocks inside a stage

// MODE 0: GEMM (C = X W);  MODE 1: fused SwiGLU.
// OUT_BF16: store bf16 (RNE) instead of fp32.
// XVEC: X rows are 16-byte aligned and K % 8 == 0 (vector loads);
//       otherwise X is read element by element.
// YVEC: Y rows allow a 4-element vector store (aligned base, ldy % 4 == 0).
template <int MODE, bool OUT_BF16, bool XVEC, bool YVEC>
__global__ __launch_bounds__(kThreads, 1) void mfma_tile_kernel(TileArgs a) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave & 1;
  const int wn = wave >> 1;

  const int total = a.tiles_m * a.tiles_n;
  const int tile = xcd_remap(blockIdx.x, total);
  const int tm = tile % a.tiles_m;  // m fastest: tiles sharing W columns
  const int tn = tile / a.tiles_m;  // run together on one XCD
  const int m0 = tm * kTileM;

  // Packed n-blocks feeding LDS weight slots 0 and 1.
  const uint8_t* wsrc[2];
  bool wvalid[2];
  if (MODE == 1) {
    wsrc[0] = a.w0 + (size_t)tn * a.KB * kBlockBytes;
    wsrc[1] = a.w1 + (size_t)tn * a.KB * kBlockBytes;
    wvalid[0] = wvalid[1] = true;
  } else {
    int nb0 = 2 * tn, nb1 = 2 * tn + 1;
    wsrc[0] = a.w0 + (size_t)nb0 * a.KB * kBlockBytes;
    wsrc[1] = a.w0 + (size_t)nb1 * a.KB * kBlockBytes;
    wvalid[0] = true;
    wvalid[1] = nb1 < a.NB;
  }

  // ---- global -> register staging: wave copies W sub-blocks
  // [wave*8, wave*8+8) of 32 and X sub-blocks [wave*8, wave*8+8) of 32.
  uint4 wreg[8], xreg[8];

  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int ws = wave * 8 + i;  // 0..31
      int b = ws >> 4, s = ws & 15;
      if (MODE == 1 || wvalid[b]) {
        const uint4* p = reinterpret_cast<const uint4*>(
            wsrc[b] + (size_t)kb * kBlockBytes + s * kSubBytes + lane * 16);
        wreg[i] = *p;
      } else {
        wreg[i] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int xs = wave * 8 + i;  // 0..31
      int kh = xs >> 4, m16 = xs & 15;
      int row = m0 + m16 * 16 + (lane & 15);
      int kk = kb * 64 + kh * 32 + (lane >> 4) * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (row < a.M) {
        const uint16_t* src = a.x + (size_t)row * a.ldx + kk;
        if (XVEC) {
          if (kk + 8 <= a.K) v = *reinterpret_cast<const uint4*>(src);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int t = 0; t < 8; ++t) e[t] = (kk + t < a.K) ? src[t] : (uint16_t)0;
          v.x = e[0] | ((uint32_t)e[1] << 16);
          v.y = e[2] | ((uint32_t)e[3] << 16);
          v.z = e[4] | ((uint32_t)e[5] << 16);
          v.w = e[6] | ((uint32_t)e[7] << 16);
        }
      }
      xreg[i] = v;
    }
  };

  auto lstore = [&](int buf) {
    uint8_t* st = smem + buf * kStageBytes;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int ws = wave * 8 + i;
      *reinterpret_cast<uint4*>(st + ws * kSubBytes + lane * 16) = wreg[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int xs = wave * 8 + i;
      *reinterpret_cast<uint4*>(st + kXOff + xs * kSubBytes + lane * 16) = xreg[i];
    }
  };

  f32x4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // LDS byte offset of the A operand i (0..7) for k half kh.
  auto a_off = [&](int i, int kh) -> int {
    if (MODE == 1) {
      int b = i >> 2;                // 0: gate, 1: up
      int n16 = wn * 4 + (i & 3);
      return b * kBlockBytes + (kh * 8 + n16) * kSubBytes;
    } else {
      return wn * kBlockBytes + (kh * 8 + i) * kSubBytes;
    }
  };

  gload(0);
  lstore(0);
  __syncthreads();

  for (int kb = 0; kb < a.KB; ++kb) {
    const int cur = kb & 1;
    const bool more = kb + 1 < a.KB;
    if (more) gload(kb + 1);
    const uint8_t* st = smem + cur * kStageBytes;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      bf16x8 bop[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        bop[j] = *reinterpret_cast<const bf16x8*>(
            st + kXOff + (kh * 16 + wm * 8 + j) * kSubBytes + lane * 16);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        bf16x8 aop = *reinterpret_cast<const bf16x8*>(st + a_off(i, kh) + lane * 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = mfma16(aop, bop[j], acc[i][j]);
      }
    }
    if (more) lstore(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds n = base + 4*(lane/16) + r, m = base + lane%16
  const int nq = 4 * (lane >> 4);
  const int mr = lane & 15;
  constexpr int NI = (MODE == 1) ? 4 : 8;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int n = (MODE == 1) ? (tn * 128 + wn * 64 + i * 16 + nq)
                              : (tn * 256 + wn * 128 + i * 16 + nq);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int m = m0 + wm * 128 + j * 16 + mr;
      if (m >= a.M || n >= a.N) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[r] = (MODE == 1) ? swiglu_act(acc[i][j][r], acc[i + 4][j][r]) : acc[i][j][r];
      if (OUT_BF16) {
        uint16_t* dst = reinterpret_cast<uint16_t*>(a.y) + (size_t)m * a.ldy + n;
        if (YVEC && n + 4 <= a.N) {
          u16x4 h = {f32_to_bf16_rne(v[0]), f32_to_bf16_rne(v[1]),
                     f32_to_bf16_rne(v[2]), f32_to_bf16_rne(v[3])};
          *reinterpret_cast<u16x4*>(dst) = h;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < a.N) dst[r] = f32_to_bf16_rne(v[r]);
        }
      } else {
        float* dst = reinterpret_cast<float*>(a.y) + (size_t)m * a.ldy + n;
        if (YVEC && n + 4 <= a.N) {
          *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < a.N) dst[r] = v[r];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
template <int MODE, bool OUT_BF16, bool XVEC, bool YVEC>
static hipError_t launch_t(const TileArgs& a, hipStream_t s) {
  auto fn = mfma_tile_kernel<MODE, OUT_BF16, XVEC, YVEC>;
  static bool attr_set = false;  // per instantiation; benign race (idempotent)
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       2 * kStageBytes);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  dim3 grid(a.tiles_m * a.tiles_n), block(kThreads);
  hipLaunchKernelGGL(fn, grid, block, 2 * kStageBytes, s, a);
  return hipGetLastError();
}

template <int MODE>
static hipError_t launch_mode(const TileArgs& a, bool out_bf16, bool xvec, bool yvec,
                              hipStream_t s) {
  if (out_bf16) {
    if (xvec) return yvec ? launch_t<MODE, true, true, true>(a, s) : launch_t<MODE, true, true, false>(a, s);
    return yvec ? launch_t<MODE, true, false, true>(a, s) : launch_t<MODE, true, false, false>(a, s);
  }
  if (xvec) return yvec ? launch_t<MODE, false, true, true>(a, s) : launch_t<MODE, false, true, false>(a, s);
  return yvec ? launch_t<MODE, false, false, true>(a, s) : launch_t<MODE, false, false, false>(a, s);
}

}  // namespace llk_gfx950

// Internal (not part of the C ABI): called by the host dispatch layer.
hipError_t llk_launch_tile(int mode, const uint16_t* x, int64_t ldx, const void* w0,
                           const void* w1, void* y, int64_t ldy, int M, int N, int K,
                           int KB, int NB, bool out_bf16, bool xvec, bool yvec,
                           hipStream_t s) {
  using namespace llk_gfx950;
  TileArgs a;
  a.x = x;
  a.w0 = static_cast<const uint8_t*>(w0);
  a.w1 = static_cast<const uint8_t*>(w1);
  a.y = y;
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.KB = KB;
  a.NB = NB;
  a.tiles_m = (M + kTileM - 1) / kTileM;
  a.tiles_n = mode == 1 ? NB : (NB + 1) / 2;
  if (mode == 1) return launch_mode<1>(a, out_bf16, xvec, yvec, s);
  return launch_mode<0>(a, out_bf16, xvec, yvec, s);
}
