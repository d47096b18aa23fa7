// mfma_tile.hip -- bf16 MFMA tile kernels for gfx950: the fused SwiGLU
// prefill kernel and the micro.mma GEMM.
//
// Computes  D^T = W^T X^T  on v_mfma_f32_32x32x16_bf16: the packed weight
// (n rows, k contiguous) is the MFMA A operand and the activation X (m rows,
// k contiguous) is the B operand, so each lane's accumulators are runs of
// four consecutive n of one output row m (8- or 16-byte stores).
//
// Workgroup: 256 threads (4 waves, 2 x 2).  Workgroup tile 256 m x 256
// MFMA rows:  GEMM -> 256 n;  SwiGLU -> 128 n of Wg + the same 128 n of Wu,
// so each wave holds the gate and up accumulators of the same (m, n) pairs
// and the SiLU(g)*u epilogue runs from registers (the reference's
// FuseDoubleContraction.cpp:175-199 epilogue, fused after the contraction of
// FuseDoubleContraction.cpp:155-173).  Wave tile: 128 m x 128 MFMA rows =
// 4 x 4 MFMA tiles of 32 x 32, 256 fp32 accumulators per lane (AGPRs).
//
// K loop: 64 k per step, two LDS stages of 64 KiB (32 KiB weights + 32 KiB
// X).  Operands go straight from memory into LDS (buffer_load_dwordx4 ...
// lds), so step kb+1 streams in while the 64 MFMAs of step kb run.  LDS
// holds every operand as a 1 KiB MFMA-ordered sub-block: every LDS read is
// one contiguous 1 KiB wave access (no bank conflicts).
//
// X must be padded to whole 64-k steps with 16-byte aligned rows (the host
// copies it into a padded buffer otherwise); rows >= M read as zero through
// the buffer resource's range check.
#include "common.h"

namespace llk_gfx950 {

struct TileArgs {
  const uint16_t* x;   // [M, K_pad] bf16, row stride ldx (multiple of 8)
  const uint8_t* w0;   // packed payload: Wg (swiglu) or B (gemm)
  const uint8_t* w1;   // packed payload: Wu (swiglu); unused for gemm
  void* y;             // [M, N] output, row stride ldy
  int64_t ldx, ldy;
  int M, N;
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
// YVEC: Y rows allow a 4-element vector store (aligned base, ldy % 4 == 0).
template <int MODE, bool OUT_BF16, bool YVEC>
__global__ __launch_bounds__(kThreads, 1) void mfma_tile_kernel(TileArgs a) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int wm = wave & 1;
  const int wn = wave >> 1;

  const int total = a.tiles_m * a.tiles_n;
  const int tile = xcd_remap(blockIdx.x, total);
  const int tm = tile % a.tiles_m;  // m fastest: tiles sharing W columns
  const int tn = tile / a.tiles_m;  // run together on one XCD
  const int m0 = tm * kTileM;

  // ---- operand streams ----------------------------------------------------
  // LDS weight slot b (0, 1) holds one packed n-block.  Waves 0-1 fill slot 0
  // and waves 2-3 slot 1: wave w copies sub-blocks (w&1)*8 .. +8 of its
  // slot's block, 8 KiB contiguous in the payload.  Every wave also copies
  // the 8 X sub-blocks of k quarter kq = w (rows m0 + 32 i + lane%32).
  const int wslot = wave >> 1;
  const uint8_t* wpanel;
  bool wvalid = true;
  if (MODE == 1) {
    wpanel = (wslot ? a.w1 : a.w0) + (size_t)tn * a.KB * kBlockBytes;
  } else {
    const int nb = 2 * tn + wslot;
    wvalid = nb < a.NB;
    wpanel = a.w0 + (size_t)(wvalid ? nb : 0) * a.KB * kBlockBytes;
  }
  wpanel += (wave & 1) * 8 * kSubBytes;
  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(wpanel), (short)0, a.KB * kBlockBytes, kBufferWord3);
  const int w_voff = lane * 16;

  // The X resource starts at row m0 and ends at row M: rows >= M read zero.
  const int rows_left = a.M - m0;
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.x) + (size_t)m0 * a.ldx, (short)0,
      (int)((int64_t)rows_left * a.ldx * 2), kBufferWord3);
  const int x_voff = ((lane & 31) * (int)a.ldx + wave * 16 + (lane >> 5) * 8) * 2;
  const int x_rowstep = 32 * (int)a.ldx * 2;

  auto dma_issue = [&](int kb, int buf) {
    uint8_t* st = smem + buf * kStageBytes;
    if (MODE == 1 || wvalid) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wrsrc, (lds_ptr_t)(st + (wave * 8 + i) * kSubBytes),
                                                 16, w_voff, kb * kBlockBytes + i * kSubBytes, 0,
                                                 0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // whole offset in the VGPR operand so the range check covers it
      const int voff = x_voff + i * x_rowstep + kb * 128;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xrsrc, (lds_ptr_t)(st + kXOff + (wave * 8 + i) * kSubBytes), 16, voff, 0, 0, 0);
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // LDS byte offsets (within a stage) of the A operand i and B operand j of
  // k quarter kq.
  auto a_off = [&](int kq, int i) -> int {
    if (MODE == 1) return (i >> 1) * kBlockBytes + (kq * 4 + wn * 2 + (i & 1)) * kSubBytes;
    return wn * kBlockBytes + (kq * 4 + i) * kSubBytes;
  };
  auto b_off = [&](int kq, int j) -> int { return kXOff + (kq * 8 + wm * 4 + j) * kSubBytes; };

  if (MODE == 0 && !wvalid) {  // missing second block of an odd-NB GEMM: zeros
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        *reinterpret_cast<uint4*>(smem + s * kStageBytes + (wave * 8 + i) * kSubBytes + lane * 16) =
            make_uint4(0, 0, 0, 0);
  }
  dma_issue(0, 0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's LDS DMA landed
  __syncthreads();

  for (int kb = 0; kb < a.KB; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < a.KB) dma_issue(kb + 1, cur ^ 1);
    const uint8_t* st = smem + cur * kStageBytes + lane * 16;
    auto rd = [&](int off) { return *reinterpret_cast<const bf16x8*>(st + off); };
    // Operand schedule: the 8 operands of k quarter kq are in registers while
    // the next quarter's 8 are read, one LDS read per two MFMAs.
    bf16x8 acur[4], bcur[4], anxt[4], bnxt[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) bcur[j] = rd(b_off(0, j));
#pragma unroll
    for (int i = 0; i < 4; ++i) acur[i] = rd(a_off(0, i));
#pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (kq < 3 && j == 0) bnxt[i] = rd(b_off(kq + 1, i));
          if (kq < 3 && j == 2) anxt[i] = rd(a_off(kq + 1, i));
          acc[i][j] = mfma32(acur[i], bcur[j], acc[i][j]);
          if (kq < 3 && (j == 0 || j == 2)) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // 2 MFMAs
          }
        }
      }
      if (kq < 3) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acur[q] = anxt[q];
          bcur[q] = bnxt[q];
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): next stage landed
    __syncthreads();
  }

  // ---- epilogue: lane holds m = base + lane%32, n = base + 8*(r/4) +
  // 4*(lane/32) + r%4 for its 16 values r of each 32 x 32 tile.
  const int h4 = 4 * (lane >> 5);
  const int mr = lane & 31;
  constexpr int NI = (MODE == 1) ? 2 : 4;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + wm * 128 + j * 32 + mr;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = (MODE == 1) ? (tn * 128 + wn * 64 + i * 32 + 8 * g + h4)
                                  : (tn * 256 + wn * 128 + i * 32 + 8 * g + h4);
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          v[q] = (MODE == 1) ? swiglu_act(acc[i][j][4 * g + q], acc[i + 2][j][4 * g + q])
                             : acc[i][j][4 * g + q];
        store4<OUT_BF16>(a.y, a.ldy, a.M, a.N, m, n, v, YVEC);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
template <int MODE, bool OUT_BF16, bool YVEC>
static hipError_t launch_t(const TileArgs& a, hipStream_t s) {
  auto fn = mfma_tile_kernel<MODE, OUT_BF16, YVEC>;
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
static hipError_t launch_mode(const TileArgs& a, bool out_bf16, bool yvec, hipStream_t s) {
  if (out_bf16) return yvec ? launch_t<MODE, true, true>(a, s) : launch_t<MODE, true, false>(a, s);
  return yvec ? launch_t<MODE, false, true>(a, s) : launch_t<MODE, false, false>(a, s);
}

}  // namespace llk_gfx950

// Largest X span (bytes, rows padded to whole tiles) the 32-bit buffer
// offsets of the tile kernel can address.
bool llk_tile_x_fits(int M, int64_t ldx) {
  const int64_t rows = ((int64_t)M + 255) / 256 * 256;
  return rows * ldx * 2 < ((int64_t)1 << 31);
}

// Internal (not part of the C ABI).  x: [M, 64*KB] bf16 with ldx % 8 == 0,
// 16-byte aligned, columns >= K zero; llk_tile_x_fits(M, ldx) must hold.
hipError_t llk_launch_tile(int mode, const uint16_t* x, int64_t ldx, const void* w0,
                           const void* w1, void* y, int64_t ldy, int M, int N, int KB, int NB,
                           bool out_bf16, bool yvec, hipStream_t s) {
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
  a.KB = KB;
  a.NB = NB;
  a.tiles_m = (M + kTileM - 1) / kTileM;
  a.tiles_n = mode == 1 ? NB : (NB + 1) / 2;
  if (mode == 1) return launch_mode<1>(a, out_bf16, yvec, s);
  return launch_mode<0>(a, out_bf16, yvec, s);
}
