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
// LOAD: how operands reach LDS.
//   kLoadDma   -- direct global->LDS: weights with global_load_lds_dwordx4,
//                 X with buffer_load_dwordx4 ... lds through a buffer
//                 resource that ends at row M, so rows >= M read as zero.
//                 Needs K % 64 == 0, 16-byte aligned X rows, and X within a
//                 32-bit byte offset.
//   kLoadVec   -- register staging, 16-byte X loads (K % 8 == 0, aligned).
//   kLoadElem  -- register staging, X read element by element (any K).
// YVEC: Y rows allow a 4-element vector store (aligned base, ldy % 4 == 0).
constexpr int kLoadDma = 0, kLoadVec = 1, kLoadElem = 2;

typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int MODE, bool OUT_BF16, int LOAD, bool YVEC>
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

  // LDS weight slot b (0, 1) holds one packed n-block; waves 0-1 copy slot 0
  // and waves 2-3 slot 1, so each wave streams from a single block:
  // sub-blocks (wave&1)*8 .. +8.  Every wave also copies X sub-blocks
  // [wave*8, wave*8+8) of 32 (sub-block xs: k half xs/16, 16 rows xs%16).
  const int wslot = wave >> 1;
  const uint8_t* wmy;
  bool wmy_valid = true;
  if (MODE == 1) {
    wmy = (wslot ? a.w1 : a.w0) + (size_t)tn * a.KB * kBlockBytes;
  } else {
    const int nb = 2 * tn + wslot;
    wmy_valid = nb < a.NB;
    wmy = a.w0 + (size_t)(wmy_valid ? nb : 0) * a.KB * kBlockBytes;
  }
  wmy += (wave & 1) * 8 * kSubBytes + lane * 16;

  // X element offset of this lane's first sub-block row / k group.
  const int xrow0 = m0 + (lane & 15);
  const int xk0 = (lane >> 4) * 8;

  // ---- direct-to-LDS path -------------------------------------------------
  // Both streams go through buffer resources whose base is wave-uniform, so
  // a lane needs one offset VGPR per stream and each k step adds a scalar.
  // Weights: the wave's 8 sub-blocks of block (nb, kb) start at
  //   panel + kb*16 KiB + (wave&1)*8 KiB, lane slot at + lane*16.
  // X: the wave copies sub-blocks xs = wave*8+i, i.e. k half kh = wave>>1
  //   and rows m0 + (wave&1)*128 + i*16 + lane%16; the resource starts at
  //   the wave's first row and ends at row M, so rows >= M read as zero.
  __amdgpu_buffer_rsrc_t wrsrc, xrsrc;
  int w_voff = 0, x_voff = 0;
  const int xrow_w = m0 + (wave & 1) * 128;  // first X row of this wave
  if (LOAD == kLoadDma) {
    const uint8_t* wpanel = wmy - lane * 16;  // wave-uniform
    wrsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(wpanel), (short)0,
                                              a.KB * kBlockBytes, 0x00020000);
    w_voff = lane * 16;
    const int rows_left = a.M - xrow_w > 0 ? a.M - xrow_w : 0;
    xrsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.x) + (size_t)(rows_left > 0 ? xrow_w : 0) * a.ldx, (short)0,
        (int)((int64_t)rows_left * a.ldx * 2), 0x00020000);
    x_voff = ((lane & 15) * (int)a.ldx + (wave >> 1) * 32 + xk0) * 2;
  }
  auto dma_issue = [&](int kb, int buf) {
    uint8_t* st = smem + buf * kStageBytes;
    if (MODE == 1 || wmy_valid) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wrsrc, (lds_ptr_t)(st + (wave * 8 + i) * kSubBytes),
                                                 16, w_voff, kb * kBlockBytes + i * kSubBytes, 0,
                                                 0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // whole offset in the VGPR operand so the range check covers it
      const int voff = x_voff + (i * 16 * (int)a.ldx + kb * 64) * 2;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xrsrc, (lds_ptr_t)(st + kXOff + (wave * 8 + i) * kSubBytes), 16, voff, 0, 0, 0);
    }
  };

  // ---- register-staged path ----------------------------------------------
  uint4 wreg[8], xreg[8];
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (wmy_valid) {
        wreg[i] = *reinterpret_cast<const uint4*>(wmy + (size_t)kb * kBlockBytes + i * kSubBytes);
      } else {
        wreg[i] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int xs = wave * 8 + i;  // 0..31
      int kh = xs >> 4, m16 = xs & 15;
      int row = xrow0 + m16 * 16;
      int kk = kb * 64 + kh * 32 + xk0;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (row < a.M) {
        const uint16_t* src = a.x + (size_t)row * a.ldx + kk;
        if (LOAD == kLoadVec) {
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
    for (int i = 0; i < 8; ++i)
      *reinterpret_cast<uint4*>(st + (wave * 8 + i) * kSubBytes + lane * 16) = wreg[i];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      *reinterpret_cast<uint4*>(st + kXOff + (wave * 8 + i) * kSubBytes + lane * 16) = xreg[i];
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

  if (LOAD == kLoadDma) {
    if (MODE == 0 && !wmy_valid) {  // missing second block of an odd-NB GEMM: zeros
      uint8_t* st = smem;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        *reinterpret_cast<uint4*>(st + (wave * 8 + i) * kSubBytes + lane * 16) = make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(st + kStageBytes + (wave * 8 + i) * kSubBytes + lane * 16) =
            make_uint4(0, 0, 0, 0);
      }
    }
    dma_issue(0, 0);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's LDS DMA landed
    __syncthreads();
  } else {
    gload(0);
    lstore(0);
    __syncthreads();
  }

  for (int kb = 0; kb < a.KB; ++kb) {
    const int cur = kb & 1;
    const bool more = kb + 1 < a.KB;
    if (more) {
      if (LOAD == kLoadDma) dma_issue(kb + 1, cur ^ 1);
      else gload(kb + 1);
    }
    const uint8_t* st = smem + cur * kStageBytes + lane * 16;
    auto rd_b = [&](int kh, int j) {
      return *reinterpret_cast<const bf16x8*>(st + kXOff + (kh * 16 + wm * 8 + j) * kSubBytes);
    };
    auto rd_a = [&](int kh, int i) {
      return *reinterpret_cast<const bf16x8*>(st + a_off(i, kh));
    };
    // Operand schedule: the 8 B operands of a k half stay in registers, the
    // A operands stream through a 3-deep ring (read two steps ahead), and
    // the next k half's B operands are read during the current half's
    // MFMAs.  Each of the 16 (kh, i) steps: <= 2 LDS reads, then 8 MFMAs.
    bf16x8 bcur[8], bnxt[8], ar[3];
#pragma unroll
    for (int j = 0; j < 8; ++j) bcur[j] = rd_b(0, j);
    ar[0] = rd_a(0, 0);
    ar[1] = rd_a(0, 1);
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int step = kh * 8 + i;
        if (step + 2 < 16) ar[(step + 2) % 3] = rd_a((step + 2) / 8, (step + 2) % 8);
        if (kh == 0) bnxt[i] = rd_b(1, i);
        if (kh == 0) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS reads
        else __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = mfma16(ar[step % 3], bcur[j], acc[i][j]);
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);  // MFMAs
      }
      if (kh == 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) bcur[j] = bnxt[j];
      }
    }
    if (LOAD == kLoadDma) {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    } else if (more) {
      lstore(cur ^ 1);
    }
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
template <int MODE, bool OUT_BF16, int LOAD, bool YVEC>
static hipError_t launch_t(const TileArgs& a, hipStream_t s) {
  auto fn = mfma_tile_kernel<MODE, OUT_BF16, LOAD, YVEC>;
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

template <int MODE, bool OUT_BF16>
static hipError_t launch_load(const TileArgs& a, int load, bool yvec, hipStream_t s) {
  switch (load) {
    case kLoadDma:
      return yvec ? launch_t<MODE, OUT_BF16, kLoadDma, true>(a, s)
                  : launch_t<MODE, OUT_BF16, kLoadDma, false>(a, s);
    case kLoadVec:
      return yvec ? launch_t<MODE, OUT_BF16, kLoadVec, true>(a, s)
                  : launch_t<MODE, OUT_BF16, kLoadVec, false>(a, s);
    default:
      return yvec ? launch_t<MODE, OUT_BF16, kLoadElem, true>(a, s)
                  : launch_t<MODE, OUT_BF16, kLoadElem, false>(a, s);
  }
}

template <int MODE>
static hipError_t launch_mode(const TileArgs& a, bool out_bf16, int load, bool yvec,
                              hipStream_t s) {
  return out_bf16 ? launch_load<MODE, true>(a, load, yvec, s)
                  : launch_load<MODE, false>(a, load, yvec, s);
}

}  // namespace llk_gfx950

// Internal (not part of the C ABI): called by the host dispatch layer.
// load_override: -1 = choose (direct-to-LDS when eligible), else a kLoad*.
hipError_t llk_launch_tile(int mode, const uint16_t* x, int64_t ldx, const void* w0,
                           const void* w1, void* y, int64_t ldy, int M, int N, int K,
                           int KB, int NB, bool out_bf16, bool xvec, bool yvec,
                           int load_override, hipStream_t s) {
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
  // Direct-to-LDS loads need whole 64-k steps of X, 16-byte aligned rows and
  // every X byte offset (incl. the padded last tile) within 2^31.
  const int64_t x_span = ((int64_t)a.tiles_m * kTileM) * ldx * 2;
  const bool dma_ok = xvec && K % 64 == 0 && x_span < ((int64_t)1 << 31);
  int load = dma_ok ? kLoadDma : (xvec ? kLoadVec : kLoadElem);
  // An override may only pick a path the operands are eligible for.
  if (load_override == kLoadDma && dma_ok) load = kLoadDma;
  if (load_override == kLoadVec && xvec) load = kLoadVec;
  if (load_override == kLoadElem) load = kLoadElem;
  if (mode == 1) return launch_mode<1>(a, out_bf16, load, yvec, s);
  return launch_mode<0>(a, out_bf16, load, yvec, s);
}
