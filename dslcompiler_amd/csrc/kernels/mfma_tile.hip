// mfma_tile.hip -- bf16 MFMA tile kernels for gfx950: the fused SwiGLU
// prefill kernel and the micro.mma GEMM.
//
// Computes  D^T = W^T X^T  on v_mfma_f32_16x16x32_bf16: the packed weight
// (n rows, k contiguous) is the MFMA A operand and the activation X (m rows,
// k contiguous) is the B operand, so each lane's accumulators are runs of
// four consecutive n of one output row m.  The 16x16x32 form issues the same
// flops per cycle as the 32x32x16 one but moves half the accumulator
// register traffic per flop; on N(0,1) data, where the board's power limit
// sets the clock, it sustains ~14% more (register-only loop: 2.07 vs 1.82
// PFLOP/s) and this kernel 5-9% more.
//
// Workgroup: 256 threads (4 waves, 2 x 2).  Workgroup tile 256 m x 256
// MFMA rows:  GEMM -> 256 n;  SwiGLU -> 128 n of Wg + the same 128 n of Wu,
// so each wave holds the gate and up accumulators of the same (m, n) pairs
// and the SiLU(g)*u epilogue runs from registers (the reference's
// FuseDoubleContraction.cpp:175-199 epilogue, fused after the contraction of
// FuseDoubleContraction.cpp:155-173).  Wave tile: 128 m x 128 MFMA rows =
// 8 x 8 MFMA tiles of 16 x 16, 256 fp32 accumulators per lane (AGPRs).
//
// K loop: 32 k per stage (one MFMA k step).  LDS holds a ring of 4 weight
// stages (16 KiB each) and a ring of 3 X blocks of 64 k (256 rows x 128
// bytes, 32 KiB each): 160 KiB.  Operands go straight from memory into LDS
// (buffer_load_dwordx4 ... lds) two or more stages ahead of the 64 MFMAs
// per wave that consume them; X loads move whole 128-byte lines.  Each
// stage's barrier sits between its two halves of 32 MFMAs; every half-stage
// issues four refill loads, one per eight MFMAs, and each next-stage
// operand is read once its register's last MFMA of this stage has issued.
// The loop body is twelve stages, the period of the two rings, so every
// ring slot, LDS address and M0 value is a compile-time constant: with one
// wave per SIMD every instruction besides the MFMAs takes an issue slot of
// the wave, and the run-time slot arithmetic of a two-stage body (ring
// indices, clamps: ~46 scalar instructions per stage) cost 4.5% of config 3
// and 3% of the 4096^3 GEMM.  Weights sit in LDS as the payload's 1 KiB sub-blocks (32 n x 16 k,
// lane order); a 16 x 32 A operand gathers two half sub-blocks, each 16-lane
// group reading 256 contiguous bytes (conflict-free).  X sits as
// XOR-swizzled 128-byte rows, conflict-free for the operand reads (16 rows x
// 16 bytes per 16 lanes) as well.
//
// The MFMAs and the LDS-DMA loads are issued from inline assembly.  The
// compiler's LDS-DMA alias tracking cannot tell ring slots indexed at run
// time apart and would wait for every load before the next LDS read
// (vmcnt(0) at most barriers); the kernel's explicit vmcnt waits encode the
// pipeline instead.  The MFMAs have the accumulator tied to its AGPRs:
// through the builtin the register allocator routes a varying set of the 64
// four-register accumulators through temporaries every stage (up to 4 AGPR
// moves and s_nops per MFMA).  What the hazard recognizer
// would otherwise see for these instructions is covered by construction:
// A/B operands come only from LDS loads (the compiler places their waits),
// accumulators are written by nothing but the MFMAs inside the K loop, and
// the epilogue reads them only after explicit padding (acc_fence).
// tests/test_isa_cpu.py checks this on the built code object.
//
// Epilogue: SiLU(g)*u (SwiGLU), rounding to the output type, and stores
// staged through the freed LDS ring so that every store instruction writes
// whole 128-byte row segments.
//
// Optional k split across workgroups (SPLIT): raw fp32 partial planes plus
// split_reduce_kernel, which sums them in split order and applies the
// epilogue.  No workgroup ever waits for another: the kernel boundary
// orders the planes before the reduce reads them.
//
// X must be padded to whole 64-k steps with 16-byte aligned rows (the host
// copies it into a padded buffer otherwise); rows >= M read as zero through
// the buffer resource's range check.
//
// Row-major form (mfma_tile_rm_kernel, the same body with RM = true): the
// weights are the caller's bf16 [K, N] matrices instead of a packed payload
// -- each stage's 32 k rows x 128 columns per half come in as 256-byte rows
// with XOR-swizzled 16-byte chunks, and each A operand is two transposed
// LDS reads (ds_read_b64_tr_b16) -- for the KernelFn entries, which read the
// caller's weights at every call.  The MFMAs see the same operands in the
// same order, so results equal the packed form's bit for bit.
#include <type_traits>

#include "common.h"
#include "launch.h"
#include "tile_ops.h"

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
  // Tile order: groups of group_m m-tiles, m fastest inside a group, then n,
  // then the next group (0: m fastest over all m-tiles).  The 32 workgroups
  // an XCD runs at once then share fewer X and weight panels when there are
  // more than 8 m-tiles (GEMM 4096^3: 4 weight + 8 X panels per XCD instead
  // of 2 + 16).
  int group_m;
  // k split across workgroups (S > 1): workgroup (tile, s) covers the 64-k
  // blocks [s * kbs, min(KB, (s + 1) * kbs)) and writes its raw fp32
  // accumulators to part[s][mat][M][n_pad]; split_reduce_kernel adds them
  // in split order and applies the epilogue.
  float* part;
  int S, kbs, n_pad;
  // GEMM only: C += A B (the existing output is read, in its own type, and
  // added in fp32 before rounding); 0: C = A B.  Taken by
  // split_reduce_kernel: an accumulating launch always goes through the
  // partial planes (S >= 1), which keeps the tile kernel's epilogue, and its
  // registers, those of C = A B.
  int accumulate;
  // The row-major form (mfma_tile_rm_kernel, fused SwiGLU): w0 / w1 are the
  // caller's bf16 [K, N] matrices with rows of ldw0 / ldw1 elements instead
  // of packed payloads.
  int64_t ldw0, ldw1;
};

constexpr int kThreads = 256;
constexpr int kTileM = 256;
constexpr int kStageK = 32;           // k per pipeline stage
constexpr int kWStageBytes = 16384;   // weights of one 32-k stage (256 MFMA rows)
constexpr int kWStages = 4;           // LDS ring of weight stages
constexpr int kXBlockBytes = 32768;   // X of one 64-k block: 256 rows x 128 bytes
constexpr int kXBlocks = 3;           // LDS ring of X blocks
constexpr int kXRingOff = kWStages * kWStageBytes;
constexpr int kLdsBytes = kXRingOff + kXBlocks * kXBlockBytes;  // 160 KiB
// Per wave: 4 buffer_load ... lds per weight stage, 8 per X block.
constexpr int kStripRow = 144;        // epilogue staging: 128-byte rows + 16-byte pad

// Orders every accumulator after the preceding inline assembly: volatile
// asm statements keep their order, and the accumulators' later readers (and
// earlier writers) depend on these.
__device__ __forceinline__ void acc_fence(f32x4 (&acc)[8][8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("" : "+a"(acc[i][j]));
}

// MODE 0: GEMM (C = X W);  MODE 1: fused SwiGLU.
// OUT: output element type (kOutBF16, kOutF16 (GEMM only), kOutF32).
// YVEC: Y rows allow a 4-element vector store (aligned base, ldy % 4 == 0).
// SPLIT: store raw fp32 partial accumulators of k split s (see TileArgs).
// RM: the weights are the caller's row-major matrices (TileArgs::ldw0/1),
// loaded and read as described at the weight stream below; everything else
// -- MFMAs, their operands' values and order, epilogue -- is the packed
// form's, so both give the same bits.
template <int MODE, int OUT, bool YVEC, bool SPLIT, bool RM>
__device__ __forceinline__ void tile_body(TileArgs a) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int wm = wave & 1;
  const int wn = wave >> 1;

  // Workgroup -> (split s, tile): tiles of one split are contiguous, so
  // after the XCD remap the tiles that share X's k slice (and, m fastest,
  // the tiles that share W columns) run on one XCD.
  const int tiles = a.tiles_m * a.tiles_n;
  const int idx = xcd_remap(blockIdx.x, tiles * (SPLIT ? a.S : 1));
  const int split = SPLIT ? idx / tiles : 0;
  const int tile = SPLIT ? idx - split * tiles : idx;
  int tm, tn;
  if (a.group_m > 0 && a.tiles_m > a.group_m) {
    const int span = a.group_m * a.tiles_n;  // tiles of one full group
    const int g = tile / span, r = tile - g * span;
    const int gm = min(a.group_m, a.tiles_m - g * a.group_m);  // last group may be short
    tm = g * a.group_m + r % gm;
    tn = r / gm;
  } else {
    tm = tile % a.tiles_m;
    tn = tile / a.tiles_m;
  }
  const int m0 = tm * kTileM;
  const int kb0 = SPLIT ? split * a.kbs : 0;
  const int nkb = SPLIT ? min(a.KB - kb0, a.kbs) : a.KB;

  // ---- operand streams ----------------------------------------------------
  // Stage t holds k range [32 t, 32 t + 32); X block u = k [64 u, 64 u + 64)
  // (stages 2u, 2u+1).
  // Weights: ring slot t % 4 holds stage t: 8 KiB of each of two packed
  // n-blocks (k quarters 2(t%2), 2(t%2)+1 of block (nb, t/2)), contiguous in
  // the payload at t * 8 KiB of the n-block's panel.  Wave w fills
  // sub-blocks (w&1)*4 .. +4 of half w>>1.
  // X: ring slot u % 3 holds block u: 256 rows of 64 k = 128 bytes, row r at
  // 128 r.  Each load instruction moves 8 whole rows -- full 128-byte lines,
  // where 64-byte rows of a single stage took half lines (measured: the
  // half-line loads cost 2.6% of config 3 on N(0,1) data, in power).  Inside
  // a row the eight 16-byte chunks c (8 k each) sit at slot c ^ ((r >> 1) & 7):
  // rows r and r + 2 share banks (128-byte rows), so the 16 rows of an MFMA
  // operand read (lane group g reading chunk 4h + g of each) land on 16
  // distinct 16-byte bank groups.  Wave w fills rows w*64 .. +64.
  const int wslot = wave >> 1;
  u32x4 wrsrc;
  int w_voff = lane * 16;
  // Row-major weights (RM): slot half h of a stage holds 32 k rows x 128
  // columns -- SwiGLU: this tile's columns of matrix h (Wg, Wu); GEMM:
  // n-block 2 tn + h of B (past N: zeros) -- 256 bytes a row, row r at
  // 256 r, its 16-byte chunk c at c ^ sw(r), sw(r) = 2 ((r & 3) | ((r >> 1)
  // & 4)).  Load i (0..7) of a half brings rows 4 i .. +4 (lane l: row
  // 4 i + l / 16, chunk position l % 16), whole 128-byte lines; wave w
  // issues loads 4 (w & 1) .. +4 of half w >> 1 (offset w_rm[i] + stage *
  // w_step).  The resource reaches from row 64 kb0 to the matrix's last
  // element: rows past K read zero.
  int w_rm[4] = {0, 0, 0, 0};
  int w_step = 0;
  if constexpr (!RM) {
    const uint8_t* wpanel;
    if (MODE == 1) {
      wpanel = (wslot ? a.w1 : a.w0) + (size_t)tn * a.KB * kBlockBytes;
    } else {
      // An odd NB leaves the last tile without a second block; its wave pair
      // streams block 0 instead and the results (n >= N) are never stored.
      const int nb = 2 * tn + wslot;
      wpanel = a.w0 + (size_t)(nb < a.NB ? nb : 0) * a.KB * kBlockBytes;
    }
    wpanel += (size_t)kb0 * kBlockBytes + (wave & 1) * 4 * kSubBytes;
    wrsrc = buffer_rsrc(wpanel, nkb * kBlockBytes);
  } else {
    const int64_t ldw = MODE == 1 && wslot ? a.ldw1 : a.ldw0;
    const uint8_t* const wmat = MODE == 1 && wslot ? a.w1 : a.w0;
    const int ncol = (MODE == 1 ? tn : 2 * tn + wslot) * 128;
    const int64_t left = ((int64_t)(a.KB * 64 - kb0 * 64 - 1) * ldw + (a.N - ncol)) * 2;
    wrsrc = buffer_rsrc(wmat + ((int64_t)kb0 * 64 * ldw + (ncol < a.N ? ncol : 0)) * 2,
                        ncol < a.N ? (int)left : 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * ((wave & 1) * 4 + i) + (lane >> 4);
      const int sw = 2 * ((r & 3) | ((r >> 1) & 4));
      w_rm[i] = (int)((r * ldw + (((lane & 15) ^ sw) * 8)) * 2);
    }
    w_step = (int)(32 * ldw * 2);
  }

  // The X resource starts at row m0, column 64 kb0, and ends at row M:
  // rows >= M read zero.
  const int rows_left = a.M - m0;
  const u32x4 xrsrc = buffer_rsrc(a.x + (size_t)m0 * a.ldx + (size_t)kb0 * 64,
                                 (int)((int64_t)rows_left * a.ldx * 2 - (int64_t)kb0 * 128));
  // Load slot p = lane of load i: row w*64 + 8 i + p/8, stored chunk p%8
  // holding logical chunk (p%8) ^ ((row >> 1) & 7) = (p%8) ^ (p/16) ^ 4(i%2).
  const int x_rowstep = 8 * (int)a.ldx * 2;
  const int x_voff[2] = {
      (((lane >> 3) + wave * 64) * (int)a.ldx + (((lane & 7) ^ (lane >> 4)) * 8)) * 2,
      (((lane >> 3) + wave * 64) * (int)a.ldx + (((lane & 7) ^ (lane >> 4) ^ 4) * 8)) * 2};

  // Load i (0..3) of this wave's share of weight stage t into ring slot wb.
  auto dma_w = [&](int t, int wb, int i) {
    const uint8_t* st = smem + wb * kWStageBytes + (wave * 4) * kSubBytes;
    if constexpr (RM)
      dma16(wrsrc, w_rm[i] + t * w_step, 0, lds_addr(st + i * kSubBytes));
    else
      dma16(wrsrc, w_voff, t * 8 * kSubBytes + i * kSubBytes, lds_addr(st + i * kSubBytes));
  };
  // Load i (0..7) of this wave's share of X block u into ring slot xb.
  auto dma_x = [&](int u, int xb, int i) {
    const uint8_t* st = smem + kXRingOff + xb * kXBlockBytes + (wave * 8) * kSubBytes;
    // whole offset in the VGPR operand so the range check covers it
    const int voff = x_voff[i & 1] + i * x_rowstep + u * (kPackK * 2);
    dma16(xrsrc, voff, 0, lds_addr(st + i * kSubBytes));
  };
  // K-loop refills go through resources whose base follows the data being
  // refilled, so that inside the loop every ring slot and load offset is a
  // compile-time constant and the buffer range check (offset < num_records)
  // turns each refill past the end into zeros with no clamp.  rw starts at
  // the weight stage a refill targets (advanced 8 KiB per stage: its
  // num_records stays a multiple of a stage, so a load is either wholly in
  // the panel or reads zeros); rx at the X block a refill targets (advanced
  // 128 bytes per block).  Per-load X offsets are fixed per load index.
  int x_off[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x_off[i] = x_voff[i & 1] + i * x_rowstep;
  // Refill load i (0..3) of weight stage s into ring slot wb, as its M0
  // write (rw_m0) and its load (rw_ld): the stage offset in the VGPR operand,
  // so the range check covers it.
  auto rw_m0 = [&](int wb, int i) {
    set_m0(lds_addr(smem + wb * kWStageBytes + (wave * 4 + i) * kSubBytes));
  };
  auto rw_ld = [&](int s, int i) {
    if constexpr (RM)
      dma16_m0(wrsrc, w_rm[i] + s * w_step, 0);
    else
      dma16_m0(wrsrc, w_voff + s * 8 * kSubBytes, i * kSubBytes);
  };
  // Refill load i (0..7) of X block u into ring slot xb.
  auto rx_m0 = [&](int xb, int i) {
    set_m0(lds_addr(smem + kXRingOff + xb * kXBlockBytes + (wave * 8 + i) * kSubBytes));
  };
  auto rx_ld = [&](int u, int i) { dma16_m0(xrsrc, x_off[i] + u * (kPackK * 2), 0); };

  // Operands of v_mfma_f32_16x16x32_bf16 (stage-local k 0..31).
  // A operand i: 16 MFMA rows; SwiGLU i < 4 -> Wg rows wn*64 + 16 i, i >= 4
  // -> the same rows of Wu; GEMM -> rows 16 i of n-block wn.  Lane l needs
  // row l%16 and k 8*(l/16) .. +8: k quarter l/32 of the stage, slot
  // (row % 32) + 32*((l/16) % 2) of that quarter's 32 n x 16 k sub-block.
  // B operand j of a stage with block half h (t % 2): X rows wm*128 + 16 j +
  // l%16, logical chunk 4h + l/16 (8 k).
  const int a_lane = (lane >> 5) * 4 * kSubBytes + ((lane & 15) + 32 * ((lane >> 4) & 1)) * 16;
  const int brow = lane & 15;
  const int b_lane[2] = {brow * 128 + (((lane >> 4) ^ (brow >> 1)) * 16),
                         brow * 128 + (((4 + (lane >> 4)) ^ (brow >> 1)) * 16)};
  auto a_off = [&](int i) -> int {
    const int slot = (MODE == 1) ? (i >> 2) : wn;
    const int nn = (MODE == 1) ? wn * 64 + 16 * (i & 3) : 16 * i;
    return slot * 8 * kSubBytes + (nn >> 5) * kSubBytes + ((nn >> 4) & 1) * 256 + a_lane;
  };
  // RM: A operand i is two transposed reads (ds_read_b64_tr_b16, k + 0..3
  // and + 4..7 of lane l's 8 k = 8 (l / 16) ..).  Such a read gives lane i'
  // of each 16-lane group, as element j, element i' % 4 of the 8 bytes named
  // by the group's lane i' / 4 + 4 j; so the group's lane 4 j + c names row
  // 8 (l / 16) + j (+ 4), columns nn + 4 c .. + 3 of the half, and lane i'
  // receives column nn + i' at four consecutive k.  With nn = 16 q, the
  // chunk (2 q + c / 2) ^ sw(row) = 2 (q ^ s) + c / 2, s = j | 4 ((l / 16) &
  // 1): one address per q of the wave (SwiGLU: q = 4 wn + i % 4 in half
  // i / 4; GEMM: q = i in half wn), the rest immediate.
  constexpr int kQ = MODE == 1 ? 4 : 8;
  int a_rm[kQ] = {};
  if constexpr (RM) {
    const int g = lane >> 4, j = (lane >> 2) & 3, c = lane & 3;
    const int s = j | (4 * (g & 1));
#pragma unroll
    for (int q = 0; q < kQ; ++q)
      a_rm[q] = (MODE == 1 ? 0 : wn * 8192) + (8 * g + j) * 256 +
                ((MODE == 1 ? 4 * wn + q : q) ^ s) * 32 + (c >> 1) * 16 + (c & 1) * 8;
  }
  auto rd_a = [&](int wb, int i) {
    if constexpr (RM) {
      typedef short v4i16 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) v4i16* lds_v4i16;
      const uint8_t* const p = smem + wb * kWStageBytes +
                               (MODE == 1 ? (i >> 2) * 8192 + a_rm[i & 3] : a_rm[i]);
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16)(p));
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16)(p + 1024));
      return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    } else {
      return *reinterpret_cast<const bf16x8*>(smem + wb * kWStageBytes + a_off(i));
    }
  };
  auto rd_b = [&](int xb, int h, int j) {
    return *reinterpret_cast<const bf16x8*>(smem + kXRingOff + xb * kXBlockBytes +
                                            (wm * 128 + j * 16) * 128 + b_lane[h]);
  };

  // Pipeline: every half-stage issues exactly four loads per wave -- two of
  // a weight refill and two of an X refill -- one per eight MFMAs, so the
  // load path sees an even stream (a half-stage with twelve loads per wave
  // outran it).  Weight slot t % 4 is free after stage t's barrier and takes
  // stage t + 4: loads 0-1 in half 1 of stage t, loads 2-3 in half 0 of
  // stage t + 1.  X slot u % 3 is free after the barrier of stage 2u + 1
  // (block u's last operand reads were for stage 2u + 1, in stage 2u) and
  // takes block u + 3: loads 0-1 in half 1 of stage 2u + 1, 2-3 in half 0
  // and 4-5 in half 1 of stage 2u + 2, 6-7 in half 0 of stage 2u + 3.  The
  // data stage t + 1 needs (its weights; at odd t its X block) was complete
  // by half 0 of stage t - 2, so at every barrier "stage t+1 has landed" is
  // one wait count: 16 loads outstanding (four half-stages of four).  The
  // prologue issues the first stages in the order the steady state would
  // have.  Refills past the end are issued all the same (the counts stay
  // uniform): in the K loop they read zeros through the range check, in the
  // prologue they re-read the last stage / block; either way into slots no
  // MFMA reads again, and all land before the epilogue reuses the ring.
  const int T = nkb * 2;  // stages
  {
    const int w1 = min(1, T - 1), w2 = min(2, T - 1), w3 = min(3, T - 1);
    const int x1 = min(1, nkb - 1), x2 = min(2, nkb - 1);
    dma_x(0, 0, 0), dma_x(0, 0, 1);                                      // half 1 of stage -5
    dma_x(0, 0, 2), dma_x(0, 0, 3);                                      // half 0 of -4
    dma_w(0, 0, 0), dma_w(0, 0, 1), dma_x(0, 0, 4), dma_x(0, 0, 5);      // half 1 of -4
    dma_w(0, 0, 2), dma_w(0, 0, 3), dma_x(0, 0, 6), dma_x(0, 0, 7);      // half 0 of -3
    dma_w(w1, 1, 0), dma_w(w1, 1, 1), dma_x(x1, 1, 0), dma_x(x1, 1, 1);  // half 1 of -3
    dma_w(w1, 1, 2), dma_w(w1, 1, 3), dma_x(x1, 1, 2), dma_x(x1, 1, 3);  // half 0 of -2
    dma_w(w2, 2, 0), dma_w(w2, 2, 1), dma_x(x1, 1, 4), dma_x(x1, 1, 5);  // half 1 of -2
    dma_w(w2, 2, 2), dma_w(w2, 2, 3), dma_x(x1, 1, 6), dma_x(x1, 1, 7);  // half 0 of -1
    dma_w(w3, 3, 0), dma_w(w3, 3, 1), dma_x(x2, 2, 0), dma_x(x2, 2, 1);  // half 1 of -1
  }

  // Accumulators: acc[i][j] = MFMA rows (n) 16 i .. +16 of the wave's 128
  // (SwiGLU: i < 4 gate, i >= 4 up of the same n), m 16 j .. +16 of its 128.
  // Zeroed while the first stages are in flight.
  f32x4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  acc_fence(acc);  // the zeroed AGPRs are written ...
  mfma_drain();    // ... well before the first MFMA reads them
  wait_vmcnt<20>();  // X0 and W0 landed (five half-stages of loads since)
  __syncthreads();

  bf16x8 A[8], B[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) B[j] = rd_b(0, 0, j);
#pragma unroll
  for (int i = 0; i < 4; ++i) A[i] = rd_a(0, i);

  // Stage t (= g + KS, KS = t % 12 a compile-time constant, H = t % 2, X
  // block u = t / 2).  Half 0: A0..3 x B0..7, A outer; A4..7 of stage t are
  // read meanwhile, and one refill per A: its M0 write after the A's first
  // MFMA, its load after the second.  Half 1: A4..7 x B0..7, B outer; a
  // refill in every other column (M0 after the column's first MFMA, the
  // load after its second), and after column j's four MFMAs B[j] (and A[j],
  // j < 4) of stage t+1 are read -- their registers' last use this stage.
  // Splitting each refill around an MFMA keeps at most three other
  // instructions between two MFMAs almost everywhere (1186 -> 1156 cycles
  // per stage on config 3).  The weight ring (4 slots) and the X ring (3
  // slots of two stages) repeat every 12 stages, so with KS constant every
  // slot index is too.
  int g = 0;  // first stage of the current group of 12
  auto stage = [&](auto KSc) {
    constexpr int KS = decltype(KSc)::value;
    constexpr int kH = KS % 2;
    constexpr int wb = KS % kWStages;         // slot of stage t
    constexpr int xb = (KS / 2) % kXBlocks;   // slot of block u
    constexpr int wb0 = (KS + 3) % kWStages;  // half 0: loads 2-3 of stage t + 3
    constexpr int xb0 = (KS / 2 + 2) % kXBlocks;  // block u + 2
    constexpr int nwb = (KS + 1) % kWStages;
    constexpr int nxb = kH == 0 ? xb : (KS / 2 + 1) % kXBlocks;
    constexpr int nh = 1 - kH;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      A[4 + i] = rd_a(wb, 4 + i);
      constexpr int xi0 = kH == 0 ? 2 : 6;
      mfma16(A[i], B[0], acc[i][0]);
      if (i < 2) rw_m0(wb0, 2 + i);
      else rx_m0(xb0, xi0 + (i - 2));
      mfma16(A[i], B[1], acc[i][1]);
      if (i < 2) rw_ld(g + KS + 3, 2 + i);
      else rx_ld(g / 2 + KS / 2 + 2, xi0 + (i - 2));
#pragma unroll
      for (int j = 2; j < 8; ++j) mfma16(A[i], B[j], acc[i][j]);
    }
    wait_lgkmcnt0();   // this wave's reads of stage t are done
    wait_vmcnt<16>();  // stage t+1 landed
    __syncthreads();   // ... for every wave; weight slot t (and X slot u at odd t) free
    // half 1: loads 0-1 of stage t + 4 into slot t % 4; X loads 4-5 of block
    // u + 2 (H = 0) or loads 0-1 of block u + 3 into slot u % 3 (H = 1)
    constexpr int xb1 = kH == 0 ? xb0 : xb;
    constexpr int du1 = kH == 0 ? 2 : 3;  // block u + 2 or u + 3
    constexpr int xi1 = kH == 0 ? 4 : 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      mfma16(A[4], B[j], acc[4][j]);
      if (j == 0 || j == 2) rw_m0(wb, j / 2);
      else if (j == 4 || j == 6) rx_m0(xb1, xi1 + (j - 4) / 2);
      mfma16(A[5], B[j], acc[5][j]);
      if (j == 0 || j == 2) rw_ld(g + KS + 4, j / 2);
      else if (j == 4 || j == 6) rx_ld(g / 2 + KS / 2 + du1, xi1 + (j - 4) / 2);
      mfma16(A[6], B[j], acc[6][j]);
      mfma16(A[7], B[j], acc[7][j]);
      B[j] = rd_b(nxb, nh, j);
      if (j < 4) A[j] = rd_a(nwb, j);
    }
  };
  using std::integral_constant;
  for (; g < T; g += 12) {
    // T is even: stages come in pairs
    stage(integral_constant<int, 0>{});
    stage(integral_constant<int, 1>{});
    if (g + 2 >= T) break;
    stage(integral_constant<int, 2>{});
    stage(integral_constant<int, 3>{});
    if (g + 4 >= T) break;
    stage(integral_constant<int, 4>{});
    stage(integral_constant<int, 5>{});
    if (g + 6 >= T) break;
    stage(integral_constant<int, 6>{});
    stage(integral_constant<int, 7>{});
    if (g + 8 >= T) break;
    stage(integral_constant<int, 8>{});
    stage(integral_constant<int, 9>{});
    if (g + 10 >= T) break;
    stage(integral_constant<int, 10>{});
    stage(integral_constant<int, 11>{});
  }
  wait_vmcnt<0>();  // the trailing refills have landed (the epilogue reuses the ring)
  mfma_drain();
  acc_fence(acc);   // the epilogue reads the accumulators only after the drain

  // ---- epilogue: acc[i][j] holds, in lane l, output row m = m0 + wm*128 +
  // 16 j + l%16 and the four consecutive n = (wave's first n) + 16 i' +
  // 4*(l/16) + 0..3, i' = i (GEMM) or i % 4 (SwiGLU: i >= 4 is the up half).
  const int h4 = 4 * (lane >> 4);
  const int mr = lane & 15;
  const int n_end = (MODE == 1) ? tn * 128 + 128 : tn * 256 + 256;
  // Outputs go through LDS: each wave writes a 128-byte-wide column strip
  // of its 128 rows into LDS (144-byte rows, 16-byte pad), then copies whole
  // 128-byte row segments out, 8 rows per instruction, where the accumulator
  // layout would store 8- or 16-byte pieces of 16 rows per instruction
  // (measured: GEMM 4096^3 epilogue 12 -> 3.4 us).  A tile wholly inside Y
  // (or the partial planes) with 16-byte aligned rows copies 16-byte chunks
  // unchecked; an edge tile checks each chunk and copies the chunks that
  // straddle a bound (or unaligned rows) element by element.  The stage ring
  // is free once every wave is past its last operand read.
  __syncthreads();
  uint8_t* const strip = smem + wave * (128 * kStripRow);
  // Copies the wave's strip to gdst (row 0, column 0 of the strip in the
  // destination; E-byte elements; rows_ok / cols_ok in bounds).
  // NT: non-temporal 16-byte stores for the final output, which nothing in
  // the launch reads again, so that it leaves L2 to the operand panels
  // (A/B on one box: GEMM 4096^3 fp32 out 97.7 -> 96.2 us, config 3 and
  // the MLP within noise); the k-split planes, which the reduce reads back,
  // keep normal stores.
  auto strip_out = [&](auto E, auto NT, bool fast, bool al16, uint8_t* gdst, int64_t ld_bytes,
                       int rows_ok, int cols_ok) {
    constexpr int kE = decltype(E)::value;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's strip writes are done
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int row = k * 8 + (lane >> 3);
      const uint4 d = *reinterpret_cast<const uint4*>(strip + row * kStripRow + (lane & 7) * 16);
      uint8_t* const out = gdst + row * ld_bytes + (lane & 7) * 16;
      const int c0 = (lane & 7) * (16 / kE);
      if (fast || (al16 && row < rows_ok && c0 + 16 / kE <= cols_ok)) {
        if constexpr (decltype(NT)::value)
          __builtin_nontemporal_store(u32x4{d.x, d.y, d.z, d.w}, reinterpret_cast<u32x4*>(out));
        else
          *reinterpret_cast<uint4*>(out) = d;
      } else if (row < rows_ok) {
        const uint32_t w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int e = 0; e < 16 / kE; ++e) {
          if (c0 + e >= cols_ok) break;
          if constexpr (kE == 4) reinterpret_cast<uint32_t*>(out)[e] = w[e];
          else reinterpret_cast<uint16_t*>(out)[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // ... and its reads, before the strip is rewritten
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
  };
  const int rows_ok = a.M - (m0 + wm * 128);
  if constexpr (SPLIT) {
    constexpr int NMAT = (MODE == 1) ? 2 : 1;
    const size_t plane = (size_t)a.M * a.n_pad;
    const bool fast = m0 + kTileM <= a.M && n_end <= a.n_pad;  // plane rows are 16-byte aligned
#pragma unroll
    for (int sp = 0; sp < 4; ++sp) {
      // Strip sp: 32 fp32 columns = accumulator rows i = 2 sp, 2 sp + 1.
      // SwiGLU: sp < 2 gate, sp >= 2 up (same n); GEMM: four n sub-tiles.
      const int mat = (MODE == 1) ? (sp >> 1) : 0;
      const int col0 = (MODE == 1) ? tn * 128 + wn * 64 + (sp & 1) * 32 : tn * 256 + wn * 128 + sp * 32;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          *reinterpret_cast<f32x4*>(strip + (j * 16 + mr) * kStripRow + (ii * 16 + h4) * 4) =
              acc[2 * sp + ii][j];
      strip_out(std::integral_constant<int, 4>{}, std::false_type{}, fast, true,
                reinterpret_cast<uint8_t*>(a.part + ((size_t)split * NMAT + mat) * plane +
                                           (size_t)(m0 + wm * 128) * a.n_pad + col0),
                (int64_t)a.n_pad * 4, rows_ok, a.n_pad - col0);
    }
    return;
  }
  constexpr int NI = (MODE == 1) ? 4 : 8;         // 16-column groups of the wave's output
  constexpr int kElem = (OUT == kOutF32) ? 4 : 2;
  constexpr int kPerStrip = 128 / (16 * kElem);  // 16-column groups per 128-byte strip: 4 or 2
  const bool al16 = ((reinterpret_cast<uintptr_t>(a.y) | (uintptr_t)(a.ldy * kElem)) & 15) == 0;
  const bool fast = YVEC && m0 + kTileM <= a.M && n_end <= a.N && al16;
  const int n_w = (MODE == 1) ? tn * 128 + wn * 64 : tn * 256 + wn * 128;
  uint8_t* const ybase =
      static_cast<uint8_t*>(a.y) + ((size_t)max(0, m0 + wm * 128) * a.ldy + n_w) * kElem;
#pragma unroll
  for (int sidx = 0; sidx < NI / kPerStrip; ++sidx) {
#pragma unroll
    for (int ii = 0; ii < kPerStrip; ++ii) {
      const int i = sidx * kPerStrip + ii;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float v[4];
        const f32x4 g = acc[i][j];
        const f32x4 u = acc[(MODE == 1) ? i + 4 : i][j];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if constexpr (MODE == 1)
            v[q] = swiglu_act(g[q], u[q]);
          else
            v[q] = g[q];
        }
        uint8_t* const dst = strip + (j * 16 + mr) * kStripRow + (ii * 16 + h4) * kElem;
        if constexpr (OUT == kOutF32) {
          *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
        } else if constexpr (OUT == kOutBF16) {
          *reinterpret_cast<uint2*>(dst) =
              make_uint2(f32x2_to_bf16x2_rne(v[0], v[1]), f32x2_to_bf16x2_rne(v[2], v[3]));
        } else {
          *reinterpret_cast<uint2*>(dst) =
              make_uint2((uint32_t)f32_to_f16_rne(v[0]) | ((uint32_t)f32_to_f16_rne(v[1]) << 16),
                         (uint32_t)f32_to_f16_rne(v[2]) | ((uint32_t)f32_to_f16_rne(v[3]) << 16));
        }
      }
    }
    strip_out(std::integral_constant<int, kElem>{}, std::true_type{}, fast, al16, ybase + sidx * 128,
              a.ldy * kElem, rows_ok, a.N - (n_w + sidx * 128 / kElem));
  }
}

template <int MODE, int OUT, bool YVEC, bool SPLIT>
__global__ __launch_bounds__(kThreads, 1) void mfma_tile_kernel(TileArgs a) {
  tile_body<MODE, OUT, YVEC, SPLIT, false>(a);
}

// The fused SwiGLU or the GEMM on the caller's row-major weights
// (TileArgs::ldw0/1).
template <int MODE, int OUT, bool YVEC, bool SPLIT>
__global__ __launch_bounds__(kThreads, 1) void mfma_tile_rm_kernel(TileArgs a) {
  tile_body<MODE, OUT, YVEC, SPLIT, true>(a);
}

// Sums the S partial planes of each output element in split order (fixed,
// so results are reproducible) and applies the epilogue.  One thread per
// 4 consecutive n of a row.
template <int MODE, int OUT, bool YVEC>
__global__ __launch_bounds__(256) void split_reduce_kernel(TileArgs a) {
  constexpr int NMAT = (MODE == 1) ? 2 : 1;
  const int quads = (a.N + 3) / 4;
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)a.M * quads) return;
  const int m = (int)(e / quads);
  const int n = (int)(e - (int64_t)m * quads) * 4;
  const size_t plane = (size_t)a.M * a.n_pad;
  const float* src = a.part + (size_t)m * a.n_pad + n;
  f32x4 sum[NMAT];
#pragma unroll
  for (int p = 0; p < NMAT; ++p) sum[p] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < a.S; ++sp)
#pragma unroll
    for (int p = 0; p < NMAT; ++p)
      sum[p] += *reinterpret_cast<const f32x4*>(src + ((size_t)sp * NMAT + p) * plane);
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if constexpr (MODE == 1)
      v[q] = swiglu_act(sum[0][q], sum[1][q]);
    else
      v[q] = sum[0][q];
  }
  if constexpr (MODE == 0) {
    if (a.accumulate) add_existing4<OUT>(a.y, a.ldy, a.M, a.N, m, n, v, YVEC);
  }
  store4<OUT>(a.y, a.ldy, a.M, a.N, m, n, v, YVEC);
}

// ---------------------------------------------------------------------------
// Host launchers (mod: a loaded per-operation code object, or null for the
// library's own kernels).  A build of one operation's code object
// (LLK_CO_OP: 1 SwiGLU, 0 GEMM) instantiates that operation's kernels only.
// ---------------------------------------------------------------------------
template <int MODE, int OUT, bool YVEC, bool SPLIT, bool RM = false>
const char* tile_symbol() {
  static const std::string name =
      std::string(RM ? "_ZN10llk_gfx95019mfma_tile_rm_kernelI" : "_ZN10llk_gfx95016mfma_tile_kernelI") +
      mangle_int(MODE) + mangle_int(OUT) + mangle_bool(YVEC) + mangle_bool(SPLIT) +
      "EEvNS_8TileArgsE";
  return name.c_str();
}

template <int MODE, int OUT, bool YVEC>
const char* split_reduce_symbol() {
  static const std::string name = "_ZN10llk_gfx95019split_reduce_kernelI" + mangle_int(MODE) +
                                  mangle_int(OUT) + mangle_bool(YVEC) + "EEvNS_8TileArgsE";
  return name.c_str();
}

template <int MODE, int OUT, bool YVEC, bool SPLIT, bool RM = false>
static hipError_t launch_tile_t(const TileArgs& a, const llk::ModuleFns* mod, hipStream_t s) {
  void (*fn)(TileArgs);
  if constexpr (RM)
    fn = mfma_tile_rm_kernel<MODE, OUT, YVEC, SPLIT>;
  else
    fn = mfma_tile_kernel<MODE, OUT, YVEC, SPLIT>;
  if (!mod) {
    static std::atomic<uint64_t> lds_set{0};  // devices configured, per instantiation
    hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(fn), kLdsBytes, lds_set);
    if (e != hipSuccess) return e;
  }
  const int tiles = a.tiles_m * a.tiles_n;
  dim3 grid(tiles * (SPLIT ? a.S : 1)), block(kThreads);
  return launch_kernel(mod, reinterpret_cast<const void*>(fn),
                       &tile_symbol<MODE, OUT, YVEC, SPLIT, RM>, grid, block, kLdsBytes, s, a);
}

// A k-split (or accumulating) launch: the tile kernel's fp32 partial planes,
// then split_reduce_kernel.
template <int MODE, int OUT, bool YVEC, bool RM = false>
static hipError_t launch_split(const TileArgs& a, const llk::ModuleFns* mod, hipStream_t s) {
  // Partials are fp32 planes with 16-byte aligned rows: one instantiation.
  hipError_t e = launch_tile_t<MODE, kOutF32, true, true, RM>(a, mod, s);
  if (e != hipSuccess) return e;
  const int64_t threads = (int64_t)a.M * ((a.N + 3) / 4);
  return launch_kernel(mod, reinterpret_cast<const void*>(split_reduce_kernel<MODE, OUT, YVEC>),
                       &split_reduce_symbol<MODE, OUT, YVEC>,
                       dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, a);
}

template <int MODE, int OUT, bool YVEC, bool RM = false>
static hipError_t launch_t(const TileArgs& a, const llk::ModuleFns* mod, hipStream_t s) {
  if (a.S <= 1 && !a.accumulate) return launch_tile_t<MODE, OUT, YVEC, false, RM>(a, mod, s);
  return launch_split<MODE, OUT, YVEC, RM>(a, mod, s);
}

template <int MODE, int OUT>
static hipError_t launch_out(const TileArgs& a, bool yvec, const llk::ModuleFns* mod,
                             hipStream_t s) {
  return yvec ? launch_t<MODE, OUT, true>(a, mod, s) : launch_t<MODE, OUT, false>(a, mod, s);
}

// fp16 output exists for the GEMM only (llk.matmul's result types).
template <int MODE>
static hipError_t launch_mode(const TileArgs& a, int out, bool yvec, const llk::ModuleFns* mod,
                              hipStream_t s) {
  if (out == kOutBF16) return launch_out<MODE, kOutBF16>(a, yvec, mod, s);
  if (out == kOutF32) return launch_out<MODE, kOutF32>(a, yvec, mod, s);
  if constexpr (MODE == 0) {
    if (out == kOutF16) return launch_out<MODE, kOutF16>(a, yvec, mod, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace llk_gfx950

// Largest X span (bytes, rows padded to whole tiles) the 32-bit buffer
// offsets of the tile kernel can address.
bool llk_tile_x_fits(int M, int64_t ldx) {
  const int64_t rows = ((int64_t)M + 255) / 256 * 256;
  return rows * ldx * 2 < ((int64_t)1 << 31);
}

// Bytes of the partial planes of a k split over S workgroups (0 if S <= 1
// and the launch does not accumulate: an accumulating GEMM launch always
// takes the planes, one at S = 1).
size_t llk_tile_split_bytes(int mode, int M, int NB, int S, bool accumulate) {
  if (S <= 1 && !accumulate) return 0;
  return (size_t)(S > 1 ? S : 1) * (mode == 1 ? 2 : 1) * M * NB * 128 * sizeof(float);
}

// Internal (not part of the C ABI).  x: [M, 64*KB] bf16 with ldx % 8 == 0,
// 16-byte aligned, columns >= K zero; llk_tile_x_fits(M, ldx) must hold.
// S > 1 splits K over S workgroups of kbs = ceil(KB / S) blocks (every split
// non-empty: the caller guarantees (S - 1) * kbs < KB); `part` (16-byte
// aligned) holds llk_tile_split_bytes(mode, M, NB, S, accumulate) bytes.
// accumulate (GEMM only): y += x w instead of y = x w.
hipError_t llk_launch_tile(int mode, const uint16_t* x, int64_t ldx, const void* w0,
                           const void* w1, void* y, int64_t ldy, int M, int N, int KB, int NB,
                           int S, void* part, int out, bool yvec, bool accumulate,
                           const llk::ModuleFns* mod, hipStream_t s) {
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
  a.group_m = 8;
  a.S = S > 1 ? S : 1;
  a.kbs = (KB + a.S - 1) / a.S;
  a.n_pad = NB * 128;
  a.part = static_cast<float*>(part);
  a.accumulate = accumulate ? 1 : 0;
  a.ldw0 = a.ldw1 = 0;
  if (a.S > 1 && (part == nullptr || (int64_t)(a.S - 1) * a.kbs >= KB)) return hipErrorInvalidValue;
  if (accumulate && (mode != 0 || part == nullptr)) return hipErrorInvalidValue;
#if !defined(LLK_CO_OP) || LLK_CO_OP == 1
  if (mode == 1) return launch_mode<1>(a, out, yvec, mod, s);
#endif
#if !defined(LLK_CO_OP) || LLK_CO_OP == 0
  if (mode == 0) return launch_mode<0>(a, out, yvec, mod, s);
#endif
  return hipErrorInvalidValue;
}

// Whether the row-major tile form takes a [K, N] weight matrix at w (row
// stride ldw elements) with X of row stride ldx: K a multiple of 64, N and
// ldw multiples of 8 (16-byte chunks wholly inside or outside a row),
// 16-byte aligned rows, and every offset the kernel forms (up to K + 128
// rows) within 32 bits.
bool llk_tile_rowmajor_fits(int M, int64_t K, int64_t ldx, const void* w, int64_t ldw,
                            int64_t N) {
  return M > 0 && K > 0 && K % 64 == 0 && N > 0 && N % 8 == 0 && ldw % 8 == 0 && ldw >= N &&
         reinterpret_cast<uintptr_t>(w) % 16 == 0 && ldx % 8 == 0 && ldx >= K &&
         (K + 128) * ldw * 2 < ((int64_t)1 << 31) && llk_tile_x_fits(M, ldx);
}

// Internal.  On row-major bf16 weights ([K, N], row strides ldw0 / ldw1;
// llk_tile_rowmajor_fits for each) and x as for llk_launch_tile with
// K = 64 KB: mode 1, the fused SwiGLU with a bf16 or fp32 result (w0 = Wg,
// w1 = Wu); mode 0, the accumulating GEMM y += x w0 (bf16, fp16 or fp32 y; part
// holds the planes at S >= 1).  The same grid, k splits and partial planes
// as llk_launch_tile(mode, ...) with NB = ceil(N / 128), and the same bits.
hipError_t llk_launch_tile_rowmajor(int mode, const uint16_t* x, int64_t ldx, const uint16_t* w0,
                                    int64_t ldw0, const uint16_t* w1, int64_t ldw1, void* y,
                                    int64_t ldy, int M, int N, int K, int S, void* part, int out,
                                    bool yvec, bool accumulate, const llk::ModuleFns* mod,
                                    hipStream_t s) {
  using namespace llk_gfx950;
  if (mode == 1 ? ((out != kOutBF16 && out != kOutF32) || accumulate ||
                   !llk_tile_rowmajor_fits(M, K, ldx, w1, ldw1, N))
                : (mode != 0 || !accumulate || part == nullptr))
    return hipErrorInvalidValue;
  if (!llk_tile_rowmajor_fits(M, K, ldx, w0, ldw0, N)) return hipErrorInvalidValue;
  TileArgs a;
  a.x = x;
  a.w0 = reinterpret_cast<const uint8_t*>(w0);
  a.w1 = reinterpret_cast<const uint8_t*>(w1);
  a.y = y;
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.KB = K / 64;
  a.NB = (N + 127) / 128;
  a.tiles_m = (M + kTileM - 1) / kTileM;
  a.tiles_n = mode == 1 ? a.NB : (a.NB + 1) / 2;
  a.group_m = 8;
  a.S = S > 1 ? S : 1;
  a.kbs = (a.KB + a.S - 1) / a.S;
  a.n_pad = a.NB * 128;
  a.part = static_cast<float*>(part);
  a.accumulate = accumulate ? 1 : 0;
  a.ldw0 = ldw0;
  a.ldw1 = ldw1;
  if (a.S > 1 && (part == nullptr || (int64_t)(a.S - 1) * a.kbs >= a.KB))
    return hipErrorInvalidValue;
#if !defined(LLK_CO_OP) || LLK_CO_OP == 1
  if (mode == 1 && out == kOutBF16)
    return yvec ? launch_t<1, kOutBF16, true, true>(a, mod, s)
                : launch_t<1, kOutBF16, false, true>(a, mod, s);
  if (mode == 1)
    return yvec ? launch_t<1, kOutF32, true, true>(a, mod, s)
                : launch_t<1, kOutF32, false, true>(a, mod, s);
#endif
#if !defined(LLK_CO_OP) || LLK_CO_OP == 0
  if (mode == 0) {  // accumulating: the planes and the reduce, which reads y
    if (out == kOutBF16)
      return yvec ? launch_split<0, kOutBF16, true, true>(a, mod, s)
                  : launch_split<0, kOutBF16, false, true>(a, mod, s);
    if (out == kOutF16)
      return yvec ? launch_split<0, kOutF16, true, true>(a, mod, s)
                  : launch_split<0, kOutF16, false, true>(a, mod, s);
    if (out == kOutF32)
      return yvec ? launch_split<0, kOutF32, true, true>(a, mod, s)
                  : launch_split<0, kOutF32, false, true>(a, mod, s);
  }
#endif
  return hipErrorInvalidValue;
}
