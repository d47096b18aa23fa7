// swiglu_wide.hip -- fused SwiGLU tile kernel with tiles of 16*B columns
// per matrix (B odd: 7 or 11), for shapes where the 128-column tile of
// mfma_tile.hip leaves the last round of workgroups partly filled.
//
// Config 3 (M = 2048, N = 11008): 128-column tiles make 8 x 86 = 688 tiles,
// 2.69 rounds of 256 CUs; 176-column tiles (B = 11) make 8 x 63 = 504, two
// rounds of 1.375x the work with 248 of 256 CUs busy in the second, and move
// 14% fewer L2 -> LDS bytes per flop (the K loop's operand stream is what the
// board's power limit charges for).  Config 5's SwiGLU at M = 1000
// (N = 13824): 4 x 108 = 432 tiles (1.69 rounds) against 4 x 124 = 496 with
// 112-column tiles (B = 7), two rounds of 0.875x the work.
//
// Same arithmetic as the fused path of mfma_tile.hip (MODE 1): D^T = W^T X^T
// on v_mfma_f32_16x16x32_bf16 with fp32 accumulators, gate = X Wg and
// up = X Wu over the whole K, then SiLU(gate) * up rounded once to bf16
// (FuseDoubleContraction.cpp:155-199).
//
// Workgroup: 256 threads, 4 waves in 2 (m) x 2 (column halves); tile 256 m
// x 16 B n.  A wave holds 128 m x B MFMA row blocks of 16 (B x 8 MFMA tiles,
// 32 B fp32 accumulators per lane: 256 AGPRs and, for B = 11, 96 VGPRs).
// With B odd the B blocks of a matrix do not split evenly between the wave
// pair, so wave wn = 0 takes gate blocks 0..C and up blocks 0..C-1, wave
// wn = 1 up blocks C..B-1 and gate blocks C+1..B-1 (C = (B-1)/2): each wave
// holds both matrices of every block but C, whose gate sits in wave 0 and up
// in wave 1; the epilogue exchanges half of block C through LDS (4 KiB each
// way per wave pair), so that each wave finishes exactly half of the tile's
// outputs.
//
// Weights: the packed payload (common.h) is in 128-column blocks; a tile
// starting at a multiple of 16 B columns starts at a multiple of 16 inside
// some block.  Each 16 x 32 MFMA A operand (16 n x 32 k of one matrix) is
// one 1 KiB LDS-DMA load gathering four 256-byte runs of the payload (16-lane
// groups: k quarters q, q+1 x their two 8-k halves), placed in LDS in lane
// order (conflict-free operand reads).  A weight stage (32 k) is 2 B such
// loads; waves issue LW loads each (4 LW >= 2 B; the spare loads read past
// the buffer's range, i.e. zeros without memory traffic, into unused LDS).
//
// LDS: ring of 2 X blocks of 64 k (256 rows x 128 bytes, XOR-swizzled as in
// mfma_tile.hip) at 0, ring of 4 weight stages (4 LW KiB each) after it:
// 160 KiB for B = 11, 128 KiB for B = 7.  The K loop body is four 32-k
// stages (the period of both rings), so every slot is a compile-time
// constant.  Refill schedule per wave, by half-stage (h = 2t + half of
// stage t), each half-stage issuing the same number of loads (5 for B = 11,
// 4 for B = 7), ordered by deadline within a half-stage:
//   X block v: loads 0-3 at h = 4v - 5, 4-7 at 4v - 4 (its slot is free
//     after the barrier of stage 2v - 3; needed at the barrier of 2v - 1);
//   weight stage s (slot free after the barrier of stage s - 4, needed at
//     the barrier of s - 1): s even: first half of its loads at 2s - 7, the
//     rest at 2s - 6; s odd (LW = 6): load 0 at 2s - 7, 1 at 2s - 6, 2-3 at
//     2s - 5, 4-5 at 2s - 4; (LW = 4): 0-1 at 2s - 5, 2-3 at 2s - 4.
// so the wait before each barrier is one constant count per stage parity.
// Refills past the end of K read the next n-block's panel or zeros into
// slots no MFMA reads again; all land before the epilogue reuses the LDS.
//
// Epilogue: SiLU(g) * u on registers, bf16 rounding, the tile's output
// staged whole in LDS (256 rows x 32 B bytes) and copied out in 16-byte
// chunks with non-temporal stores.
//
// WNT (one m tile, M <= 256: every weight byte is read by one workgroup):
// the weight loads are non-temporal, so the stream passes L2 without
// evicting X (config 5's SwiGLU at M = 255: K loop 58.9 -> 52.2 us, launch
// 84.6 -> 80.5 us in per-workgroup timestamps; 86.2 -> 79.1-80.4 us through
// the library, the MLP 150.4 -> 138.5-140.1 us; with several m tiles, which
// re-read the weight panels from L2, `nt` is slower: M = 1000 +3%, config 3
// +4%; A/B on one box).
//
// Optional k split (SPLIT, config 5's SwiGLU at M = 255: 124 tiles of B = 7
// x 2 splits = 248 workgroups where the 128-column kernel runs 108 x 2 =
// 216): workgroup (tile, s) covers the 64-k blocks [s kbs, (s + 1) kbs) and
// stores its raw fp32 accumulators in register order -- each wave's R x 8
// quads as R x 8 coalesced 1 KiB stores, no LDS staging -- and
// wide_reduce_kernel sums the S partials of every output in split order
// (fixed, so results are reproducible; with the same k ranges they equal
// the 128-column kernel's split sums bit for bit) and applies the epilogue.
#include <type_traits>

#include "common.h"
#include "launch.h"
#include "tile_ops.h"

namespace llk_gfx950 {

struct WideArgs {
  const uint16_t* x;   // [M, K_pad] bf16, row stride ldx (multiple of 8), 16-byte aligned
  const uint8_t* w0;   // packed Wg payload
  const uint8_t* w1;   // packed Wu payload
  uint16_t* y;         // [M, N] bf16, row stride ldy
  int64_t ldx, ldy;
  int M, N;
  int KB;              // K_pad / 64
  int NB;              // packed n-blocks of 128
  int tiles_m, tiles_n;
  int group_m;         // tile order as TileArgs::group_m
  // k split (S > 1): partials [S][tiles][4 waves][R][8][64 lanes] x f32x4,
  // kbs 64-k blocks per split (every split non-empty).
  float* part;
  int S, kbs;
};

template <int B>
struct WideCfg {
  static_assert(B == 7 || B == 11, "wide SwiGLU tiles have 7 or 11 blocks of 16 columns");
  static constexpr int kThreads = 256;
  static constexpr int R = B;                    // MFMA row blocks per wave
  static constexpr int C = (B - 1) / 2;          // the block split between the wave pair
  static constexpr int H0 = (B + 1) / 2;         // row blocks of half 0
  static constexpr int LW = B == 11 ? 6 : 4;     // weight loads per wave per stage
  static constexpr int LH = LW / 2;              // ... per matrix
  static constexpr int kFrag = 2 * LW;           // fragment places per matrix in a stage slot
  static constexpr int kWSlot = 2 * kFrag * 1024;
  static constexpr int kXBlock = 32768;          // 256 rows x 128 bytes
  static constexpr int kWRing = 2 * kXBlock;     // X ring (2 blocks) at 0, weights after it
  static constexpr int kLds = kWRing + 4 * kWSlot;
  static constexpr int kN = 16 * B;              // columns per tile (each matrix)
  static constexpr int kRowBytes = 2 * kN;       // one tile row of bf16 output
  static constexpr int kXch = 0;                 // epilogue: block-C exchange (32 KiB)
  static constexpr int kStage = 32768;           // epilogue: output staging
  static_assert(kStage + 256 * kRowBytes <= kLds, "staging fits the LDS");
  // Loads outstanding at the barrier of an even / odd stage, and before the
  // first stage (see the schedule above).
  static constexpr int kWaitEven = LW == 6 ? 13 : 10;
  static constexpr int kWaitOdd = LW == 6 ? 11 : 8;
  static constexpr int kWaitFirst = LW == 6 ? 16 : 12;
};

// One refill load of a half-stage: kind 0 = weight load `idx` of stage t + d,
// kind 1 = X load `idx` of block t/2 + d (t/2 rounded down).
struct WLoad {
  int kind, d, idx;
};
struct HalfLoads {
  int n;
  WLoad l[5];
};

// The schedule of the header comment, per (loads per wave LW, stage parity,
// half), in issue order.
constexpr HalfLoads half_loads(int LW, int H, int half) {
  if (LW == 6) {
    if (H == 0 && half == 0) return {5, {{1, 1, 4}, {1, 1, 5}, {1, 1, 6}, {1, 1, 7}, {0, 3, 1}}};
    if (H == 0 && half == 1) return {5, {{0, 3, 2}, {0, 3, 3}, {0, 4, 0}, {0, 4, 1}, {0, 4, 2}}};
    if (H == 1 && half == 0) return {5, {{0, 2, 4}, {0, 2, 5}, {0, 3, 3}, {0, 3, 4}, {0, 3, 5}}};
    return {5, {{1, 2, 0}, {1, 2, 1}, {1, 2, 2}, {1, 2, 3}, {0, 4, 0}}};
  }
  if (H == 0 && half == 0) return {4, {{1, 1, 4}, {1, 1, 5}, {1, 1, 6}, {1, 1, 7}, {0, 0, 0}}};
  if (H == 0 && half == 1) return {4, {{0, 3, 0}, {0, 3, 1}, {0, 4, 0}, {0, 4, 1}, {0, 0, 0}}};
  if (H == 1 && half == 0) return {4, {{0, 2, 2}, {0, 2, 3}, {0, 3, 2}, {0, 3, 3}, {0, 0, 0}}};
  return {4, {{1, 2, 0}, {1, 2, 1}, {1, 2, 2}, {1, 2, 3}, {0, 0, 0}}};
}

// Half-1 column of load k (0..n-1): spread over the 8 columns.
constexpr int half1_load_at(int n, int col) {
  for (int k = 0; k < n; ++k)
    if (k * 8 / n == col) return k;
  return -1;
}

// Calls f(integral_constant<int, I>) for I = 0 .. N-1, in order.
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
template <int V>
using ic = std::integral_constant<int, V>;

// Orders accumulator row block r (AGPRs for r < 8, VGPRs after) after the
// preceding inline assembly: volatile asm statements keep their order.
template <int r>
__device__ __forceinline__ void acc_order(f32x4& v) {
  if constexpr (r < 8) asm volatile("" : "+a"(v));
  else asm volatile("" : "+v"(v));
}

// Tile index -> (m tile, n tile): XCD-aware order of mfma_tile_kernel, m
// fastest inside groups of group_m m-tiles.
__device__ __forceinline__ void wide_tile_mn(const WideArgs& a, int tile, int& tm, int& tn) {
  if (a.group_m > 0 && a.tiles_m > a.group_m) {
    const int span = a.group_m * a.tiles_n;
    const int g = tile / span, r = tile - g * span;
    const int gm = min(a.group_m, a.tiles_m - g * a.group_m);
    tm = g * a.group_m + r % gm;
    tn = r / gm;
  } else {
    tm = tile % a.tiles_m;
    tn = tile / a.tiles_m;
  }
}

template <int B, bool SPLIT, bool WNT>
__global__ __launch_bounds__(256, 1) void mfma_swiglu_wide_kernel(WideArgs a) {
  using Cfg = WideCfg<B>;
  constexpr int R = Cfg::R, C = Cfg::C, H0 = Cfg::H0, LW = Cfg::LW, LH = Cfg::LH;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int wm = wave & 1;
  const int wn = wave >> 1;

  // Workgroup -> (split, tile): tiles of one split are contiguous, so after
  // the XCD remap the tiles sharing X's k slice run on one XCD.
  const int tiles = a.tiles_m * a.tiles_n;
  const int idx = xcd_remap(blockIdx.x, tiles * (SPLIT ? a.S : 1));
  const int split = SPLIT ? idx / tiles : 0;
  const int tile = SPLIT ? idx - split * tiles : idx;
  int tm, tn;
  wide_tile_mn(a, tile, tm, tn);
  const int m0 = tm * 256;
  const int n0 = tn * Cfg::kN;
  const int kb0 = SPLIT ? split * a.kbs : 0;
  const int nkb = SPLIT ? min(a.KB - kb0, a.kbs) : a.KB;
  const int T = 2 * nkb;  // 32-k stages

  // ---- weight stream --------------------------------------------------------
  // One resource per matrix from the first packed n-block the tile touches
  // to the payload's end (the host keeps three panels plus the stage offsets
  // below 2^31, so every real load is in range and the spare loads, at
  // 2^31 + ..., are not).
  // A split starts kb0 blocks into every panel.
  const int nbf = n0 >> 7;
  const int64_t panel = (int64_t)a.KB * kBlockBytes;
  const int64_t wspan = (int64_t)(a.NB - nbf) * panel - (int64_t)kb0 * kBlockBytes;
  const int wbytes = (int)(wspan < 0x7fffffff ? wspan : 0x7fffffff);
  const size_t wbase = (size_t)nbf * panel + (size_t)kb0 * kBlockBytes;
  const u32x4 rg = buffer_rsrc(a.w0 + wbase, wbytes);
  const u32x4 ru = buffer_rsrc(a.w1 + wbase, wbytes);
  // Lane l of a fragment load fetches row l%16 of a 16-column block, k
  // 8*(l/16) .. +8 of the stage: sub-block k quarter l/32 (+4 KiB), slot half
  // (l/16)%2 (+512 bytes) of it.  Stage t adds t * 8 KiB (two k quarters).
  const int w_lane = (lane >> 5) * 4096 + ((lane >> 4) & 1) * 512 + (lane & 15) * 16;
  // This wave's loads k and k + LH fetch block b = wave * LH + k of Wg and of
  // Wu (b >= B: a spare load, out of range).
  int w_vo[LH];
#pragma unroll
  for (int k = 0; k < LH; ++k) {
    const int b = wave * LH + k;
    const int n = n0 + 16 * b, nn = n & 127;
    w_vo[k] = b < B ? (int)((int64_t)((n >> 7) - nbf) * panel) + (nn >> 5) * 1024 +
                          ((nn >> 4) & 1) * 256 + w_lane
                    : (int)0x80000000;
  }
  // LDS place of this wave's load k: fragment (k >= LH) * 2 LW + wave * LH +
  // k % LH of the stage slot.
  const uint32_t w_lds0 = lds_addr(smem + Cfg::kWRing) + (uint32_t)(wave * LH) * 1024;

  // ---- X stream (as mfma_tile_kernel) ---------------------------------------
  // X from row m0, column 64 kb0, to row M (rows >= M read zero).
  const int rows_left = a.M - m0;
  const u32x4 xrsrc = buffer_rsrc(a.x + (size_t)m0 * a.ldx + (size_t)kb0 * 64,
                                 (int)((int64_t)rows_left * a.ldx * 2 - (int64_t)kb0 * 128));
  const int x_rowstep = 8 * (int)a.ldx * 2;
  int x_off[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    x_off[i] = (((lane >> 3) + wave * 64) * (int)a.ldx +
                (((lane & 7) ^ (lane >> 4) ^ ((i & 1) * 4)) * 8)) * 2 + i * x_rowstep;
  const uint32_t x_lds0 = lds_addr(smem) + (uint32_t)(wave * 8) * 1024;

  // LDS address and voff of a load of stage / block index s.
  auto w_m0 = [&](int slot, int k) {
    return w_lds0 + (uint32_t)(slot * Cfg::kWSlot + ((k >= LH) ? 2 * LW : 0) * 1024 + (k % LH) * 1024);
  };
  auto x_m0 = [&](int slot, int i) { return x_lds0 + (uint32_t)(slot * Cfg::kXBlock + i * 1024); };
  auto w_voff = [&](int s, int k) { return w_vo[k % LH] + s * 8192; };
  auto x_voff = [&](int blk, int i) { return x_off[i] + blk * 128; };
  // Prologue form (M0 write, wait state and load in one statement).
  auto pre_w = [&](int s, int k) {
    if constexpr (WNT) dma16_nt(k < LH ? rg : ru, w_voff(s, k), 0, w_m0(s & 3, k));
    else dma16(k < LH ? rg : ru, w_voff(s, k), 0, w_m0(s & 3, k));
  };
  auto pre_x = [&](int blk, int i) { dma16(xrsrc, x_voff(blk, i), 0, x_m0(blk & 1, i)); };

  // ---- operand reads --------------------------------------------------------
  // A operand of row block r: fragment q of the stage slot, q = r (wave 0, r
  // <= C: gate r), 2 LW + r - C - 1 (wave 0, r > C: up r - C - 1), 2 LW + C + r
  // (wave 1, r <= C: up C + r), r (wave 1, r > C: gate r).
  const int a_lo = Cfg::kWRing + lane * 16 + wn * (2 * LW + C) * 1024;
  const int a_hi = Cfg::kWRing + lane * 16 + (1 - wn) * (2 * LW - C - 1) * 1024;
  auto rd_a = [&](int slot, int r) {
    return *reinterpret_cast<const bf16x8*>(smem + slot * Cfg::kWSlot + r * 1024 +
                                            (r <= C ? a_lo : a_hi));
  };
  // B operand j of a stage with block half h: X rows wm*128 + 16 j + l%16,
  // logical chunk 4h + l/16 of the swizzled 128-byte row.
  const int brow = lane & 15;
  const int b_lane[2] = {wm * 128 * 128 + brow * 128 + (((lane >> 4) ^ (brow >> 1)) * 16),
                         wm * 128 * 128 + brow * 128 + (((4 + (lane >> 4)) ^ (brow >> 1)) * 16)};
  auto rd_b = [&](int slot, int h, int j) {
    return *reinterpret_cast<const bf16x8*>(smem + slot * Cfg::kXBlock + j * 16 * 128 + b_lane[h]);
  };

  // ---- prologue: the loads the steady state issues before stage 0 ----------
  if constexpr (LW == 6) {
    pre_w(0, 0), pre_w(0, 1), pre_w(0, 2);                              // h = -7
    pre_w(0, 3), pre_w(0, 4), pre_w(0, 5);                              // h = -6
    pre_x(0, 0), pre_x(0, 1), pre_x(0, 2), pre_x(0, 3), pre_w(1, 0);    // h = -5
    pre_x(0, 4), pre_x(0, 5), pre_x(0, 6), pre_x(0, 7), pre_w(1, 1);    // h = -4
    pre_w(1, 2), pre_w(1, 3), pre_w(2, 0), pre_w(2, 1), pre_w(2, 2);    // h = -3
    pre_w(1, 4), pre_w(1, 5), pre_w(2, 3), pre_w(2, 4), pre_w(2, 5);    // h = -2
    pre_x(1, 0), pre_x(1, 1), pre_x(1, 2), pre_x(1, 3), pre_w(3, 0);    // h = -1
  } else {
    pre_w(0, 0), pre_w(0, 1);                                           // h = -7
    pre_w(0, 2), pre_w(0, 3);                                           // h = -6
    pre_x(0, 0), pre_x(0, 1), pre_x(0, 2), pre_x(0, 3);                 // h = -5
    pre_x(0, 4), pre_x(0, 5), pre_x(0, 6), pre_x(0, 7);                 // h = -4
    pre_w(1, 0), pre_w(1, 1), pre_w(2, 0), pre_w(2, 1);                 // h = -3
    pre_w(1, 2), pre_w(1, 3), pre_w(2, 2), pre_w(2, 3);                 // h = -2
    pre_x(1, 0), pre_x(1, 1), pre_x(1, 2), pre_x(1, 3);                 // h = -1
  }

  // Accumulators: acc[r][j] = row block r of the wave (matrix and block as
  // rd_a), m 16 j .. +16 of its 128 rows.  Rows 0-7 in AGPRs, the rest in
  // VGPRs.  Zeroed while the first stages are in flight.
  f32x4 acc[R][8];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[r][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto fence = [&]() {
    static_for<R>([&](auto rc) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc_order<decltype(rc)::value>(acc[decltype(rc)::value][j]);
    });
  };
  fence();
  mfma_drain();
  wait_vmcnt<Cfg::kWaitFirst>();  // weight stage 0 and X block 0 landed
  __syncthreads();

  bf16x8 A[R], Bf[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) Bf[j] = rd_b(0, 0, j);
#pragma unroll
  for (int r = 0; r < H0; ++r) A[r] = rd_a(0, r);

  int g = 0;  // first stage of the current group of four
  auto mma = [&](auto rc, int j) {
    constexpr int r = decltype(rc)::value;
    if constexpr (r < 8) mfma16(A[r], Bf[j], acc[r][j]);
    else mfma16_v(A[r], Bf[j], acc[r][j]);
  };
  // M0 write / load of one scheduled refill of stage t = g + KS: L is
  // ic<kind>, D ic<d>, I ic<idx> (the schedule's WLoad, as constants).
  auto issue_m0 = [&](auto KSc, auto L, auto D, auto I) {
    constexpr int KS = decltype(KSc)::value, d = decltype(D)::value, idx = decltype(I)::value;
    if constexpr (decltype(L)::value == 0) set_m0(w_m0((KS + d) & 3, idx));
    else set_m0(x_m0(((KS >> 1) + d) & 1, idx));
  };
  auto issue_ld = [&](auto KSc, auto L, auto D, auto I) {
    constexpr int KS = decltype(KSc)::value, d = decltype(D)::value, idx = decltype(I)::value;
    if constexpr (decltype(L)::value == 0 && WNT)
      dma16_m0_nt(idx < LH ? rg : ru, w_vo[idx % LH] + (g + KS + d) * 8192, 0);
    else if constexpr (decltype(L)::value == 0)
      dma16_m0(idx < LH ? rg : ru, w_vo[idx % LH] + (g + KS + d) * 8192, 0);
    else
      dma16_m0(xrsrc, x_off[idx] + ((g >> 1) + (KS >> 1) + d) * 128, 0);
  };
  auto stage = [&](auto KSc) {
    constexpr int KS = decltype(KSc)::value;
    constexpr int H = KS & 1;
    constexpr int wb = KS & 3;                                 // weight slot of stage t
    constexpr int nwb = (KS + 1) & 3;                          // ... of stage t + 1
    constexpr int nxb = H == 0 ? (KS >> 1) & 1 : ((KS >> 1) + 1) & 1;  // X slot of stage t + 1
    constexpr int nh = 1 - H;
    constexpr HalfLoads L0 = half_loads(LW, H, 0);
    constexpr HalfLoads L1 = half_loads(LW, H, 1);
    // Half 0: rows 0..H0-1 x columns 0..7; rows H0.. of stage t read
    // meanwhile; refill r split around row r's first two MFMAs.
    static_for<H0>([&](auto rc) {
      constexpr int r = decltype(rc)::value;
      if constexpr (r < R - H0) A[H0 + r] = rd_a(wb, H0 + r);
      mma(rc, 0);
      if constexpr (r < L0.n)
        issue_m0(KSc, ic<L0.l[r].kind>{}, ic<L0.l[r].d>{}, ic<L0.l[r].idx>{});
      mma(rc, 1);
      if constexpr (r < L0.n)
        issue_ld(KSc, ic<L0.l[r].kind>{}, ic<L0.l[r].d>{}, ic<L0.l[r].idx>{});
#pragma unroll
      for (int j = 2; j < 8; ++j) mma(rc, j);
    });
    wait_lgkmcnt0();  // this wave's reads of stage t are done
    if constexpr (H == 0) wait_vmcnt<Cfg::kWaitEven>();  // stage t + 1 landed
    else wait_vmcnt<Cfg::kWaitOdd>();
    __syncthreads();  // ... for every wave; weight slot t (and at odd t X slot t/2) free
    // Half 1: rows H0..R-1 column by column; after column j, B[j] and (j < H0)
    // A[j] of stage t + 1.
    static_for<8>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      constexpr int li = half1_load_at(L1.n, j);
      mma(ic<H0>{}, j);
      if constexpr (li >= 0)
        issue_m0(KSc, ic<L1.l[li].kind>{}, ic<L1.l[li].d>{}, ic<L1.l[li].idx>{});
      mma(ic<H0 + 1>{}, j);
      if constexpr (li >= 0)
        issue_ld(KSc, ic<L1.l[li].kind>{}, ic<L1.l[li].d>{}, ic<L1.l[li].idx>{});
      static_for<R - H0 - 2>([&](auto rc) { mma(ic<H0 + 2 + decltype(rc)::value>{}, j); });
      Bf[j] = rd_b(nxb, nh, j);
      if constexpr (j < H0) A[j] = rd_a(nwb, j);
    });
  };
  for (; g < T; g += 4) {
    // T is even: stages come in pairs
    stage(ic<0>{});
    stage(ic<1>{});
    if (g + 2 >= T) break;
    stage(ic<2>{});
    stage(ic<3>{});
  }
  wait_vmcnt<0>();  // the trailing refills have landed (the epilogue reuses the LDS)
  mfma_drain();
  fence();

  if constexpr (SPLIT) {
    // Raw accumulators in register order: quad (r, j) of this wave, lane l,
    // at ((split * tiles + tile) * 4 + wave) * R * 8 + r * 8 + j quads of
    // 64 lanes -- one coalesced 1 KiB store per wave and quad.
    f32x4* const dst = reinterpret_cast<f32x4*>(a.part) +
                       ((size_t)(split * tiles + tile) * 4 + wave) * (R * 8 * 64) + lane;
    static_for<R>([&](auto rc) {
#pragma unroll
      for (int j = 0; j < 8; ++j) dst[(decltype(rc)::value * 8 + j) * 64] = acc[decltype(rc)::value][j];
    });
    return;
  }

  // ---- epilogue -------------------------------------------------------------
  // acc[r][j], lane l: output row wm*128 + 16 j + l%16 of the tile, columns
  // 16 b + 4 (l/16) + 0..3 of block b (the wave's row block r).
  __syncthreads();  // every wave is past its last operand read
  const int mr = lane & 15;
  const int h4 = 4 * (lane >> 4);
  // Block C: wave 0 finishes its m blocks 0-3 (gate here, up from wave 1's
  // row 0), wave 1 its m blocks 4-7 (up here, gate from wave 0's row C).
  // Every wave writes both halves a partner could need (wave-independent
  // code: a branch on the wave that picked different accumulators made the
  // compiler merge them through AGPR moves and scratch): row C's m blocks
  // 4-7 and row 0's m blocks 0-3, to its own 8 KiB ([half][jj] x 1 KiB).
  uint8_t* const xch_own = smem + Cfg::kXch + wave * 8192 + lane * 16;
  uint8_t* const xch_peer = smem + Cfg::kXch + (wave ^ 2) * 8192 + lane * 16;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    *reinterpret_cast<f32x4*>(xch_own + jj * 1024) = acc[C][4 + jj];
    *reinterpret_cast<f32x4*>(xch_own + 4096 + jj * 1024) = acc[0][jj];
  }
  uint8_t* const stg = smem + Cfg::kStage;
  auto put = [&](const f32x4& gv, const f32x4& uv, int blk, int j) {
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = swiglu_act(gv[q], uv[q]);
    uint8_t* const dst = stg + (wm * 128 + j * 16 + mr) * Cfg::kRowBytes + (blk * 16 + h4) * 2;
    *reinterpret_cast<uint2*>(dst) =
        make_uint2(f32x2_to_bf16x2_rne(v[0], v[1]), f32x2_to_bf16x2_rne(v[2], v[3]));
  };
  // Pairs in an order that frees the VGPR-held rows (8..R-1) first; the
  // scheduling barriers keep the compiler from reading ahead (it would
  // otherwise hold many AGPR reads and the VGPR rows at once and spill).
  // Wave 0: gate row p with up row p + C + 1 (block p); wave 1: up row p with
  // gate row C + p (block C + p).
  auto pair0 = [&](auto pc) {
    constexpr int p = decltype(pc)::value;
#pragma unroll
    for (int j = 0; j < 8; ++j) put(acc[p][j], acc[p + C + 1][j], p, j);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto pair1 = [&](auto pc) {
    constexpr int p = decltype(pc)::value;
#pragma unroll
    for (int j = 0; j < 8; ++j) put(acc[C + p][j], acc[p][j], C + p, j);
    __builtin_amdgcn_sched_barrier(0);
  };
  if (wn == 0) {
    // rows p + C + 1 >= 8 first: p from 7 - C up to C - 1, then p < 7 - C
    static_for<C>([&](auto ic_) { pair0(ic<(decltype(ic_)::value + 7 - C) % C>{}); });
  } else {
    // rows C + p >= 8 first: p from 8 - C up to C, then 1 .. 7 - C
    static_for<C>([&](auto ic_) { pair1(ic<(decltype(ic_)::value + 7 - C) % C + 1>{}); });
  }
  __syncthreads();  // the block-C halves are in LDS
  if (wn == 0) {  // up of block C, m blocks 0-3: the peer's row 0
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      put(acc[C][jj], *reinterpret_cast<const f32x4*>(xch_peer + 4096 + jj * 1024), C, jj);
  } else {  // gate of block C, m blocks 4-7: the peer's row C
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      put(*reinterpret_cast<const f32x4*>(xch_peer + jj * 1024), acc[0][4 + jj], C, 4 + jj);
  }
  __syncthreads();
  // Copy-out: 256 rows x 2 B chunks of 16 bytes.
  constexpr int kChunks = Cfg::kRowBytes / 16;
  const bool al16 = ((reinterpret_cast<uintptr_t>(a.y) | (uintptr_t)(a.ldy * 2)) & 15) == 0;
  const bool fast = al16 && m0 + 256 <= a.M && n0 + Cfg::kN <= a.N;
#pragma unroll 2
  for (int it = 0; it < kChunks; ++it) {
    const int c = it * 256 + (int)threadIdx.x;
    const int row = c / kChunks, ch = c - row * kChunks;
    const uint4 d = *reinterpret_cast<const uint4*>(stg + row * Cfg::kRowBytes + ch * 16);
    const int m = m0 + row, n = n0 + ch * 8;
    // Chunks wholly outside Y (the columns past N of the last tile column,
    // rows past M) are skipped before any other test: on those lanes the
    // element-wise path below would otherwise run its eight checks for
    // nothing, and the last column's tiles, which run in the last round, set
    // the launch's end.
    if (!fast && (m >= a.M || n >= a.N)) continue;
    uint16_t* const out = a.y + (size_t)m * a.ldy + n;
    if (fast || (al16 && n + 8 <= a.N)) {
      __builtin_nontemporal_store(u32x4{d.x, d.y, d.z, d.w}, reinterpret_cast<u32x4*>(out));
    } else {
      const uint32_t w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (n + e < a.N) out[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
    }
  }
}

// Sums the S register-order partials of each output in split order and
// applies the SiLU epilogue.  One wave per (tile, wave row wm, block b, m
// block j): lane l owns output row m0 + wm*128 + 16 j + l%16, columns
// n0 + 16 b + 4 (l/16) + 0..3; its gate and up quads sit in the wave and
// row block that held them in the tile kernel (gate b: wave wm + 2 (b > C),
// row b; up b: wave wm + 2 (b >= C), row b + C + 1 (b < C) or b - C).
template <int B>
__global__ __launch_bounds__(256) void wide_reduce_kernel(WideArgs a) {
  using Cfg = WideCfg<B>;
  constexpr int R = Cfg::R, C = Cfg::C;
  const int lane = threadIdx.x & 63;
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int tiles = a.tiles_m * a.tiles_n;
  if (unit >= (int64_t)tiles * 2 * B * 8) return;
  const int j = (int)(unit % 8);
  const int b = (int)(unit / 8 % B);
  const int wm = (int)(unit / (8 * B) % 2);
  const int tile = (int)(unit / (16 * B));
  int tm, tn;
  wide_tile_mn(a, tile, tm, tn);
  const int m = tm * 256 + wm * 128 + 16 * j + (lane & 15);
  const int n = tn * Cfg::kN + 16 * b + 4 * (lane >> 4);
  const int wg = wm + (b > C ? 2 : 0), rg = b;
  const int wu = wm + (b >= C ? 2 : 0), ru = b < C ? b + C + 1 : b - C;
  const f32x4* const src = reinterpret_cast<const f32x4*>(a.part) + lane;
  const size_t per_split = (size_t)tiles * 4 * R * 8 * 64;
  const size_t og = ((size_t)tile * 4 + wg) * (R * 8 * 64) + (size_t)(rg * 8 + j) * 64;
  const size_t ou = ((size_t)tile * 4 + wu) * (R * 8 * 64) + (size_t)(ru * 8 + j) * 64;
  f32x4 g = src[og], u = src[ou];
  for (int sp = 1; sp < a.S; ++sp) {
    g += src[sp * per_split + og];
    u += src[sp * per_split + ou];
  }
  if (m >= a.M || n >= a.N) return;
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = swiglu_act(g[q], u[q]);
  const bool vec = ((reinterpret_cast<uintptr_t>(a.y) | (uintptr_t)(a.ldy * 2)) & 7) == 0;
  store4<kOutBF16>(a.y, a.ldy, a.M, a.N, m, n, v, vec);
}

template <int B, bool SPLIT, bool WNT>
const char* wide_symbol() {
  static const std::string name = "_ZN10llk_gfx95023mfma_swiglu_wide_kernelI" + mangle_int(B) +
                                  mangle_bool(SPLIT) + mangle_bool(WNT) + "EEvNS_8WideArgsE";
  return name.c_str();
}

template <int B>
const char* wide_reduce_symbol() {
  static const std::string name = "_ZN10llk_gfx95018wide_reduce_kernelI" + mangle_int(B) +
                                  "EEvNS_8WideArgsE";
  return name.c_str();
}

template <int B, bool SPLIT, bool WNT>
static hipError_t launch_wide_kernel(const WideArgs& a, const llk::ModuleFns* mod,
                                     hipStream_t s) {
  auto fn = mfma_swiglu_wide_kernel<B, SPLIT, WNT>;
  if (!mod) {
    static std::atomic<uint64_t> lds_set{0};
    hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(fn), WideCfg<B>::kLds, lds_set);
    if (e != hipSuccess) return e;
  }
  return launch_kernel(mod, reinterpret_cast<const void*>(fn), &wide_symbol<B, SPLIT, WNT>,
                       dim3(a.tiles_m * a.tiles_n * (SPLIT ? a.S : 1)), dim3(256),
                       WideCfg<B>::kLds, s, a);
}

template <int B>
static hipError_t launch_wide_t(const WideArgs& a, const llk::ModuleFns* mod, hipStream_t s) {
  const bool wnt = a.tiles_m == 1;
  if (a.S <= 1)
    return wnt ? launch_wide_kernel<B, false, true>(a, mod, s)
               : launch_wide_kernel<B, false, false>(a, mod, s);
  hipError_t e = wnt ? launch_wide_kernel<B, true, true>(a, mod, s)
                     : launch_wide_kernel<B, true, false>(a, mod, s);
  if (e != hipSuccess) return e;
  const int64_t waves = (int64_t)a.tiles_m * a.tiles_n * 2 * B * 8;
  return launch_kernel(mod, reinterpret_cast<const void*>(wide_reduce_kernel<B>),
                       &wide_reduce_symbol<B>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                       s, a);
}

}  // namespace llk_gfx950

// Whether the wide kernel can address its weight panels (a tile's columns
// touch at most three 128-column panels of K; plus the refill stages past
// the end; 32-bit offsets) -- the host falls back to mfma_tile_kernel
// otherwise.  The same bound holds for any B and split.
bool llk_swiglu_wide_fits(int B, int KB) {
  (void)B;
  return (int64_t)3 * KB * 16384 + (int64_t)(2 * KB + 8) * 8192 < ((int64_t)1 << 31);
}

// Bytes of the register-order partials of a k split over S workgroups per
// tile (0 if S <= 1).
size_t llk_swiglu_wide_split_bytes(int B, int M, int N, int S) {
  if (S <= 1) return 0;
  const size_t tiles = (size_t)((M + 255) / 256) * ((N + 16 * B - 1) / (16 * B));
  return (size_t)S * tiles * 4 * B * 8 * 64 * 16;
}

// Internal (not part of the C ABI).  Fused SwiGLU with bf16 output over
// 16 B-column tiles.  x: [M, 64*KB] bf16, ldx % 8 == 0, 16-byte aligned,
// columns >= K zero; llk_tile_x_fits(M, ldx) and llk_swiglu_wide_fits(B, KB)
// must hold.  S > 1 splits K over S workgroups of kbs = ceil(KB / S) blocks
// (every split non-empty: the caller guarantees (S - 1) * kbs < KB); `part`
// (16-byte aligned) holds llk_swiglu_wide_split_bytes(B, M, N, S) bytes.
hipError_t llk_launch_swiglu_wide(int B, const uint16_t* x, int64_t ldx, const void* wg,
                                  const void* wu, void* y, int64_t ldy, int M, int N, int KB,
                                  int NB, int S, void* part, const llk::ModuleFns* mod,
                                  hipStream_t s) {
  using namespace llk_gfx950;
  WideArgs a;
  a.x = x;
  a.w0 = static_cast<const uint8_t*>(wg);
  a.w1 = static_cast<const uint8_t*>(wu);
  a.y = static_cast<uint16_t*>(y);
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.KB = KB;
  a.NB = NB;
  a.tiles_m = (M + 255) / 256;
  a.tiles_n = (N + 16 * B - 1) / (16 * B);
  a.group_m = 8;
  a.S = S > 1 ? S : 1;
  a.kbs = (KB + a.S - 1) / a.S;
  a.part = static_cast<float*>(part);
  if (KB < 1 || !llk_swiglu_wide_fits(B, KB)) return hipErrorInvalidValue;
  if (a.S > 1 && (part == nullptr || (int64_t)(a.S - 1) * a.kbs >= KB)) return hipErrorInvalidValue;
#if !defined(LLK_CO_OP) || LLK_CO_OP == 1
  if (B == 11) return launch_wide_t<11>(a, mod, s);
  if (B == 7) return launch_wide_t<7>(a, mod, s);
#endif
  return hipErrorInvalidValue;
}
