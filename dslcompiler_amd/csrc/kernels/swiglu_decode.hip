// swiglu_decode.hip -- bandwidth-bound kernels for small M (decode).
//
// NMAT = 2: fused SwiGLU  Y = SiLU(X Wg) * (X Wu);   NMAT = 1: C = X W.
// For M <= 32 * MT rows the weights dominate the traffic (K*N bf16 per
// matrix, read once), so the kernel is an HBM stream over the packed
// payload: every wave load is one contiguous 1 KiB MFMA operand
// (v_mfma_f32_32x32x16_bf16 A operand); X (at most 64 rows) is tiny and
// served from L2.
//
// Grid: (4 * NB / W workgroups) x S k-splits.  A workgroup owns W adjacent
// 32-column groups (of one 128-column n-block) of every matrix, as G wave
// groups of GW groups each with KS waves per wave group; each wave group's
// k range is divided among its KS waves, each streaming its part with
// UNROLL 64-k steps of loads in flight, and the waves of a k part read
// neighbouring 1 KiB sub-blocks of the same 4 KiB together.  The waves'
// partial sums meet in LDS, in wave order (a fixed order, so results are
// deterministic).  With S == 1 the workgroup then applies the epilogue
// (FuseDoubleContraction.cpp:175-199 for SwiGLU) and stores Y.  With S > 1
// it writes fp32 partials to a workspace and a second kernel adds the S
// partials in split order and applies the epilogue -- the kernel boundary
// orders the two, so no device-scope fences are needed.
#include "common.h"
#include "launch.h"
#include "tile_ops.h"

namespace llk_gfx950 {

struct SkinnyArgs {
  const uint16_t* x;  // [M, K]
  const uint8_t* w0;  // packed (Wg, or B for GEMM)
  const uint8_t* w1;  // packed (Wu), NMAT == 2
  void* y;            // [M, N]
  float* part;        // [S][NMAT][MT*32][n_pad] fp32 partials (S > 1)
  int64_t ldx, ldy;
  int M, N, K, KB, NB, S, kb_per_split, n_pad;
  bool yvec;
  bool accumulate;  // GEMM only: y += x w (the existing y read in its type)
};

template <int MT, bool XVEC>
__device__ __forceinline__ void load_x_frags(const SkinnyArgs& a, int kb, int lane,
                                             bf16x8 (&xf)[4][MT]) {
#pragma unroll
  for (int kq = 0; kq < 4; ++kq)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = t * 32 + (lane & 31);
      const int kk = kb * 64 + kq * 16 + (lane >> 5) * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (m < a.M) {
        const uint16_t* src = a.x + (size_t)m * a.ldx + kk;
        if (XVEC) {
          if (kk + 8 <= a.K) v = *reinterpret_cast<const uint4*>(src);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) e[q] = (kk + q < a.K) ? src[q] : (uint16_t)0;
          v.x = e[0] | ((uint32_t)e[1] << 16);
          v.y = e[2] | ((uint32_t)e[3] << 16);
          v.z = e[4] | ((uint32_t)e[5] << 16);
          v.w = e[6] | ((uint32_t)e[7] << 16);
        }
      }
      xf[kq][t] = *reinterpret_cast<bf16x8*>(&v);
    }
}

// A workgroup covers G * GW adjacent 32-column groups of one 128-column
// n-block: G wave groups of GW groups each, KS waves per wave group, each
// streaming a contiguous part of the k range.  Wave w serves wave group
// w % G and k part w / G; it loads each X fragment once for its GW groups
// (X traffic per workgroup is G * M * K * 2 bytes, against the weights'
// G * GW * 32 * K * 2 * NMAT), and the G * GW sub-blocks a k part reads at
// one k step are neighbouring 1 KiB pieces of the same 4 KiB.
// Floats of one matrix's partial sums in the reduction buffer, and whether
// both matrices' fit (128 KiB) so that they reduce in one pass.
constexpr int skinny_red_floats(int KS, int G, int GW, int MT) { return KS * G * GW * MT * 16 * 64; }
constexpr bool skinny_one_pass(int NMAT, int red_floats) {
  return NMAT == 2 && 2 * red_floats * (int)sizeof(float) <= 131072;
}

// PIPE: the weight loads of the next 64-k step are issued before this
// step's MFMAs (one step of weights in flight per wave beyond the one being
// used; UNROLL is then unused) -- the form for the shapes whose register
// budget holds two steps, measured 1.5% faster at decode M = 8 and 3-8%
// faster for SwiGLU at M = 40-64 (N = 14336, K = 4096).
template <int NMAT, int MT, int KS, int G, int GW, int OUT, bool XVEC, int UNROLL, bool PIPE>
__global__ __launch_bounds__(KS * G * 64) void skinny_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) float red[];  // [1 or NMAT][KS][G][GW][MT][16][64]
  constexpr int NT = KS * G * 64;
  constexpr int TOT = G * GW * MT * 4 * 64;  // output quads of the workgroup
  constexpr int EPT = (TOT + NT - 1) / NT;   // quads per thread
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gi = wave % G;
  const int kpart = wave / G;
  const int nwg = a.NB * 4 / (G * GW);  // workgroups per k split
  const int wg = blockIdx.x % nwg;
  const int split = blockIdx.x / nwg;
  const int grp0 = (wg * G + gi) * GW;  // first 32-column group of this wave

  // k range of this workgroup, then of this wave (contiguous chunks).
  const int kb0 = split * a.kb_per_split;
  const int kb1 = min(a.KB, kb0 + a.kb_per_split);
  const int span = kb1 > kb0 ? kb1 - kb0 : 0;
  const int per_wave = (span + KS - 1) / KS;
  const int wb0 = kb0 + kpart * per_wave;
  const int wb1 = min(kb1, wb0 + per_wave);

  f32x16 acc[GW][NMAT][MT];
#pragma unroll
  for (int j = 0; j < GW; ++j)
#pragma unroll
    for (int p = 0; p < NMAT; ++p)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][p][t][r] = 0.0f;

  // Sub-block (kq, n32 + j) of block (nb, kb): + kb*16K + (kq*4 + n32 + j)*1K;
  // GW divides 4 and grp0, so the GW groups share the n-block.
  const int nb = grp0 >> 2, n32 = grp0 & 3;
  const size_t panel = (size_t)nb * a.KB * kBlockBytes + n32 * kSubBytes + lane * 16;
  const uint8_t* wbase[2] = {a.w0 + panel, (NMAT == 2 ? a.w1 : a.w0) + panel};

  // One 64-k step: the weight operands (NMAT matrices x 4 k quarters x GW
  // column groups, 1 KiB wave loads) and this step's MFMAs.
  auto load_w = [&](int kbb, u32x4 (&w)[NMAT][4][GW]) {
#pragma unroll
    for (int p = 0; p < NMAT; ++p)
#pragma unroll
      for (int kq = 0; kq < 4; ++kq)
#pragma unroll
        for (int j = 0; j < GW; ++j)
          w[p][kq][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
              wbase[p] + (size_t)kbb * kBlockBytes + (kq * 4 + j) * kSubBytes));
  };
  auto step = [&](const u32x4 (&w)[NMAT][4][GW], const bf16x8 (&xf)[4][MT]) {
#pragma unroll
    for (int kq = 0; kq < 4; ++kq)
#pragma unroll
      for (int j = 0; j < GW; ++j)
#pragma unroll
        for (int p = 0; p < NMAT; ++p) {
          const bf16x8 wop = *reinterpret_cast<const bf16x8*>(&w[p][kq][j]);
#pragma unroll
          for (int t = 0; t < MT; ++t) acc[j][p][t] = mfma32(wop, xf[kq][t], acc[j][p][t]);
        }
  };
  if constexpr (PIPE) {
    // Weights of step kb+1 are requested before step kb's MFMAs; X (from
    // L2) just before its step, ahead of those weights so that its wait
    // does not include them.
    u32x4 w0[NMAT][4][GW], w1[NMAT][4][GW];
    bf16x8 xf[4][MT];
    int kb = wb0;
    if (kb < wb1) load_w(kb, w0);
    for (; kb + 2 <= wb1; kb += 2) {
      load_x_frags<MT, XVEC>(a, kb, lane, xf);
      load_w(kb + 1, w1);
      step(w0, xf);
      load_x_frags<MT, XVEC>(a, kb + 1, lane, xf);
      if (kb + 2 < wb1) load_w(kb + 2, w0);
      step(w1, xf);
    }
    if (kb < wb1) {
      load_x_frags<MT, XVEC>(a, kb, lane, xf);
      step(w0, xf);
    }
  } else {
    int kb = wb0;
    for (; kb + UNROLL <= wb1; kb += UNROLL) {
      u32x4 w[UNROLL][NMAT][4][GW];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) load_w(kb + u, w[u]);
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        bf16x8 xf[4][MT];
        load_x_frags<MT, XVEC>(a, kb + u, lane, xf);
        step(w[u], xf);
      }
    }
    for (; kb < wb1; ++kb) {  // remainder steps
      u32x4 w[NMAT][4][GW];
      load_w(kb, w);
      bf16x8 xf[4][MT];
      load_x_frags<MT, XVEC>(a, kb, lane, xf);
      step(w, xf);
    }
  }

  // ---- reduce the KS waves' partial sums in LDS, in wave order: both
  // matrices in one pass when their partials fit 128 KiB, else one matrix
  // per pass.  Quad e of the workgroup = (group ge, t, g, ln): rows m = t*32 +
  // ln%32 and the 4 consecutive columns 8g + 4*(ln/32) + 0..3 (accumulator
  // r = 4g + q) of group ge; thread x handles quads x, x + NT, ...
  constexpr int kRed = skinny_red_floats(KS, G, GW, MT);  // per matrix
  constexpr bool kOnePass = skinny_one_pass(NMAT, kRed);
  float sum[EPT][NMAT][4];
  auto write_red = [&](int p, float* base) {
#pragma unroll
    for (int j = 0; j < GW; ++j)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          base[(((wave * GW + j) * MT + t) * 16 + r) * 64 + lane] = acc[j][p][t][r];
  };
  auto read_red = [&](int p, const float* base) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int e = threadIdx.x + i * NT;
      if (TOT % NT != 0 && e >= TOT) break;
      const int ln = e & 63, g = (e >> 6) & 3, t = (e >> 8) % MT, ge = e / (MT * 4 * 64);
      const int gg = ge / GW, j = ge % GW;  // wave group, group within the wave
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float s = 0.0f;
        for (int w2 = 0; w2 < KS; ++w2)
          s += base[((((w2 * G + gg) * GW + j) * MT + t) * 16 + 4 * g + q) * 64 + ln];
        sum[i][p][q] = s;
      }
    }
  };
  if constexpr (kOnePass) {
#pragma unroll
    for (int p = 0; p < NMAT; ++p) write_red(p, red + p * kRed);
    __syncthreads();
#pragma unroll
    for (int p = 0; p < NMAT; ++p) read_red(p, red + p * kRed);
  } else {
#pragma unroll
    for (int p = 0; p < NMAT; ++p) {
      if (p > 0) __syncthreads();  // the previous pass's readers are done
      write_red(p, red);
      __syncthreads();
      read_red(p, red);
    }
  }

  // With S == 1 apply the epilogue (FuseDoubleContraction.cpp:175-199 for
  // SwiGLU) and store Y; with S > 1 write the fp32 partials.
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int e = threadIdx.x + i * NT;
    if (TOT % NT != 0 && e >= TOT) break;
    const int ln = e & 63, g = (e >> 6) & 3, t = (e >> 8) % MT, ge = e / (MT * 4 * 64);
    const int eg = wg * G * GW + ge;
    const int m = t * 32 + (ln & 31);
    const int n = (eg >> 2) * kPackN + (eg & 3) * 32 + 8 * g + 4 * (ln >> 5);
    if (a.S > 1) {
      if (n < a.n_pad && m < a.M) {  // the reduce reads rows < M only
#pragma unroll
        for (int p = 0; p < NMAT; ++p) {
          float* dst = a.part + (((size_t)split * NMAT + p) * (MT * 32) + m) * a.n_pad + n;
          *reinterpret_cast<f32x4*>(dst) =
              f32x4{sum[i][p][0], sum[i][p][1], sum[i][p][2], sum[i][p][3]};
        }
      }
    } else {
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if constexpr (NMAT == 2)
          v[q] = swiglu_act(sum[i][0][q], sum[i][1][q]);
        else
          v[q] = sum[i][0][q];
      }
      if constexpr (NMAT == 1) {
        if (a.accumulate) add_existing4<OUT>(a.y, a.ldy, a.M, a.N, m, n, v, a.yvec);
      }
      store4<OUT>(a.y, a.ldy, a.M, a.N, m, n, v, a.yvec);
    }
  }
}

// Adds the S partials in split order and applies the epilogue: thread
// handles 4 consecutive n of one row.
template <int NMAT, int OUT>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(SkinnyArgs a, int rows) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int quads = a.n_pad / 4;
  if (e >= (int64_t)a.M * quads) return;
  const int m = (int)(e / quads);
  const int n = (int)(e % quads) * 4;
  f32x4 s[NMAT];
#pragma unroll
  for (int p = 0; p < NMAT; ++p) s[p] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < a.S; ++sp)
#pragma unroll
    for (int p = 0; p < NMAT; ++p)
      s[p] += *reinterpret_cast<const f32x4*>(a.part + (((size_t)sp * NMAT + p) * rows + m) * a.n_pad + n);
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if constexpr (NMAT == 2)
      v[q] = swiglu_act(s[0][q], s[1][q]);
    else
      v[q] = s[0][q];
  }
  if constexpr (NMAT == 1) {
    if (a.accumulate) add_existing4<OUT>(a.y, a.ldy, a.M, a.N, m, n, v, a.yvec);
  }
  store4<OUT>(a.y, a.ldy, a.M, a.N, m, n, v, a.yvec);
}

// Launch shape for (NMAT, MT) and a workgroup width of W 32-column groups:
// GW groups per wave, G = W / GW wave groups, KS waves per wave group,
// UNROLL k steps of weight loads in flight.  One matrix with M <= 32 rows
// already holds an X fragment for two groups (GW = 2, the X traffic halves);
// SwiGLU with M <= 32 keeps GW = 1 and 16 waves (X is a small part of its
// traffic, the deeper wave count wins); with M > 32 both use GW = 2 (at
// M = 64 X traffic equals the weights').  Register budgets: KS * G * 64
// threads with at most 512 / waves-per-SIMD VGPRs each; the SwiGLU M > 32
// form holds 2 x 2 x 2 accumulators (128 AGPRs) plus 2 k steps of loads
// (376 VGPRs with the pipelined loop, one wave per SIMD).  LDS: KS * G * GW * MT * 4 KiB per matrix, both matrices
// at once when that fits 128 KiB.
template <int NMAT, int MT, int W>
struct SkinnyCfg {
  static constexpr int GW = (W == 1 || (NMAT == 2 && MT == 1)) ? 1 : 2;
  static constexpr int G = W / GW;
  static constexpr int KS =
      GW == 1 ? (G == 1 ? ((NMAT * MT <= 2) ? 8 : 4)
                        : (32 / (G * NMAT * MT) < 16 / G ? 32 / (G * NMAT * MT) : 16 / G))
              : (NMAT == 2 ? 4 / G : (MT == 1 ? 16 / G : 4));
  static constexpr int UNROLL = (GW == 2 && NMAT == 1 && MT == 1) ? 1 : 2;
  // M <= 32 with one group per wave or one wave group, up to 8 waves per
  // wave group, and SwiGLU with M > 32 (one wave group of two groups, four
  // waves): two steps of weights in flight fit the registers (the 4-group
  // forms with 4 waves per group spill).  The GEMM with M > 32 keeps the
  // plain loop, 1-4% faster there (M = 48, 64).
  static constexpr bool PIPE =
      (MT == 1 && (GW == 1 || G == 1) && G * GW <= 2) || (NMAT == 2 && MT == 2 && G == 1 && GW == 2);
  static constexpr size_t lds = (size_t)skinny_red_floats(KS, G, GW, MT) * sizeof(float) *
                                (skinny_one_pass(NMAT, skinny_red_floats(KS, G, GW, MT)) ? 2 : 1);
  static_assert(G * GW == W && KS * G <= 16 && lds <= 131072, "small-M launch shape");
};

template <int NMAT, int MT, int KS, int G, int GW, int OUT, bool XVEC, int UNROLL, bool PIPE>
const char* skinny_symbol() {
  static const std::string name = "_ZN10llk_gfx95013skinny_kernelI" + mangle_int(NMAT) +
                                  mangle_int(MT) + mangle_int(KS) + mangle_int(G) +
                                  mangle_int(GW) + mangle_int(OUT) + mangle_bool(XVEC) +
                                  mangle_int(UNROLL) + mangle_bool(PIPE) +
                                  "EEvNS_10SkinnyArgsE";
  return name.c_str();
}

template <int NMAT, int OUT>
const char* skinny_reduce_symbol() {
  static const std::string name = "_ZN10llk_gfx95020skinny_reduce_kernelI" + mangle_int(NMAT) +
                                  mangle_int(OUT) + "EEvNS_10SkinnyArgsEi";
  return name.c_str();
}

// mod: a loaded per-operation code object, or null for the library's own
// kernels.
template <int NMAT, int MT, int W, int OUT, bool XVEC>
static hipError_t launch_skinny_t(const SkinnyArgs& a, const llk::ModuleFns* mod,
                                  hipStream_t s) {
  using C = SkinnyCfg<NMAT, MT, W>;
  // (the element-wise X path of unaligned rows needs the registers the
  // second step of weights would take)
  constexpr bool kPipe = C::PIPE && XVEC;
  auto fn = skinny_kernel<NMAT, MT, C::KS, C::G, C::GW, OUT, XVEC, C::UNROLL, kPipe>;
  if (C::lds > 65536 && !mod) {
    static std::atomic<uint64_t> lds_set{0};  // devices configured, per instantiation
    hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(fn), (int)C::lds, lds_set);
    if (e != hipSuccess) return e;
  }
  hipError_t e = launch_kernel(
      mod, reinterpret_cast<const void*>(fn),
      &skinny_symbol<NMAT, MT, C::KS, C::G, C::GW, OUT, XVEC, C::UNROLL, kPipe>,
      dim3(a.NB * 4 / W * a.S), dim3(C::KS * C::G * 64), (unsigned)C::lds, s, a);
  if (e != hipSuccess || a.S == 1) return e;
  const int64_t threads = (int64_t)a.M * (a.n_pad / 4);
  return launch_kernel(mod, reinterpret_cast<const void*>(skinny_reduce_kernel<NMAT, OUT>),
                       &skinny_reduce_symbol<NMAT, OUT>,
                       dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, a, MT * 32);
}

template <int NMAT, int MT, int W, int OUT>
static hipError_t launch_skinny_o(const SkinnyArgs& a, bool xvec, const llk::ModuleFns* mod,
                                  hipStream_t s) {
  return xvec ? launch_skinny_t<NMAT, MT, W, OUT, true>(a, mod, s)
              : launch_skinny_t<NMAT, MT, W, OUT, false>(a, mod, s);
}

// fp16 output exists for the GEMM (NMAT 1) only.
template <int NMAT, int MT, int W>
static hipError_t launch_skinny_g(const SkinnyArgs& a, int out, bool xvec,
                                  const llk::ModuleFns* mod, hipStream_t s) {
  if (out == kOutBF16) return launch_skinny_o<NMAT, MT, W, kOutBF16>(a, xvec, mod, s);
  if (out == kOutF32) return launch_skinny_o<NMAT, MT, W, kOutF32>(a, xvec, mod, s);
  if constexpr (NMAT == 1) {
    if (out == kOutF16) return launch_skinny_o<NMAT, MT, W, kOutF16>(a, xvec, mod, s);
  }
  return hipErrorInvalidValue;
}

template <int NMAT, int MT>
static hipError_t launch_skinny_mt(const SkinnyArgs& a, int W, int out, bool xvec,
                                   const llk::ModuleFns* mod, hipStream_t s) {
  if (W == 4) return launch_skinny_g<NMAT, MT, 4>(a, out, xvec, mod, s);
  if (W == 2) return launch_skinny_g<NMAT, MT, 2>(a, out, xvec, mod, s);
  return launch_skinny_g<NMAT, MT, 1>(a, out, xvec, mod, s);
}

template <int NMAT, int MT>
static int skinny_threads_w(int W) {
  if (W == 4) return SkinnyCfg<NMAT, MT, 4>::KS * SkinnyCfg<NMAT, MT, 4>::G * 64;
  if (W == 2) return SkinnyCfg<NMAT, MT, 2>::KS * SkinnyCfg<NMAT, MT, 2>::G * 64;
  return SkinnyCfg<NMAT, MT, 1>::KS * SkinnyCfg<NMAT, MT, 1>::G * 64;
}


// ---- decode tile kernel ------------------------------------------------------
//
// The small-M form for K a multiple of 64 and X rows 16-byte aligned
// (ldx % 8 == 0): a workgroup streams its columns' weights and all of X
// through a ring of three 64-k step slots in LDS, every byte by LDS-DMA
// (buffer_load_dwordx4 ... lds, as the tile kernels), two steps ahead of the
// MFMAs.  Weights are the packed payload's contiguous 1 KiB sub-blocks, read
// non-temporal: each weight byte is read once, and streaming them past L2
// keeps X there (decode M = 64, N = 14336, K = 4096: 43.3 us with ordinary
// weight loads, 37.7 us with `nt`).  X moves as whole 128-byte row segments
// (64 rows; rows >= M read zero through the buffer range check), its 16-byte
// chunks XOR-swizzled by row & 7 in LDS, so that an MFMA B operand (32 rows x
// 16 bytes per half wave) hits every bank once.  Every wave issues four
// weight loads, then two X loads per step, so "step kb has landed" is
// vmcnt(6) for each wave, then one barrier for the workgroup; the slot the
// barrier frees (step kb - 1's) takes step kb + 2, and X, like the weights,
// is loaded two steps ahead of its use.  (Issuing only the X loads that have
// rows < M, X first with vmcnt(4), left X one step ahead: at M = 16 and 32,
// where a few waves read the same X lines as every other workgroup, 46 and
// 45 us instead of 37 and 38.)  The kernel has no k parts inside a workgroup
// and no partial sums in LDS.
//
// A step is 16 weight sub-blocks (16 KiB) + 8 KiB of X per 64 rows.  SwiGLU
// (NMAT 2): a workgroup covers 64 columns (half an n-block) of Wg and Wu;
// GEMM (NMAT 1): 128 columns (one n-block).  Wave w = (column group
// c = w & 1, m half h = w >> 1) accumulates acc[p][t] = 32 columns x 32 rows
// (rows 32 (MT h + t) .. +32, t < MT), p = 0, 1 (SwiGLU: gate and up of the
// same columns, so the epilogue is register-local; GEMM: column groups c and
// 2 + c).  With S > 1 workgroup (columns, s) covers the 64-k blocks
// [s kbs, (s + 1) kbs) and writes fp32 partials in the layout of
// skinny_kernel's, which skinny_reduce_kernel adds in split order.
//
// MT (32-row MFMA tiles per wave: 1, 2, 4) sets the rows a workgroup holds,
// 64 MT: MT = 1 for M <= 64 (decode), 2 and 4 for mid M (65..256 rows, one
// m tile), where every weight byte is still read by one workgroup only --
// the tile kernels need 256-row tiles and a k split to give 256 CUs work
// there, and write fp32 partial planes for it.  Each step then carries 8 MT
// KiB of X (from L2) beside the same 16 KiB of weights and 8 MT MFMAs per
// wave; the ring keeps three slots (144 KiB at MT = 4).  Measured on config
// 5's MLP (K = 5120, N = 13824): M = 65 and 128 take 86 and 100 us against
// 114 and 126 us on the tile kernels, but at MT = 4 a step takes ~1.2 us
// (the SwiGLU at M = 255: 97 us, against 74 us + 11 us of reduce for the
// wide kernel's two k splits): per CU the loads in flight, not the MFMAs,
// set the pace (about 34 KiB at once), and 32 KiB of X per step share them
// with 16 KiB of weights -- so the dispatcher stops at 128 rows by default.
struct DecTileArgs {
  const uint16_t* x;  // [M, K], row stride ldx
  const uint8_t* w0;  // packed (Wg, or B for the GEMM)
  const uint8_t* w1;  // packed (Wu), NMAT == 2
  void* y;            // [M, N]
  float* part;        // [S][NMAT][rows][n_pad] fp32 partials (S > 1)
  int64_t ldx, ldy;
  int M, N, KB, NB, S, kbs, n_pad, rows;
  bool yvec;
  bool accumulate;  // GEMM only, S == 1: y += x w (the existing y read in its type)
  // The row-major form (RM): w0 / w1 are bf16 [K, N] with rows of ldw0 /
  // ldw1 elements instead of packed payloads.
  int64_t ldw0, ldw1;
};

constexpr int kDecSlots = 3;  // ring slots (64-k steps)
constexpr int kDecW = 16384;  // weights per slot, then X (8 KiB per 64 rows)
constexpr int dec_slot_bytes(int MT) { return kDecW + 8192 * MT; }
constexpr int dec_lds_bytes(int MT) { return kDecSlots * dec_slot_bytes(MT); }  // 72 / 96 / 144 KiB
// 32-row MFMA tiles per wave for M rows (M <= 256).
constexpr int dec_mt(int M) { return M <= 64 ? 1 : M <= 128 ? 2 : 4; }

template <int NMAT, int OUT, int MT, bool RM>
__global__ __launch_bounds__(256) void decode_tile_kernel(DecTileArgs a) {
  static_assert(MT == 1 || MT == 2 || MT == 4, "64, 128 or 256 rows per workgroup");
  constexpr int kAhead = kDecSlots - 1;
  constexpr int kDecSlot = dec_slot_bytes(MT);
  constexpr int kXL = 2 * MT;       // X loads per wave and step (8 rows each)
  constexpr int kLoads = 4 + kXL;   // loads per wave and step
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cg = wave & 1, mh = wave >> 1;
  const int per_split = NMAT == 2 ? a.NB * 2 : a.NB;
  const int grp = blockIdx.x % per_split;
  const int split = blockIdx.x / per_split;
  const int nb = NMAT == 2 ? grp >> 1 : grp;
  const int kb0 = split * a.kbs;
  const int nkb = min(a.KB - kb0, a.kbs);

  // Weight resources and this wave's four loads per 64-k step (offset of
  // step kb: w_vo[q] + kb * w_step, LDS place: w_lds[q] in the slot).
  u32x4 rw_lo, rw_hi;
  int w_vo[4];
  uint32_t w_lds[4];
  int w_step;
  if constexpr (!RM) {
    // Packed: this n-block's panel from 64-k block kb0 (loads past the panel
    // read zero).  Sub-blocks i = 4 wave + q of the step, i.e. operand
    // p = i >> 3, k quarter (i >> 1) & 3, column group c = i & 1 -- packed
    // 32-column group 2 (grp & 1) + c of matrix p (SwiGLU) or 2 p + c
    // (GEMM) -- placed at ((p * 2 + c) * 4 + kq) KiB of the slot.
    const int64_t panel = (int64_t)a.KB * kBlockBytes;
    const int64_t woff = (int64_t)nb * panel + (int64_t)kb0 * kBlockBytes;
    const int wbytes = (int)(panel - (int64_t)kb0 * kBlockBytes);
    rw_lo = buffer_rsrc(a.w0 + woff, wbytes);
    rw_hi = buffer_rsrc((NMAT == 2 ? a.w1 : a.w0) + woff, wbytes);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = wave * 4 + q, p = i >> 3, kq = (i >> 1) & 3, c = i & 1;
      const int n32 = NMAT == 2 ? 2 * (grp & 1) + c : 2 * p + c;
      w_vo[q] = (kq * 4 + n32) * kSubBytes + lane * 16;
      w_lds[q] = (uint32_t)(((p * 2 + c) * 4 + kq) * 1024);
    }
    w_step = kBlockBytes;
  } else {
    // Row-major: slab p of the slot (8 KiB: 64 k rows x 64 columns, 128 bytes
    // a row) holds matrix p's 64 columns of this workgroup (SwiGLU) or its
    // columns 64 p .. +64 (GEMM).  Load i = 4 wave + q fetches slab i >> 3,
    // rows 8 (i & 7) .. +8, lane l row r = 8 (i & 7) + l / 8 and 16-byte
    // chunk l & 7 of the LDS row, which holds the row's chunk (l & 7) ^ sw(r),
    // sw(r) = 4 (bit 1 of r ^ bit 3 of r): the row's 64-byte halves swapped
    // where the two bits differ, so that the transposed reads of an A
    // operand (rows k .. k + 3 in each half-wave) meet 64 distinct banks.
    // Resources reach from row 64 kb0 to the matrix's last element: rows
    // past K and columns of a slab starting at or past N read zero.
    const int K = a.KB * 64;
    auto slab = [&](const uint8_t* w, int64_t ldw, int ncol) {
      const int64_t left = ((int64_t)(K - kb0 * 64 - 1) * ldw + (a.N - ncol)) * 2;
      return buffer_rsrc(w + ((int64_t)kb0 * 64 * ldw + ncol) * 2, ncol < a.N ? (int)left : 0);
    };
    const int n0 = NMAT == 2 ? grp * 64 : nb * kPackN;
    rw_lo = slab(a.w0, a.ldw0, n0);
    rw_hi = NMAT == 2 ? slab(a.w1, a.ldw1, n0) : slab(a.w0, a.ldw0, n0 + 64);
    const int64_t ldw = NMAT == 2 && wave >= 2 ? a.ldw1 : a.ldw0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = wave * 4 + q;
      const int r = (i & 7) * 8 + (lane >> 3);
      const int sw = 4 * (((lane >> 4) ^ i) & 1);  // bits 1 and 3 of r
      w_vo[q] = (int)((r * ldw + (((lane & 7) ^ sw) * 8)) * 2);
      w_lds[q] = (uint32_t)((i >> 3) * 8192 + (i & 7) * 1024);
    }
    w_step = (int)(64 * ldw * 2);
  }
  const u32x4 rx = buffer_rsrc(a.x + (size_t)kb0 * 64,
                               (int)((int64_t)a.M * a.ldx * 2 - (int64_t)kb0 * 128));
  // This wave's X loads: rows 8 f .. 8 f + 7 for f = 2 MT wave + q, lane l
  // fetching physical chunk l & 7 of row 8 f + l / 8, i.e. logical chunk
  // (l & 7) ^ (row & 7).  Loads of rows >= M read zeros (no memory traffic)
  // but are issued all the same, so that every wave waits for one count.
  int x_vo[kXL];
#pragma unroll
  for (int q = 0; q < kXL; ++q) {
    const int row = 8 * (wave * kXL + q) + (lane >> 3);
    x_vo[q] = (row * (int)a.ldx + (((lane & 7) ^ (row & 7)) * 8)) * 2;
  }
  const uint32_t lds0 = lds_addr(smem);
  const u32x4 rw_mine = wave < 2 ? rw_lo : rw_hi;  // operand p = wave >> 1
  auto issue = [&](int kb, int slot) {
    const uint32_t base = lds0 + (uint32_t)(slot * kDecSlot);
#pragma unroll
    for (int q = 0; q < 4; ++q) dma16_nt(rw_mine, w_vo[q] + kb * w_step, 0, base + w_lds[q]);
#pragma unroll
    for (int q = 0; q < kXL; ++q)
      dma16(rx, x_vo[q] + kb * 128, 0, base + kDecW + (uint32_t)(wave * kXL + q) * 1024);
  };
  // Steps past the split's end read zeros (weights) or unused X into slots
  // no MFMA reads: the load count per step stays uniform.
#pragma unroll
  for (int s = 0; s < kAhead; ++s) issue(s, s);

  f32x16 acc[2][MT];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[p][t][r] = 0.0f;
  const uint8_t* const a_rd = smem + cg * 4096 + lane * 16;  // + slot + p * 8 KiB + kq KiB
  // RM: lane l's A operand -- k = 16 kq + 8 (l / 32) + 0..7 of column
  // n = 32 cg + l % 32 -- is two transposed reads (ds_read_b64_tr_b16, k
  // + 0..3 and + 4..7).  Such a read gives lane i of each 16-lane group, as
  // element j, element i % 4 of the 8 bytes named by the group's lane
  // i / 4 + 4 j; so the group's lane 4 j + c names row k + j, columns
  // n0 + 4 c .. + 3 (n0 = 32 cg + 16 (g & 1), g = l / 16), and lane i
  // receives column n0 + i at rows k .. k + 3 (element (k, n) of a slab at
  // k * 128 + 2 n, its 16-byte chunk XOR sw(k) as loaded).
  const int a_g = lane >> 4, a_j = (lane >> 2) & 3, a_c = lane & 3;
  const int a_chunk = (4 * cg + 2 * (a_g & 1) + (a_c >> 1)) ^ (4 * ((a_j >> 1) ^ (a_g >> 1)));
  const uint16_t* const a_rm = reinterpret_cast<const uint16_t*>(smem) +
                               (8 * (a_g >> 1) + a_j) * 64 + a_chunk * 8 + 4 * (a_c & 1);
  auto rd_a = [&](int off, int p, int kq) -> bf16x8 {
    if constexpr (!RM) {
      return *reinterpret_cast<const bf16x8*>(a_rd + off + p * 8192 + kq * 1024);
    } else {
      typedef short v4i16 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) v4i16* lds_v4i16;
      const uint16_t* const src = a_rm + (off + p * 8192) / 2 + kq * 16 * 64;
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16)(src));
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16)(src + 4 * 64));
      return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };
  const int xm = mh * 32 * MT + (lane & 31);                  // the B operand's row (t = 0)
  const uint8_t* const b_rd = smem + kDecW + xm * 128;        // + t * 4 KiB: tile t's rows
  int slot = 0, fill = kAhead;
  if constexpr (MT == 1) {
    for (int kb = 0; kb < nkb; ++kb) {
      wait_vmcnt<kLoads * (kAhead - 1)>();  // this wave's loads of step kb have landed
      __syncthreads();                      // ... every wave's; slot `fill` (step kb - 1) is free
      issue(kb + kAhead, fill);
      fill = fill + 1 == kDecSlots ? 0 : fill + 1;
      const int off = slot * kDecSlot;
      bf16x8 A[2][4], Bx[4];
#pragma unroll
      for (int kq = 0; kq < 4; ++kq) {
        Bx[kq] = *reinterpret_cast<const bf16x8*>(b_rd + off +
                                                  (((2 * kq + (lane >> 5)) ^ (xm & 7)) * 16));
#pragma unroll
        for (int p = 0; p < 2; ++p)
          A[p][kq] = rd_a(off, p, kq);
      }
#pragma unroll
      for (int kq = 0; kq < 4; ++kq)
#pragma unroll
        for (int p = 0; p < 2; ++p) acc[p][0] = mfma32(A[p][kq], Bx[kq], acc[p][0]);
      slot = slot + 1 == kDecSlots ? 0 : slot + 1;
    }
  } else {
    // 2 MT MFMAs per 16-k quarter kq, and the LDS serves 4 (2 + MT) KiB of
    // operands per quarter to the workgroup's waves beside the ring's DMA
    // writes: the operand reads of quarter kq + 1 are issued before the
    // MFMAs of quarter kq (two register sets), and step kb + 1's barrier --
    // after this wave's reads of step kb are done -- comes before step kb's
    // last quarter, whose MFMAs then cover step kb + 1's first reads.
    bf16x8 A[2][2], Bx[2][MT];
    auto rd = [&](int off, int kq, int buf) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
        Bx[buf][t] = *reinterpret_cast<const bf16x8*>(
            b_rd + off + t * 4096 + (((2 * kq + (lane >> 5)) ^ (xm & 7)) * 16));
#pragma unroll
      for (int p = 0; p < 2; ++p)
        A[buf][p] = rd_a(off, p, kq);
    };
    auto mf = [&](int buf) {
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[p][t] = mfma32(A[buf][p], Bx[buf][t], acc[p][t]);
      __builtin_amdgcn_sched_barrier(0);
    };
    wait_vmcnt<kLoads * (kAhead - 1)>();  // step 0 has landed (this wave's loads) ...
    __syncthreads();                      // ... and every wave's
    issue(kAhead, fill);
    fill = 0;
    rd(0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    for (int kb = 0; kb < nkb; ++kb) {
      const int off = slot * kDecSlot;
      rd(off, 1, 1);
      mf(0);
      rd(off, 2, 0);
      mf(1);
      rd(off, 3, 1);
      mf(0);
      if (kb + 1 < nkb) {
        wait_lgkmcnt0();                      // this wave's reads of step kb are done
        wait_vmcnt<kLoads * (kAhead - 1)>();  // its loads of step kb + 1 have landed
        __syncthreads();                      // every wave's; slot `fill` (step kb) is free
        issue(kb + 1 + kAhead, fill);
        fill = fill + 1 == kDecSlots ? 0 : fill + 1;
        slot = slot + 1 == kDecSlots ? 0 : slot + 1;
        rd(slot * kDecSlot, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      mf(1);
    }
  }
  wait_vmcnt<0>();  // the trailing loads have landed before the workgroup ends

  // acc[p][t] register r, lane l: row m = 32 (MT h + t) + l % 32, column
  // 8 (r / 4) + 4 (l / 32) + r % 4 of the wave's 32-column group of operand p.
  const int n_col = NMAT == 2 ? grp * 64 + cg * 32 : nb * kPackN + cg * 32;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = xm + 32 * t;
    if (MT > 1 && m >= a.rows) continue;  // rows past M's last 32-row group
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n_off = 8 * g + 4 * (lane >> 5);
      if (a.S > 1) {
        if (m < a.M) {  // the reduce reads rows < M only
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            const int mat = NMAT == 2 ? p : 0;
            const int n = n_col + (NMAT == 2 ? 0 : p * 64) + n_off;
            float* dst = a.part + (((size_t)split * NMAT + mat) * a.rows + m) * a.n_pad + n;
            *reinterpret_cast<f32x4*>(dst) = f32x4{acc[p][t][4 * g], acc[p][t][4 * g + 1],
                                                   acc[p][t][4 * g + 2], acc[p][t][4 * g + 3]};
          }
        }
      } else if constexpr (NMAT == 2) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          v[q] = swiglu_act(acc[0][t][4 * g + q], acc[1][t][4 * g + q]);
        store4<OUT>(a.y, a.ldy, a.M, a.N, m, n_col + n_off, v, a.yvec);
      } else {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = acc[p][t][4 * g + q];
          const int n = n_col + p * 64 + n_off;
          if (a.accumulate) add_existing4<OUT>(a.y, a.ldy, a.M, a.N, m, n, v, a.yvec);
          store4<OUT>(a.y, a.ldy, a.M, a.N, m, n, v, a.yvec);
        }
      }
    }
  }
}

template <int NMAT, int OUT, int MT, bool RM>
const char* decode_tile_symbol() {
  static const std::string name = "_ZN10llk_gfx95018decode_tile_kernelI" + mangle_int(NMAT) +
                                  mangle_int(OUT) + mangle_int(MT) + mangle_bool(RM) +
                                  "EEvNS_11DecTileArgsE";
  return name.c_str();
}

template <int NMAT, int OUT, int MT, bool RM>
static hipError_t launch_decode_tile_t(const DecTileArgs& a, const llk::ModuleFns* mod,
                                       hipStream_t s) {
  auto fn = decode_tile_kernel<NMAT, OUT, MT, RM>;
  constexpr int kLds = dec_lds_bytes(MT);
  if (!mod) {
    static std::atomic<uint64_t> lds_set{0};
    hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(fn), kLds, lds_set);
    if (e != hipSuccess) return e;
  }
  const unsigned groups = (unsigned)((NMAT == 2 ? a.NB * 2 : a.NB) * a.S);
  hipError_t e = launch_kernel(mod, reinterpret_cast<const void*>(fn),
                               &decode_tile_symbol<NMAT, OUT, MT, RM>, dim3(groups), dim3(256), kLds,
                               s, a);
  if (e != hipSuccess || a.S == 1) return e;
  SkinnyArgs r{};
  r.y = a.y;
  r.part = a.part;
  r.ldy = a.ldy;
  r.M = a.M;
  r.N = a.N;
  r.S = a.S;
  r.n_pad = a.n_pad;
  r.yvec = a.yvec;
  r.accumulate = a.accumulate;
  const int64_t threads = (int64_t)a.M * (a.n_pad / 4);
  return launch_kernel(mod, reinterpret_cast<const void*>(skinny_reduce_kernel<NMAT, OUT>),
                       &skinny_reduce_symbol<NMAT, OUT>,
                       dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, r, a.rows);
}

template <int NMAT, int OUT>
static hipError_t launch_decode_tile_mt(const DecTileArgs& a, int mt, const llk::ModuleFns* mod,
                                        hipStream_t s) {
  if (mt == 1) return launch_decode_tile_t<NMAT, OUT, 1, false>(a, mod, s);
  if (mt == 2) return launch_decode_tile_t<NMAT, OUT, 2, false>(a, mod, s);
  return launch_decode_tile_t<NMAT, OUT, 4, false>(a, mod, s);
}

// The row-major form exists for 64 and 128 rows (MT = 1, 2).
template <int NMAT, int OUT>
static hipError_t launch_decode_rowmajor_mt(const DecTileArgs& a, int mt,
                                            const llk::ModuleFns* mod, hipStream_t s) {
  if (mt == 1) return launch_decode_tile_t<NMAT, OUT, 1, true>(a, mod, s);
  if (mt == 2) return launch_decode_tile_t<NMAT, OUT, 2, true>(a, mod, s);
  return hipErrorInvalidValue;
}

}  // namespace llk_gfx950

// Rows of the partial buffer for M rows (whole 32-row MFMA groups).
static int skinny_rows(int M) { return (M + 31) / 32 * 32; }

// Threads per workgroup of the small-M kernel for (nmat, M, G), G = 32-column
// groups per workgroup.
int llk_skinny_threads(int nmat, int M, int G) {
  using namespace llk_gfx950;
  const int w = (G == 2 || G == 4) ? G : 1;
  if (nmat == 2) return M <= 32 ? skinny_threads_w<2, 1>(w) : skinny_threads_w<2, 2>(w);
  return M <= 32 ? skinny_threads_w<1, 1>(w) : skinny_threads_w<1, 2>(w);
}

size_t llk_skinny_workspace_bytes(int nmat, int M, int N_pad, int S) {
  if (S <= 1) return 0;
  return (size_t)S * nmat * skinny_rows(M) * N_pad * sizeof(float);
}

// Internal: called by the host dispatch layer.  mode 1 = SwiGLU (w0 = Wg,
// w1 = Wu), mode 0 = GEMM (w0 = B).  M <= 64.  G (1, 2, 4): 32-column
// groups per workgroup (the W of SkinnyCfg).  `ws` must hold llk_skinny_workspace_bytes(nmat, M,
// 128*NB, S) bytes when S > 1.
hipError_t llk_launch_skinny(int mode, const uint16_t* x, int64_t ldx, const void* w0,
                             const void* w1, void* y, int64_t ldy, int M, int N, int K, int KB,
                             int NB, int S, int G, void* ws, int out, bool xvec, bool yvec,
                             bool accumulate, const llk::ModuleFns* mod, hipStream_t s) {
  using namespace llk_gfx950;
  if (M < 1 || M > 64 || (G != 1 && G != 2 && G != 4)) return hipErrorInvalidValue;
  SkinnyArgs a;
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
  a.S = S < 1 ? 1 : S;
  a.kb_per_split = (KB + a.S - 1) / a.S;
  a.n_pad = NB * kPackN;
  a.yvec = yvec;
  a.accumulate = accumulate;
  a.part = static_cast<float*>(ws);
  if (accumulate && mode != 0) return hipErrorInvalidValue;
  // Every split must own at least one 64-k block (the dispatcher passes
  // S = ceil(KB / ceil(KB / S_requested))).
  if (a.S > 1 && (ws == nullptr || (int64_t)(a.S - 1) * a.kb_per_split >= KB))
    return hipErrorInvalidValue;
  const int mt = (M + 31) / 32;
#if !defined(LLK_CO_OP) || LLK_CO_OP == 1
  if (mode == 1)
    return mt == 1 ? launch_skinny_mt<2, 1>(a, G, out, xvec, mod, s)
                   : launch_skinny_mt<2, 2>(a, G, out, xvec, mod, s);
#endif
#if !defined(LLK_CO_OP) || LLK_CO_OP == 0
  if (mode == 0)
    return mt == 1 ? launch_skinny_mt<1, 1>(a, G, out, xvec, mod, s)
                   : launch_skinny_mt<1, 2>(a, G, out, xvec, mod, s);
#endif
  return hipErrorInvalidValue;
}

// Whether the decode tile kernel takes a shape: M <= 256, K a multiple of
// 64, X rows 16-byte aligned (ldx % 8 == 0 and a 16-byte aligned base, the
// caller's check), and the 32-bit buffer offsets: the workgroup's 64 MT rows
// of X plus the trailing steps, and one weight panel plus them.
bool llk_decode_tile_fits(int M, int64_t K, int64_t ldx) {
  if (M < 1 || M > 256 || K < 64 || K % 64 != 0 || ldx < K || ldx % 8 != 0) return false;
  const int64_t KB = K / 64, rows = 64 * (int64_t)llk_gfx950::dec_mt(M);
  return rows * ldx * 2 + (KB + 2) * 128 < ((int64_t)1 << 31) &&
         (KB + 2) * (int64_t)llk_gfx950::kBlockBytes < ((int64_t)1 << 31);
}

// Whether the row-major form takes a shape (beside llk_decode_tile_fits):
// at most 128 rows, each weight matrix bf16 [K, N] with 16-byte aligned rows
// of ldw >= N elements, and K + 128 rows of it within 32-bit offsets.
bool llk_decode_rowmajor_fits(int M, int64_t K, int64_t ldx, const void* w, int64_t ldw,
                              int64_t N) {
  return M <= 128 && llk_decode_tile_fits(M, K, ldx) && w != nullptr &&
         reinterpret_cast<uintptr_t>(w) % 16 == 0 && ldw % 8 == 0 && ldw >= N &&
         (K + 128) * ldw * 2 < ((int64_t)1 << 31);
}

// Internal: the decode tile kernel.  mode 1 = SwiGLU (w0 = Wg, w1 = Wu),
// mode 0 = GEMM (w0 = B); llk_decode_tile_fits(M, 64 * KB, ldx) must hold.
// S > 1 splits K over S workgroups of kbs = ceil(KB / S) blocks (every split
// non-empty: (S - 1) * kbs < KB) through `ws`, which holds
// llk_skinny_workspace_bytes(nmat, M, 128 * NB, S) bytes; accumulate (GEMM
// only) adds the existing y.
hipError_t llk_launch_decode_tile(int mode, const uint16_t* x, int64_t ldx, const void* w0,
                                  const void* w1, void* y, int64_t ldy, int M, int N, int KB,
                                  int NB, int S, void* ws, int out, bool yvec, bool accumulate,
                                  const llk::ModuleFns* mod, hipStream_t s) {
  using namespace llk_gfx950;
  if (!llk_decode_tile_fits(M, (int64_t)KB * 64, ldx) || NB < 1 || (accumulate && mode != 0))
    return hipErrorInvalidValue;
  DecTileArgs a{};
  a.x = x;
  a.w0 = static_cast<const uint8_t*>(w0);
  a.w1 = static_cast<const uint8_t*>(w1);
  a.y = y;
  a.part = static_cast<float*>(ws);
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.KB = KB;
  a.NB = NB;
  a.S = S < 1 ? 1 : S;
  a.kbs = (KB + a.S - 1) / a.S;
  a.n_pad = NB * kPackN;
  a.rows = skinny_rows(M);
  a.yvec = yvec;
  a.accumulate = accumulate;
  if (a.S > 1 && (ws == nullptr || (int64_t)(a.S - 1) * a.kbs >= KB)) return hipErrorInvalidValue;
  const int mt = dec_mt(M);
#if !defined(LLK_CO_OP) || LLK_CO_OP == 1
  if (mode == 1) {
    if (out == kOutBF16) return launch_decode_tile_mt<2, kOutBF16>(a, mt, mod, s);
    if (out == kOutF32) return launch_decode_tile_mt<2, kOutF32>(a, mt, mod, s);
  }
#endif
#if !defined(LLK_CO_OP) || LLK_CO_OP == 0
  if (mode == 0) {
    if (out == kOutBF16) return launch_decode_tile_mt<1, kOutBF16>(a, mt, mod, s);
    if (out == kOutF32) return launch_decode_tile_mt<1, kOutF32>(a, mt, mod, s);
    if (out == kOutF16) return launch_decode_tile_mt<1, kOutF16>(a, mt, mod, s);
  }
#endif
  return hipErrorInvalidValue;
}

// Internal: the decode tile kernel reading row-major weights (no packed
// payload): w0 / w1 are bf16 [K, N] with rows of ldw0 / ldw1 elements,
// llk_decode_rowmajor_fits must hold for each; otherwise as
// llk_launch_decode_tile (grid, k splits, workspace and results: the same
// MFMA operands in the same order, so the same bits as the packed form).
hipError_t llk_launch_decode_rowmajor(int mode, const uint16_t* x, int64_t ldx,
                                      const uint16_t* w0, int64_t ldw0, const uint16_t* w1,
                                      int64_t ldw1, void* y, int64_t ldy, int M, int N, int K,
                                      int S, void* ws, int out, bool yvec, bool accumulate,
                                      const llk::ModuleFns* mod, hipStream_t s) {
  using namespace llk_gfx950;
  if (N < 1 || !llk_decode_rowmajor_fits(M, K, ldx, w0, ldw0, N) ||
      (mode == 1 && !llk_decode_rowmajor_fits(M, K, ldx, w1, ldw1, N)) ||
      (accumulate && mode != 0))
    return hipErrorInvalidValue;
  DecTileArgs a{};
  a.x = x;
  a.w0 = reinterpret_cast<const uint8_t*>(w0);
  a.w1 = reinterpret_cast<const uint8_t*>(mode == 1 ? w1 : w0);
  a.ldw0 = ldw0;
  a.ldw1 = mode == 1 ? ldw1 : ldw0;
  a.y = y;
  a.part = static_cast<float*>(ws);
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.KB = K / 64;
  a.NB = (N + kPackN - 1) / kPackN;
  a.S = S < 1 ? 1 : S;
  a.kbs = (a.KB + a.S - 1) / a.S;
  a.n_pad = a.NB * kPackN;
  a.rows = skinny_rows(M);
  a.yvec = yvec;
  a.accumulate = accumulate;
  if (a.S > 1 && (ws == nullptr || (int64_t)(a.S - 1) * a.kbs >= a.KB)) return hipErrorInvalidValue;
  const int mt = dec_mt(M);
#if !defined(LLK_CO_OP) || LLK_CO_OP == 1
  if (mode == 1) {
    if (out == kOutBF16) return launch_decode_rowmajor_mt<2, kOutBF16>(a, mt, mod, s);
    if (out == kOutF32) return launch_decode_rowmajor_mt<2, kOutF32>(a, mt, mod, s);
  }
#endif
#if !defined(LLK_CO_OP) || LLK_CO_OP == 0
  if (mode == 0) {
    if (out == kOutBF16) return launch_decode_rowmajor_mt<1, kOutBF16>(a, mt, mod, s);
    if (out == kOutF32) return launch_decode_rowmajor_mt<1, kOutF32>(a, mt, mod, s);
    if (out == kOutF16) return launch_decode_rowmajor_mt<1, kOutF16>(a, mt, mod, s);
  }
#endif
  return hipErrorInvalidValue;
}
