// swiglu_decode.hip -- bandwidth-bound kernels for small M (decode).
//
// NMAT = 2: fused SwiGLU  Y = SiLU(X Wg) * (X Wu);   NMAT = 1: C = X W.
// For M <= 32 * MT rows the weights dominate the traffic (K*N bf16 per
// matrix, read once), so the kernel is an HBM stream over the packed
// payload: every wave load is one contiguous 1 KiB MFMA operand
// (v_mfma_f32_32x32x16_bf16 A operand); X (at most 64 rows) is tiny and
// served from L2.
//
// Grid: (4 * NB / G workgroups) x S k-splits.  A workgroup owns G adjacent
// 32-column groups (of one 128-column n-block) of every matrix with KS
// waves per group; each group's k range is divided among its KS waves, each
// streaming its part with UNROLL 64-k steps of loads in flight, and the G
// waves of a k part read neighbouring 1 KiB sub-blocks of the same 4 KiB
// together.  The waves' partial sums meet in LDS, in wave order (a fixed
// order, so results are deterministic).  With S == 1 the workgroup then
// applies the epilogue (FuseDoubleContraction.cpp:175-199 for SwiGLU) and
// stores Y.  With S > 1 it writes fp32 partials to a workspace and a second
// kernel adds the S partials in split order and applies the epilogue -- the
// kernel boundary orders the two, so no device-scope fences are needed.
#include "common.h"

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

// G: 32-column groups per workgroup (1, 2 or 4 of one 128-column n-block);
// KS: waves per group, each streaming a contiguous part of the k range.
// Wave w serves group w % G and k part w / G, so the G waves of a k part
// read neighbouring 1 KiB sub-blocks of the same 4 KiB (G = 4) at the same
// time.
template <int NMAT, int MT, int KS, int G, int OUT, bool XVEC, int UNROLL>
__global__ __launch_bounds__(KS * G * 64) void skinny_kernel(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) float red[];  // [KS][G][NMAT][MT][16][64]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gi = wave % G;
  const int kpart = wave / G;
  const int nwg = a.NB * 4 / G;  // workgroups per k split
  const int wg = blockIdx.x % nwg;
  const int split = blockIdx.x / nwg;
  const int grp = wg * G + gi;  // 32-column group of this wave
  const int nb = grp >> 2, n32 = grp & 3;

  // k range of this workgroup, then of this wave (contiguous chunks).
  const int kb0 = split * a.kb_per_split;
  const int kb1 = min(a.KB, kb0 + a.kb_per_split);
  const int span = kb1 > kb0 ? kb1 - kb0 : 0;
  const int per_wave = (span + KS - 1) / KS;
  const int wb0 = kb0 + kpart * per_wave;
  const int wb1 = min(kb1, wb0 + per_wave);

  f32x16 acc[NMAT][MT];
#pragma unroll
  for (int p = 0; p < NMAT; ++p)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[p][t][r] = 0.0f;

  // Sub-block (kq, n32) of block (nb, kb): + kb*16K + (kq*4 + n32)*1K.
  const size_t panel = (size_t)nb * a.KB * kBlockBytes + n32 * kSubBytes + lane * 16;
  const uint8_t* wbase[2] = {a.w0 + panel, (NMAT == 2 ? a.w1 : a.w0) + panel};

  int kb = wb0;
  for (; kb + UNROLL <= wb1; kb += UNROLL) {
    u32x4 w[UNROLL][NMAT][4];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int p = 0; p < NMAT; ++p)
#pragma unroll
        for (int kq = 0; kq < 4; ++kq)
          w[u][p][kq] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
              wbase[p] + (size_t)(kb + u) * kBlockBytes + kq * 4 * kSubBytes));
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      bf16x8 xf[4][MT];
      load_x_frags<MT, XVEC>(a, kb + u, lane, xf);
#pragma unroll
      for (int kq = 0; kq < 4; ++kq)
#pragma unroll
        for (int p = 0; p < NMAT; ++p) {
          const bf16x8 wop = *reinterpret_cast<const bf16x8*>(&w[u][p][kq]);
#pragma unroll
          for (int t = 0; t < MT; ++t) acc[p][t] = mfma32(wop, xf[kq][t], acc[p][t]);
        }
    }
  }
  for (; kb < wb1; ++kb) {  // remainder steps
    bf16x8 xf[4][MT];
    load_x_frags<MT, XVEC>(a, kb, lane, xf);
#pragma unroll
    for (int kq = 0; kq < 4; ++kq)
#pragma unroll
      for (int p = 0; p < NMAT; ++p) {
        const u32x4 wv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
            wbase[p] + (size_t)kb * kBlockBytes + kq * 4 * kSubBytes));
        const bf16x8 wop = *reinterpret_cast<const bf16x8*>(&wv);
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[p][t] = mfma32(wop, xf[kq][t], acc[p][t]);
      }
  }

  // ---- reduce the KS waves' partial sums in LDS, in wave order ----------
  constexpr bool kLds = KS * G > 1;
  if (kLds) {
#pragma unroll
    for (int p = 0; p < NMAT; ++p)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          red[(((wave * NMAT + p) * MT + t) * 16 + r) * 64 + lane] = acc[p][t][r];
    __syncthreads();
  }

  // Thread e handles (group ge, t, g, ln): rows m = t*32 + ln%32 and the 4
  // consecutive columns n = 8g + 4*(ln/32) + 0..3 (accumulator r = 4g+q) of
  // the workgroup's group ge.  Without LDS (one wave) e = lane + 64 j, so
  // the values are this lane's own accumulators.
  for (int e = threadIdx.x; e < G * MT * 4 * 64; e += KS * G * 64) {
    const int ln = e & 63;
    const int g = (e >> 6) & 3;
    const int t = (e >> 8) % MT;
    const int ge = e / (MT * 4 * 64);
    float sum[NMAT][4];
#pragma unroll
    for (int p = 0; p < NMAT; ++p)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float s = 0.0f;
        if (kLds) {
          for (int w2 = 0; w2 < KS; ++w2)
            s += red[((((w2 * G + ge) * NMAT + p) * MT + t) * 16 + 4 * g + q) * 64 + ln];
        } else {
          s = acc[p][t][4 * g + q];
        }
        sum[p][q] = s;
      }
    const int eg = wg * G + ge;
    const int m = t * 32 + (ln & 31);
    const int n = (eg >> 2) * kPackN + (eg & 3) * 32 + 8 * g + 4 * (ln >> 5);
    if (a.S > 1) {
      if (n < a.n_pad) {
#pragma unroll
        for (int p = 0; p < NMAT; ++p) {
          float* dst = a.part + (((size_t)split * NMAT + p) * (MT * 32) + m) * a.n_pad + n;
          *reinterpret_cast<f32x4*>(dst) = f32x4{sum[p][0], sum[p][1], sum[p][2], sum[p][3]};
        }
      }
    } else {
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        v[q] = (NMAT == 2) ? swiglu_act(sum[0][q], sum[1][q]) : sum[0][q];
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
  for (int q = 0; q < 4; ++q) v[q] = (NMAT == 2) ? swiglu_act(s[0][q], s[1][q]) : s[0][q];
  store4<OUT>(a.y, a.ldy, a.M, a.N, m, n, v, a.yvec);
}

template <int NMAT, int MT, int KS, int G, int OUT, bool XVEC>
static hipError_t launch_skinny_t(const SkinnyArgs& a, hipStream_t s) {
  auto fn = skinny_kernel<NMAT, MT, KS, G, OUT, XVEC, 2>;
  const size_t lds = KS * G > 1 ? (size_t)KS * G * NMAT * MT * 16 * 64 * sizeof(float) : 0;
  static bool attr_set = false;  // per instantiation; benign race (idempotent)
  if (!attr_set && lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  attr_set = true;
  hipLaunchKernelGGL(fn, dim3(a.NB * 4 / G * a.S), dim3(KS * G * 64), lds, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.S == 1) return e;
  const int64_t threads = (int64_t)a.M * (a.n_pad / 4);
  hipLaunchKernelGGL((skinny_reduce_kernel<NMAT, OUT>), dim3((unsigned)((threads + 255) / 256)),
                     dim3(256), 0, s, a, MT * 32);
  return hipGetLastError();
}

// Waves per group: KS * G <= 16 (1024 threads) and the LDS reduction buffer
// (KS * G * NMAT * MT * 4 KiB) at most 128 KiB.
template <int NMAT, int MT, int G>
constexpr int skinny_ks() {
  return G == 1 ? ((NMAT * MT <= 2) ? 8 : 4) : (32 / (G * NMAT * MT) < 16 / G ? 32 / (G * NMAT * MT) : 16 / G);
}

template <int NMAT, int MT, int G, int OUT>
static hipError_t launch_skinny_o(const SkinnyArgs& a, bool xvec, hipStream_t s) {
  constexpr int KS = skinny_ks<NMAT, MT, G>();
  return xvec ? launch_skinny_t<NMAT, MT, KS, G, OUT, true>(a, s)
              : launch_skinny_t<NMAT, MT, KS, G, OUT, false>(a, s);
}

// fp16 output exists for the GEMM (NMAT 1) only.
template <int NMAT, int MT, int G>
static hipError_t launch_skinny_g(const SkinnyArgs& a, int out, bool xvec, hipStream_t s) {
  if (out == kOutBF16) return launch_skinny_o<NMAT, MT, G, kOutBF16>(a, xvec, s);
  if (out == kOutF32) return launch_skinny_o<NMAT, MT, G, kOutF32>(a, xvec, s);
  if constexpr (NMAT == 1) {
    if (out == kOutF16) return launch_skinny_o<NMAT, MT, G, kOutF16>(a, xvec, s);
  }
  return hipErrorInvalidValue;
}

template <int NMAT, int MT>
static hipError_t launch_skinny_mt(const SkinnyArgs& a, int G, int out, bool xvec,
                                   hipStream_t s) {
  if (G == 4) return launch_skinny_g<NMAT, MT, 4>(a, out, xvec, s);
  if (G == 2) return launch_skinny_g<NMAT, MT, 2>(a, out, xvec, s);
  return launch_skinny_g<NMAT, MT, 1>(a, out, xvec, s);
}

}  // namespace llk_gfx950

// Rows of the partial buffer for M rows (whole 32-row MFMA groups).
static int skinny_rows(int M) { return (M + 31) / 32 * 32; }

// Threads per workgroup of the small-M kernel for (nmat, M, G).
int llk_skinny_threads(int nmat, int M, int G) {
  using namespace llk_gfx950;
  const bool mt1 = M <= 32;
  const int g = (G == 2 || G == 4) ? G : 1;
  int ks;
  if (nmat == 2)
    ks = mt1 ? (g == 1 ? skinny_ks<2, 1, 1>() : g == 2 ? skinny_ks<2, 1, 2>() : skinny_ks<2, 1, 4>())
             : (g == 1 ? skinny_ks<2, 2, 1>() : g == 2 ? skinny_ks<2, 2, 2>() : skinny_ks<2, 2, 4>());
  else
    ks = mt1 ? (g == 1 ? skinny_ks<1, 1, 1>() : g == 2 ? skinny_ks<1, 1, 2>() : skinny_ks<1, 1, 4>())
             : (g == 1 ? skinny_ks<1, 2, 1>() : g == 2 ? skinny_ks<1, 2, 2>() : skinny_ks<1, 2, 4>());
  return ks * g * 64;
}

size_t llk_skinny_workspace_bytes(int nmat, int M, int N_pad, int S) {
  if (S <= 1) return 0;
  return (size_t)S * nmat * skinny_rows(M) * N_pad * sizeof(float);
}

// Internal: called by the host dispatch layer.  mode 1 = SwiGLU (w0 = Wg,
// w1 = Wu), mode 0 = GEMM (w0 = B).  M <= 64.  G (1, 2, 4): 32-column
// groups per workgroup.  `ws` must hold llk_skinny_workspace_bytes(nmat, M,
// 128*NB, S) bytes when S > 1.
hipError_t llk_launch_skinny(int mode, const uint16_t* x, int64_t ldx, const void* w0,
                             const void* w1, void* y, int64_t ldy, int M, int N, int K, int KB,
                             int NB, int S, int G, void* ws, int out, bool xvec, bool yvec,
                             hipStream_t s) {
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
  a.part = static_cast<float*>(ws);
  if (a.S > 1 && ws == nullptr) return hipErrorInvalidValue;
  const int mt = (M + 31) / 32;
  if (mode == 1)
    return mt == 1 ? launch_skinny_mt<2, 1>(a, G, out, xvec, s)
                   : launch_skinny_mt<2, 2>(a, G, out, xvec, s);
  return mt == 1 ? launch_skinny_mt<1, 1>(a, G, out, xvec, s)
                 : launch_skinny_mt<1, 2>(a, G, out, xvec, s);
}
