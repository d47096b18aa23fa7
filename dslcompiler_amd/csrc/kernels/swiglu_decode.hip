// swiglu_decode.hip -- bandwidth-bound fused SwiGLU for small M (decode).
//
// Y = SiLU(X Wg) * (X Wu) for M <= 16 * MT rows.  The weights dominate the
// traffic (2*K*N bf16 read once), so the kernel is an HBM stream over the
// packed payload: every wave load is one contiguous 1 KiB MFMA operand.
// X (at most 64 rows) is tiny and served from L2.
//
// Grid: (NB n-blocks of 128) x S k-splits.  Workgroup = 4 waves; wave w owns
// n16 groups {2w, 2w+1} of the block for both Wg and Wu, so a lane's gate and
// up partial sums describe the same (m, n) pairs.  Each k step (64 k) a wave
// issues 8 independent 1 KiB loads per step, UNROLL steps at a time.
//
// With S > 1 each workgroup writes fp32 partial sums to a workspace; the last
// workgroup of an n-block to finish (device-scope counter) adds the S
// partials in split order -- a fixed order, so results are deterministic --
// and applies the SiLU(g)*u epilogue (FuseDoubleContraction.cpp:175-199).
// It then resets the counter, so the workspace needs zeroing only once.
#include "common.h"

namespace llk_gfx950 {

struct DecodeArgs {
  const uint16_t* x;  // [M, K]
  const uint8_t* wg;  // packed
  const uint8_t* wu;  // packed
  void* y;            // [M, N]
  float* part;        // [S][2][MT*16][N_pad] fp32 partials (S > 1)
  unsigned* counter;  // [NB] arrival counters (S > 1), zero between calls
  int64_t ldx, ldy;
  int M, N, K, KB, NB, S, kb_per_split, n_pad;
};

constexpr int kDecThreads = 256;

template <int MT, bool OUT_BF16, bool XVEC>
__device__ __forceinline__ void load_x_frag(const DecodeArgs& a, int kb, int kh, int lane,
                                            bf16x8 (&xf)[MT]) {
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    int m = t * 16 + (lane & 15);
    int kk = kb * 64 + kh * 32 + (lane >> 4) * 8;
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
    xf[t] = *reinterpret_cast<bf16x8*>(&v);
  }
}

template <bool OUT_BF16>
__device__ __forceinline__ void store_y4(const DecodeArgs& a, int m, int n, const float (&v)[4],
                                         bool yvec) {
  if (m >= a.M || n >= a.N) return;
  if (OUT_BF16) {
    uint16_t* dst = reinterpret_cast<uint16_t*>(a.y) + (size_t)m * a.ldy + n;
    if (yvec && n + 4 <= a.N) {
      u16x4 h = {f32_to_bf16_rne(v[0]), f32_to_bf16_rne(v[1]), f32_to_bf16_rne(v[2]),
                 f32_to_bf16_rne(v[3])};
      *reinterpret_cast<u16x4*>(dst) = h;
    } else {
      for (int r = 0; r < 4; ++r)
        if (n + r < a.N) dst[r] = f32_to_bf16_rne(v[r]);
    }
  } else {
    float* dst = reinterpret_cast<float*>(a.y) + (size_t)m * a.ldy + n;
    if (yvec && n + 4 <= a.N) {
      *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
    } else {
      for (int r = 0; r < 4; ++r)
        if (n + r < a.N) dst[r] = v[r];
    }
  }
}

template <int MT, bool OUT_BF16, bool XVEC, bool YVEC, int UNROLL>
__global__ __launch_bounds__(kDecThreads) void swiglu_decode_kernel(DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nb = blockIdx.x % a.NB;
  const int split = blockIdx.x / a.NB;
  const int kb_begin = split * a.kb_per_split;
  const int kb_end = min(a.KB, kb_begin + a.kb_per_split);

  // acc[mat][g][t]: mat 0 gate / 1 up, g = n16 group 2*wave+g, t = m16 group
  f32x4 acc[2][2][MT];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[p][g][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const size_t col_base = (size_t)nb * a.KB * kBlockBytes;
  const uint8_t* wbase[2] = {a.wg + col_base, a.wu + col_base};

  int kb = kb_begin;
  for (; kb + UNROLL <= kb_end; kb += UNROLL) {
    u32x4 w[UNROLL][2][2][2];  // [step][mat][kh][g]
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int g = 0; g < 2; ++g) {
            const uint8_t* src = wbase[p] + (size_t)(kb + u) * kBlockBytes +
                                 (kh * 8 + wave * 2 + g) * kSubBytes + lane * 16;
            w[u][p][kh][g] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
          }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        bf16x8 xf[MT];
        load_x_frag<MT, OUT_BF16, XVEC>(a, kb + u, kh, lane, xf);
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
          for (int g = 0; g < 2; ++g) {
            bf16x8 wop = *reinterpret_cast<bf16x8*>(&w[u][p][kh][g]);
#pragma unroll
            for (int t = 0; t < MT; ++t) acc[p][g][t] = mfma16(wop, xf[t], acc[p][g][t]);
          }
      }
  }
  for (; kb < kb_end; ++kb) {  // remainder steps
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      bf16x8 xf[MT];
      load_x_frag<MT, OUT_BF16, XVEC>(a, kb, kh, lane, xf);
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const uint8_t* src = wbase[p] + (size_t)kb * kBlockBytes +
                               (kh * 8 + wave * 2 + g) * kSubBytes + lane * 16;
          u32x4 wv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
          bf16x8 wop = *reinterpret_cast<bf16x8*>(&wv);
#pragma unroll
          for (int t = 0; t < MT; ++t) acc[p][g][t] = mfma16(wop, xf[t], acc[p][g][t]);
        }
    }
  }

  // Lane holds n = nb*128 + (2*wave+g)*16 + 4*(lane/16) + r, m = t*16 + lane%16.
  const int nq = 4 * (lane >> 4);
  const int mr = lane & 15;

  if (a.S == 1) {
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = swiglu_act(acc[0][g][t][r], acc[1][g][t][r]);
        store_y4<OUT_BF16>(a, t * 16 + mr, nb * 128 + (2 * wave + g) * 16 + nq, v, YVEC);
      }
    return;
  }

  // ---- split-K: publish partials, last arrival reduces in split order
  constexpr int kRows = MT * 16;
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int m = t * 16 + mr;
        if (m >= a.M) continue;
        const int n = nb * 128 + (2 * wave + g) * 16 + nq;
        float* dst = a.part + (((size_t)split * 2 + p) * kRows + m) * a.n_pad + n;
        *reinterpret_cast<f32x4*>(dst) = acc[p][g][t];
      }
  __threadfence();
  __syncthreads();
  __shared__ unsigned last;
  if (threadIdx.x == 0) {
    unsigned prev = atomicAdd(&a.counter[nb], 1u);
    last = (prev == (unsigned)(a.S - 1)) ? 1u : 0u;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();

  // 128 n x kRows m of this block: thread handles 4 consecutive n of a row.
  for (int e = threadIdx.x; e < kRows * 32; e += kDecThreads) {
    const int m = e / 32;
    const int n = nb * 128 + (e % 32) * 4;
    if (m >= a.M) continue;
    f32x4 gs = {0.f, 0.f, 0.f, 0.f}, us = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < a.S; ++s) {
      const float* pg = a.part + (((size_t)s * 2 + 0) * kRows + m) * a.n_pad + n;
      const float* pu = a.part + (((size_t)s * 2 + 1) * kRows + m) * a.n_pad + n;
      gs += *reinterpret_cast<const f32x4*>(pg);
      us += *reinterpret_cast<const f32x4*>(pu);
    }
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = swiglu_act(gs[r], us[r]);
    store_y4<OUT_BF16>(a, m, n, v, YVEC);
  }
  if (threadIdx.x == 0) a.counter[nb] = 0u;
}

template <int MT, bool OUT_BF16, bool XVEC, bool YVEC>
static hipError_t launch_dec_t(const DecodeArgs& a, hipStream_t s) {
  dim3 grid(a.NB * a.S), block(kDecThreads);
  hipLaunchKernelGGL((swiglu_decode_kernel<MT, OUT_BF16, XVEC, YVEC, 2>), grid, block, 0, s, a);
  return hipGetLastError();
}

template <int MT>
static hipError_t launch_dec_mt(const DecodeArgs& a, bool out_bf16, bool xvec, bool yvec,
                                hipStream_t s) {
  if (out_bf16) {
    if (xvec) return yvec ? launch_dec_t<MT, true, true, true>(a, s) : launch_dec_t<MT, true, true, false>(a, s);
    return yvec ? launch_dec_t<MT, true, false, true>(a, s) : launch_dec_t<MT, true, false, false>(a, s);
  }
  if (xvec) return yvec ? launch_dec_t<MT, false, true, true>(a, s) : launch_dec_t<MT, false, true, false>(a, s);
  return yvec ? launch_dec_t<MT, false, false, true>(a, s) : launch_dec_t<MT, false, false, false>(a, s);
}

}  // namespace llk_gfx950

// Split-K workspace layout: a fixed region of kDecodeMaxCounters arrival
// counters at offset 0 (zero before first use; every launch leaves the
// counters it used at zero), then the fp32 partials.  The counters never
// move, so partials of an earlier, larger launch can never land on them.
constexpr int kDecodeMaxCounters = 16384;
constexpr size_t kDecodeCounterBytes = kDecodeMaxCounters * sizeof(unsigned);

int llk_decode_max_counters() { return kDecodeMaxCounters; }

size_t llk_decode_workspace_bytes(int M, int N_pad, int NB, int S) {
  if (S <= 1) return 0;
  (void)NB;
  int mt = (M + 15) / 16;
  size_t part = (size_t)S * 2 * (mt * 16) * N_pad * sizeof(float);
  return kDecodeCounterBytes + part;
}

// Internal: called by the host dispatch layer.  `ws` must hold
// llk_decode_workspace_bytes(M, N_pad, NB, S) bytes with its counter region
// zeroed, and NB <= kDecodeMaxCounters when S > 1.
hipError_t llk_launch_decode(const uint16_t* x, int64_t ldx, const void* wg, const void* wu,
                             void* y, int64_t ldy, int M, int N, int K, int KB, int NB, int S,
                             void* ws, bool out_bf16, bool xvec, bool yvec, hipStream_t s) {
  using namespace llk_gfx950;
  DecodeArgs a;
  a.x = x;
  a.wg = static_cast<const uint8_t*>(wg);
  a.wu = static_cast<const uint8_t*>(wu);
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
  a.part = nullptr;
  a.counter = nullptr;
  if (a.S > 1) {
    if (NB > kDecodeMaxCounters || ws == nullptr) return hipErrorInvalidValue;
    a.counter = static_cast<unsigned*>(ws);
    a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kDecodeCounterBytes);
  }
  const int mt = (M + 15) / 16;
  switch (mt) {
    case 1: return launch_dec_mt<1>(a, out_bf16, xvec, yvec, s);
    case 2: return launch_dec_mt<2>(a, out_bf16, xvec, yvec, s);
    case 3: return launch_dec_mt<3>(a, out_bf16, xvec, yvec, s);
    case 4: return launch_dec_mt<4>(a, out_bf16, xvec, yvec, s);
    default: return hipErrorInvalidValue;
  }
}
