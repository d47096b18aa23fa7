// oracle.cpp -- CPU restatement of skg7on/DSLCompiler's fused-SwiGLU /
// micro.mma hot path.
//
// TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
// calls this file.  It is used by tests/, by __graft_entry__.smoke() and by
// bench.py's cpu_baseline leg, always as the checker (or the timed CPU
// baseline), never as the thing that is measured or shipped.
//
// Every function names the reference file:line it restates.  Pinning status
// (what checks each function against something other than itself):
//   orc_bf16_to_f32 / orc_f32_to_bf16_rne / orc_f32_to_bf16_testhelper
//       pinned: reference round-trip values, IEEE special cases, and the
//       reference's own helper compiled from source (oracle/_ref).
//   orc_swiglu_fused                pinned: reference known-answer values,
//       exact small-integer cases, reference fp32/fp64 routines compiled from
//       source (oracle/_ref), fp64 closed form.
//   orc_swiglu_fp64                 pinned: reference fp64 routine (oracle/_ref)
//       and known-answer values.
//   orc_gemm / orc_gemm_init        pinned: exact small-integer cases, brute
//       force fp64, identity / permutation matrices; with an initial
//       accumulator, the integer closed form C0 + A B.
//   orc_gemm_avx2_mt                pinned against orc_gemm_init (bit-equal).
//   orc_mlp                         pinned through its two parts above.
//   orc_classify_m, tiling helpers  pinned: reference test tables.
//   orc_kernel_key_hash             pinned: reference header compiled from
//       source (oracle/_ref).
//   orc_pack_weight_matrix          pinned: byte-identity with the row-major
//       input when K % BK == 0 and the reference metadata formulas.
//   orc_swiglu_avx2_mt              pinned against orc_swiglu_fused.
//   The exact bit pattern of the reference's JIT'd AVX2 output (its vector
//   reduction order and LLVM's expf lowering) is parity unpinned: it needs an
//   MLIR/LLVM 22 build that does not exist here.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include <immintrin.h>

extern "C" {

// ---------------------------------------------------------------------------
// bf16 conversions
// ---------------------------------------------------------------------------

// bf16 -> f32 is a 16-bit left shift (swiglu_reference.cpp:19-24).
float orc_bf16_to_f32(uint16_t h) {
  uint32_t bits = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// f32 -> bf16 as `arith.truncf` lowers it (FuseDoubleContraction.cpp:197,
// LLKToLinalg.cpp:149): IEEE round-to-nearest-even; NaN stays NaN (quiet).
uint16_t orc_f32_to_bf16_rne(float f) {
  uint32_t bits;
  std::memcpy(&bits, &f, 4);
  if ((bits & 0x7fffffffu) > 0x7f800000u)  // NaN: keep sign, force quiet bit
    return static_cast<uint16_t>((bits >> 16) | 0x0040u);
  uint32_t lsb = (bits >> 16) & 1u;
  bits += 0x7fffu + lsb;
  return static_cast<uint16_t>(bits >> 16);
}

// The reference tests' own input-quantisation helper
// (swiglu_reference.cpp:26-32, swiglu_vector_avx2.cpp:80-86,
// swiglu_scalar.cpp:77-83, vector_vs_scalar.cpp:28-34):
// bits += 0x8000 + lsb, then truncate.  This is NOT round-to-nearest-even
// (a tie with an even lsb rounds up, and 0x7fff with an odd lsb rounds up);
// it is restated so the reference tests' inputs can be reproduced exactly.
uint16_t orc_f32_to_bf16_testhelper(float f) {
  uint32_t bits;
  std::memcpy(&bits, &f, 4);
  bits += 0x8000u + ((bits >> 16) & 1u);
  return static_cast<uint16_t>(bits >> 16);
}

void orc_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(in[i]);
}
void orc_f32_to_bf16_rne_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16_rne(in[i]);
}

// ---------------------------------------------------------------------------
// SwiGLU epilogue (FuseDoubleContraction.cpp:175-199):
//   neg = -g; e = exp(neg); den = 1 + e; sig = 1 / den; silu = g * sig;
//   r = silu * u.          `math.exp` is the exact libm exp
// (MathApproximation.cpp:74-83 maps strict / triton_fast to math.exp; the
// fused path always emits math::ExpOp directly, :190).
// ---------------------------------------------------------------------------
static inline float swiglu_epilogue(float g, float u) {
  float neg = -g;
  float e = std::exp(neg);
  float den = 1.0f + e;
  float sig = 1.0f / den;
  float silu = g * sig;
  return silu * u;
}

float orc_swiglu_epilogue(float g, float u) { return swiglu_epilogue(g, u); }

// ---------------------------------------------------------------------------
// Fused SwiGLU, the canonical semantics (FuseDoubleContraction.cpp:119-199):
// fp32 accumulators filled with 0 (:119-135); per reduction step
// g += f32(x)*f32(wg), u += f32(x)*f32(wu) (:155-173); epilogue as above;
// `truncf` to bf16.  Reduction order here is sequential in k.  Since a
// bf16*bf16 product is exact in fp32, mul+add equals fma bit for bit.
//
// x: [M,K] with row stride ldx; wg/wu: [K,N] with row stride ldw;
// y_f32 (optional): pre-truncf value, row stride ldy;
// y_bf16 (optional): truncf'd result, row stride ldy.
// ---------------------------------------------------------------------------
void orc_swiglu_fused(const uint16_t* x, int64_t ldx, const uint16_t* wg,
                      const uint16_t* wu, int64_t ldw, int64_t M, int64_t N,
                      int64_t K, float* y_f32, uint16_t* y_bf16, int64_t ldy) {
  std::vector<float> gacc(static_cast<size_t>(N)), uacc(static_cast<size_t>(N));
  std::vector<float> xr(static_cast<size_t>(K));
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t k = 0; k < K; ++k) xr[k] = orc_bf16_to_f32(x[m * ldx + k]);
    std::fill(gacc.begin(), gacc.end(), 0.0f);
    std::fill(uacc.begin(), uacc.end(), 0.0f);
    for (int64_t k = 0; k < K; ++k) {
      const float xv = xr[k];
      const uint16_t* gr = wg + k * ldw;
      const uint16_t* ur = wu + k * ldw;
      for (int64_t n = 0; n < N; ++n) {
        gacc[n] = gacc[n] + xv * orc_bf16_to_f32(gr[n]);
        uacc[n] = uacc[n] + xv * orc_bf16_to_f32(ur[n]);
      }
    }
    for (int64_t n = 0; n < N; ++n) {
      float r = swiglu_epilogue(gacc[n], uacc[n]);
      if (y_f32) y_f32[m * ldy + n] = r;
      if (y_bf16) y_bf16[m * ldy + n] = orc_f32_to_bf16_rne(r);
    }
  }
}

// Same contraction without the epilogue: writes the fp32 gate and up sums.
void orc_swiglu_accumulators(const uint16_t* x, int64_t ldx, const uint16_t* wg,
                             const uint16_t* wu, int64_t ldw, int64_t M,
                             int64_t N, int64_t K, float* gate, float* up) {
  for (int64_t m = 0; m < M; ++m) {
    float* g = gate + m * N;
    float* u = up + m * N;
    for (int64_t n = 0; n < N; ++n) g[n] = u[n] = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float xv = orc_bf16_to_f32(x[m * ldx + k]);
      for (int64_t n = 0; n < N; ++n) {
        g[n] = g[n] + xv * orc_bf16_to_f32(wg[k * ldw + n]);
        u[n] = u[n] + xv * orc_bf16_to_f32(wu[k * ldw + n]);
      }
    }
  }
}

// fp64 closed form (swiglu_reference.cpp:77-99, edge_cases.cpp:18-40):
// gate/up summed in double, silu = g / (1 + exp(-g)), y = silu * up.
void orc_swiglu_fp64(const double* x, const double* wg, const double* wu,
                     double* y, int64_t M, int64_t N, int64_t K) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      double sg = 0.0, su = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        sg += x[m * K + k] * wg[k * N + n];
        su += x[m * K + k] * wu[k * N + n];
      }
      y[m * N + n] = sg / (1.0 + std::exp(-sg)) * su;
    }
}

// ---------------------------------------------------------------------------
// micro.mma / matmul semantics.  The micro.mma contract is
// acc[M,N] += lhs[M,K] * rhs[K,N] with bf16 inputs and an f32 accumulator
// (MicroOps.td:196-222, MicroOps.cpp:246-291).  llk.matmul carries an
// accumulator_type (LLKOps.td:210-255); with accumulator f32 the sums are
// fp32 and the result is cast once to the result type (f32: as is; bf16:
// truncf RNE).  Sequential-k order.
// a: [M,K] stride lda; b: [K,N] stride ldb.
// ---------------------------------------------------------------------------
void orc_gemm_init(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                   int64_t M, int64_t N, int64_t K, const float* c_init,
                   int64_t ldi, float* c_f32, uint16_t* c_bf16, int64_t ldc);

void orc_gemm(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
              int64_t M, int64_t N, int64_t K, float* c_f32, uint16_t* c_bf16,
              int64_t ldc) {
  orc_gemm_init(a, lda, b, ldb, M, N, K, nullptr, 0, c_f32, c_bf16, ldc);
}

// micro.mma with a non-zero accumulator: acc[M,N] += lhs * rhs
// (MicroOps.td:196-222; linalg.matmul accumulates into its `outs` operand,
// the init of llk.matmul's outs(init), LLKOps.td:210-255).  The fp32
// accumulator starts at c_init (row stride ldi; NULL = 0, as the fused
// path's zero-filled accumulators, FuseDoubleContraction.cpp:119-135) and
// takes the products in k order; the result is cast once to the output type.
void orc_gemm_init(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                   int64_t M, int64_t N, int64_t K, const float* c_init,
                   int64_t ldi, float* c_f32, uint16_t* c_bf16, int64_t ldc) {
  std::vector<float> acc(static_cast<size_t>(N));
  for (int64_t m = 0; m < M; ++m) {
    if (c_init)
      std::copy(c_init + m * ldi, c_init + m * ldi + N, acc.begin());
    else
      std::fill(acc.begin(), acc.end(), 0.0f);
    for (int64_t k = 0; k < K; ++k) {
      const float av = orc_bf16_to_f32(a[m * lda + k]);
      const uint16_t* br = b + k * ldb;
      for (int64_t n = 0; n < N; ++n) acc[n] = acc[n] + av * orc_bf16_to_f32(br[n]);
    }
    for (int64_t n = 0; n < N; ++n) {
      if (c_f32) c_f32[m * ldc + n] = acc[n];
      if (c_bf16) c_bf16[m * ldc + n] = orc_f32_to_bf16_rne(acc[n]);
    }
  }
}

// Brute-force fp64 matmul of bf16 inputs (the "closed form" check for gemm).
void orc_gemm_fp64(const uint16_t* a, const uint16_t* b, double* c, int64_t M,
                   int64_t N, int64_t K) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      double s = 0.0;
      for (int64_t k = 0; k < K; ++k)
        s += static_cast<double>(orc_bf16_to_f32(a[m * K + k])) *
             static_cast<double>(orc_bf16_to_f32(b[k * N + n]));
      c[m * N + n] = s;
    }
}

// Full MLP block: Y = bf16(SiLU(X Wg) * (X Wu)) (fused semantics above),
// then Z = bf16(Y Wd) with fp32 accumulation.  Wd is [N, K] row-major.
void orc_mlp(const uint16_t* x, const uint16_t* wg, const uint16_t* wu,
             const uint16_t* wd, int64_t M, int64_t N, int64_t K,
             uint16_t* y_bf16, uint16_t* z_bf16) {
  orc_swiglu_fused(x, K, wg, wu, N, M, N, K, nullptr, y_bf16, N);
  orc_gemm(y_bf16, N, wd, K, M, K, N, nullptr, z_bf16, K);
}

// ---------------------------------------------------------------------------
// Integer metadata
// ---------------------------------------------------------------------------

// classifyM (ScheduleLoader.cpp:19-29, = ShapeSpecialization.cpp:38-48):
// 1 -> 0, <=4 -> 1, <=16 -> 2, <=64 -> 3, else 4.  M <= 0 lands in bucket 1.
int orc_classify_m(int64_t M) {
  if (M == 1) return 0;
  if (M <= 4) return 1;
  if (M <= 16) return 2;
  if (M <= 64) return 3;
  return 4;
}

// TilingUtils.h:28-50.
int64_t orc_num_tiles(int64_t dim, int64_t tile) {
  if (tile == 0) return 1;
  return (dim + tile - 1) / tile;
}
int64_t orc_tile_size(int64_t dim, int64_t tile, int64_t idx) {
  int64_t start = idx * tile;
  if (start >= dim) return 0;
  int64_t rem = dim - start;
  return rem < tile ? rem : tile;
}
int64_t orc_num_inner_tiles(int64_t outer, int64_t inner) {
  if (inner == 0) return 1;
  return (outer + inner - 1) / inner;
}

// KernelKey::hash (KernelKey.h:60-86): splitmix64 finaliser over the twelve
// fields in declaration order, seed 0x9ae16a3b2f90404f.  Byte-typed fields are
// fed as their unsigned byte value; int64 fields reinterpret to uint64.
static inline uint64_t key_mix(uint64_t x) {
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
  return x ^ (x >> 31);
}
uint64_t orc_kernel_key_hash(uint8_t op, uint8_t in_t, uint8_t out_t,
                             int64_t m_bucket, int64_t n, int64_t k,
                             uint8_t layout, uint8_t isa, uint8_t math,
                             uint16_t threads, uint64_t compiler_version,
                             uint64_t schedule_version) {
  uint64_t h = 0x9ae16a3b2f90404fULL;
  const uint64_t fields[12] = {op,
                               in_t,
                               out_t,
                               static_cast<uint64_t>(m_bucket),
                               static_cast<uint64_t>(n),
                               static_cast<uint64_t>(k),
                               layout,
                               isa,
                               math,
                               threads,
                               compiler_version,
                               schedule_version};
  for (uint64_t f : fields) h = key_mix(h ^ f);
  return h;
}

// packWeightMatrix metadata (PackedWeights.cpp:5-15): N = dim1, K_blocks =
// ceil(K/BK), block_size = BK*N*2 bytes, dtype BF16 (0).
// out = {K_blocks, N, block_size, BK, dtype}.
void orc_pack_weight_meta(int64_t K, int64_t N, int64_t BK, int64_t* out) {
  out[0] = (K + BK - 1) / BK;
  out[1] = N;
  out[2] = BK * N * 2;
  out[3] = BK;
  out[4] = 0;
}

// packWeightMatrix payload (PackedWeights.cpp:17-31): buffer
// [K_blocks][BK][N] of bf16, zero-filled, each row k copied from
// W + k*stride0.  `out` must hold K_blocks*BK*N elements.
void orc_pack_weight_matrix(const uint16_t* w, int64_t K, int64_t N,
                            int64_t stride0, int64_t BK, uint16_t* out) {
  int64_t kb_count = (K + BK - 1) / BK;
  std::memset(out, 0, static_cast<size_t>(kb_count * BK * N) * 2);
  for (int64_t kb = 0; kb < kb_count; ++kb) {
    int64_t k0 = kb * BK;
    int64_t rows = std::min(BK, K - k0);
    for (int64_t ki = 0; ki < rows; ++ki)
      std::memcpy(out + (kb * BK + ki) * N, w + (k0 + ki) * stride0,
                  static_cast<size_t>(N) * 2);
  }
}

// ---------------------------------------------------------------------------
// CPU baseline: AVX2 restatement of the reference's vectorised fused kernel.
// Tile structure BM=32, BN=64, BK=64, VM=4, VN=8 (TileAndVectorize.cpp:53-57;
// m3-fused-memory.md:20-35): a parallel loop over ceil(M/32)*ceil(N/64)
// tiles; inside a tile, fp32 gate/up accumulators, a K loop of step 64, and
// 4x8 register blocks of FMAs on widened bf16; epilogue with exact expf and
// RNE truncation.  Tiles are dispatched by a pool with the reference
// ThreadPool's semantics (ThreadPool.cpp:65-104): dynamic fetch_add chunks of
// `grain` tiles, caller thread participates.
// ---------------------------------------------------------------------------
namespace {

class TilePool {
 public:
  explicit TilePool(int threads) : nworkers_(std::max(0, threads - 1)) {
    for (int i = 0; i < nworkers_; ++i) workers_.emplace_back([this, i] { loop(i); });
  }
  ~TilePool() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
    }
    cv_work_.notify_all();
    for (auto& t : workers_) t.join();
  }
  void parallel_for(int64_t total, int64_t grain,
                    const std::function<void(int64_t)>& cb) {
    if (total <= 0) return;
    {
      std::lock_guard<std::mutex> lk(mu_);
      total_ = total;
      grain_ = std::max<int64_t>(1, grain);
      next_.store(0);
      cb_ = &cb;
      pending_ = nworkers_;
      ++epoch_;
    }
    cv_work_.notify_all();
    drain(cb);  // the caller participates
    std::unique_lock<std::mutex> lk(mu_);
    cv_done_.wait(lk, [&] { return pending_ == 0; });
    cb_ = nullptr;
  }

 private:
  void drain(const std::function<void(int64_t)>& cb) {
    for (;;) {
      int64_t s = next_.fetch_add(grain_);
      if (s >= total_) break;
      int64_t e = std::min(s + grain_, total_);
      for (int64_t t = s; t < e; ++t) cb(t);
    }
  }
  void loop(int) {
    uint64_t seen = 0;
    for (;;) {
      const std::function<void(int64_t)>* cb;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_work_.wait(lk, [&] { return stop_ || epoch_ != seen; });
        if (stop_) return;
        seen = epoch_;
        cb = cb_;
      }
      drain(*cb);
      std::lock_guard<std::mutex> lk(mu_);
      if (--pending_ == 0) cv_done_.notify_one();
    }
  }
  int nworkers_;
  std::vector<std::thread> workers_;
  std::mutex mu_;
  std::condition_variable cv_work_, cv_done_;
  std::atomic<int64_t> next_{0};
  int64_t total_ = 0, grain_ = 1;
  const std::function<void(int64_t)>* cb_ = nullptr;
  int pending_ = 0;
  uint64_t epoch_ = 0;
  bool stop_ = false;
};

constexpr int64_t kBM = 32, kBN = 64, kBK = 64, kVM = 4, kVN = 8;

__attribute__((target("avx2,fma"))) inline __m256 load8_bf16(const uint16_t* p) {
  __m128i h = _mm_loadu_si128(reinterpret_cast<const __m128i*>(p));
  return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
}

// One BM x BN tile.  Full 8-wide column groups use AVX2; the N tail
// (fewer than 8 columns) uses scalar code with the same per-k order.
__attribute__((target("avx2,fma"))) void avx2_tile(
    const uint16_t* x, int64_t ldx, const uint16_t* wg, const uint16_t* wu,
    int64_t ldw, int64_t M, int64_t N, int64_t K, uint16_t* y, float* yf,
    int64_t ldy, int64_t m0, int64_t n0) {
  alignas(32) float gacc[kBM][kBN];
  alignas(32) float uacc[kBM][kBN];
  const int64_t bm = std::min(kBM, M - m0), bn = std::min(kBN, N - n0);
  std::memset(gacc, 0, sizeof(gacc));
  std::memset(uacc, 0, sizeof(uacc));
  alignas(32) float xf[kBM][kBK];  // the X tile widened once per K step
  for (int64_t k0 = 0; k0 < K; k0 += kBK) {
    const int64_t bk = std::min(kBK, K - k0);
    for (int64_t mi = 0; mi < bm; ++mi)
      for (int64_t k = 0; k < bk; ++k) xf[mi][k] = orc_bf16_to_f32(x[(m0 + mi) * ldx + k0 + k]);
    for (int64_t mi = 0; mi < bm; mi += kVM) {
      const int64_t vm = std::min(kVM, bm - mi);
      int64_t ni = 0;
      for (; ni + kVN <= bn; ni += kVN) {
        __m256 g[kVM], u[kVM];
        for (int r = 0; r < kVM; ++r) {
          g[r] = _mm256_load_ps(&gacc[mi + r][ni]);
          u[r] = _mm256_load_ps(&uacc[mi + r][ni]);
        }
        for (int64_t k = k0; k < k0 + bk; ++k) {
          __m256 wgv = load8_bf16(wg + k * ldw + n0 + ni);
          __m256 wuv = load8_bf16(wu + k * ldw + n0 + ni);
          for (int r = 0; r < kVM; ++r) {
            if (r >= vm) break;
            __m256 xv = _mm256_broadcast_ss(&xf[mi + r][k - k0]);
            g[r] = _mm256_fmadd_ps(xv, wgv, g[r]);
            u[r] = _mm256_fmadd_ps(xv, wuv, u[r]);
          }
        }
        for (int r = 0; r < kVM; ++r) {
          _mm256_store_ps(&gacc[mi + r][ni], g[r]);
          _mm256_store_ps(&uacc[mi + r][ni], u[r]);
        }
      }
      for (; ni < bn; ++ni)  // masked tail: scalar, same order
        for (int64_t r = 0; r < vm; ++r)
          for (int64_t k = k0; k < k0 + bk; ++k) {
            float xv = xf[mi + r][k - k0];
            gacc[mi + r][ni] += xv * orc_bf16_to_f32(wg[k * ldw + n0 + ni]);
            uacc[mi + r][ni] += xv * orc_bf16_to_f32(wu[k * ldw + n0 + ni]);
          }
    }
  }
  for (int64_t mi = 0; mi < bm; ++mi)
    for (int64_t ni = 0; ni < bn; ++ni) {
      float r = swiglu_epilogue(gacc[mi][ni], uacc[mi][ni]);
      if (y) y[(m0 + mi) * ldy + n0 + ni] = orc_f32_to_bf16_rne(r);
      if (yf) yf[(m0 + mi) * ldy + n0 + ni] = r;
    }
}

}  // namespace

// threads >= 1.  y (bf16) and/or yf (fp32) may be null.
void orc_swiglu_avx2_mt(const uint16_t* x, int64_t ldx, const uint16_t* wg,
                        const uint16_t* wu, int64_t ldw, int64_t M, int64_t N,
                        int64_t K, uint16_t* y, float* yf, int64_t ldy,
                        int threads, int64_t grain) {
  const int64_t mt = (M + kBM - 1) / kBM, nt = (N + kBN - 1) / kBN;
  TilePool pool(std::max(1, threads));
  pool.parallel_for(mt * nt, grain, [&](int64_t t) {
    avx2_tile(x, ldx, wg, wu, ldw, M, N, K, y, yf, ldy, (t / nt) * kBM,
              (t % nt) * kBN);
  });
}

// The same GEMM as orc_gemm_init, multithreaded and vectorised for
// full-size parity checks: 32 x 64 output tiles on the pool above, each
// element's fp32 accumulator taking the products in k order from its
// initial value.  A bf16 x bf16 product is exact in fp32, so the AVX2 fma
// rounds exactly as the scalar multiply-then-add: bit-equal to orc_gemm_init.
namespace {

__attribute__((target("avx2,fma"))) void avx2_gemm_tile(
    const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, int64_t M, int64_t N,
    int64_t K, const float* c_init, int64_t ldi, float* cf, uint16_t* cb, int64_t ldc,
    int64_t m0, int64_t n0) {
  alignas(32) float acc[kBM][kBN];
  const int64_t bm = std::min(kBM, M - m0), bn = std::min(kBN, N - n0);
  for (int64_t mi = 0; mi < bm; ++mi)
    for (int64_t ni = 0; ni < bn; ++ni)
      acc[mi][ni] = c_init ? c_init[(m0 + mi) * ldi + n0 + ni] : 0.0f;
  for (int64_t mi = 0; mi < bm; mi += kVM) {
    const int64_t vm = std::min(kVM, bm - mi);
    int64_t ni = 0;
    for (; ni + kVN <= bn; ni += kVN) {
      __m256 c[kVM];
      for (int r = 0; r < kVM; ++r) c[r] = _mm256_load_ps(&acc[mi + r][ni]);
      for (int64_t k = 0; k < K; ++k) {
        const __m256 bv = load8_bf16(b + k * ldb + n0 + ni);
        for (int r = 0; r < kVM; ++r) {
          if (r >= vm) break;
          const __m256 av = _mm256_set1_ps(orc_bf16_to_f32(a[(m0 + mi + r) * lda + k]));
          c[r] = _mm256_fmadd_ps(av, bv, c[r]);
        }
      }
      for (int r = 0; r < kVM; ++r) _mm256_store_ps(&acc[mi + r][ni], c[r]);
    }
    for (; ni < bn; ++ni)  // N tail: scalar, same order
      for (int64_t r = 0; r < vm; ++r)
        for (int64_t k = 0; k < K; ++k)
          acc[mi + r][ni] += orc_bf16_to_f32(a[(m0 + mi + r) * lda + k]) *
                             orc_bf16_to_f32(b[k * ldb + n0 + ni]);
  }
  for (int64_t mi = 0; mi < bm; ++mi)
    for (int64_t ni = 0; ni < bn; ++ni) {
      if (cf) cf[(m0 + mi) * ldc + n0 + ni] = acc[mi][ni];
      if (cb) cb[(m0 + mi) * ldc + n0 + ni] = orc_f32_to_bf16_rne(acc[mi][ni]);
    }
}

}  // namespace

void orc_gemm_avx2_mt(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                      int64_t M, int64_t N, int64_t K, const float* c_init, int64_t ldi,
                      float* cf, uint16_t* cb, int64_t ldc, int threads) {
  const int64_t mt = (M + kBM - 1) / kBM, nt = (N + kBN - 1) / kBN;
  TilePool pool(std::max(1, threads));
  pool.parallel_for(mt * nt, 1, [&](int64_t t) {
    avx2_gemm_tile(a, lda, b, ldb, M, N, K, c_init, ldi, cf, cb, ldc, (t / nt) * kBM,
                   (t % nt) * kBN);
  });
}

int orc_cpu_has_avx2_fma(void) {
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

}  // extern "C"
