// ThreadSanitizer driver for the oracle's tile pool (ThreadPool semantics of
// the CPU baseline): the multithreaded AVX2 restatement must match the
// scalar oracle bit for bit on ragged shapes, run after run.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

extern "C" {
void orc_swiglu_fused(const uint16_t* x, int64_t ldx, const uint16_t* wg, const uint16_t* wu,
                      int64_t ldw, int64_t M, int64_t N, int64_t K, float* y_f32,
                      uint16_t* y_bf16, int64_t ldy);
void orc_swiglu_avx2_mt(const uint16_t* x, int64_t ldx, const uint16_t* wg, const uint16_t* wu,
                        int64_t ldw, int64_t M, int64_t N, int64_t K, uint16_t* y, float* yf,
                        int64_t ldy, int threads, int64_t grain);
}

int main() {
  uint64_t s = 7;
  auto bits = [&]() {
    s ^= s << 13; s ^= s >> 7; s ^= s << 17;
    float f = ((int)(s % 2001) - 1000) / 500.0f;
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return (uint16_t)(b >> 16);
  };
  const int64_t shapes[][3] = {{70, 130, 100}, {33, 257, 64}, {1, 64, 7}};
  for (auto& sh : shapes) {
    const int64_t M = sh[0], N = sh[1], K = sh[2];
    std::vector<uint16_t> x(M * K), wg(K * N), wu(K * N), y0(M * N), y1(M * N);
    for (auto& v : x) v = bits();
    for (auto& v : wg) v = bits();
    for (auto& v : wu) v = bits();
    orc_swiglu_fused(x.data(), K, wg.data(), wu.data(), N, M, N, K, nullptr, y0.data(), N);
    for (int rep = 0; rep < 3; ++rep)
      for (int threads : {2, 8}) {
        std::fill(y1.begin(), y1.end(), 0);
        orc_swiglu_avx2_mt(x.data(), K, wg.data(), wu.data(), N, M, N, K, y1.data(), nullptr, N,
                           threads, 1);
        if (y0 != y1) {
          std::printf("mismatch M=%ld N=%ld K=%ld threads=%d\n", (long)M, (long)N, (long)K,
                      threads);
          return 1;
        }
      }
  }
  std::printf("pool_race ok\n");
  return 0;
}
