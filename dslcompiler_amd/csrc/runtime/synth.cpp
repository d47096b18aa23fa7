// synth.cpp -- deterministic synthetic inputs for llk-bench / bench.py.
//
// Element i of stream `stream` under `seed`:
//   s0 = seed ^ (stream * G), z_j = mix(s0 + (j + 1) * G), G = 0x9E3779B97F4A7C15,
//   mix = splitmix64 finaliser;  pair p uses z_{2p}, z_{2p+1}:
//   u1 = ((z_{2p} >> 11) + 0.5) * 2^-53,  u2 = (z_{2p+1} >> 11) * 2^-53,
//   r = sqrt(-2 ln u1);  x_{2p} = r cos(2 pi u2),  x_{2p+1} = r sin(2 pi u2)
//   value = bf16_rne(float(x) * sigma)     (scaled in fp32)
// Counter-based, so any chunk can be generated independently (threads).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <thread>
#include <vector>

#include "llk/llk_abi.h"

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ULL;

inline uint64_t mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

inline uint16_t rne(float f) {
  uint32_t b;
  __builtin_memcpy(&b, &f, 4);
  if ((b & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((b >> 16) | 0x40u);
  b += 0x7fffu + ((b >> 16) & 1u);
  return static_cast<uint16_t>(b >> 16);
}

void fill_range(uint64_t s0, float sigma, uint16_t* out, int64_t n, int64_t p_begin,
                int64_t p_end) {
  const double two_pi = 6.283185307179586476925286766559;
  for (int64_t p = p_begin; p < p_end; ++p) {
    const uint64_t z0 = mix(s0 + static_cast<uint64_t>(2 * p + 1) * kGolden);
    const uint64_t z1 = mix(s0 + static_cast<uint64_t>(2 * p + 2) * kGolden);
    const double u1 = (static_cast<double>(z0 >> 11) + 0.5) * 0x1p-53;
    const double u2 = static_cast<double>(z1 >> 11) * 0x1p-53;
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double a = two_pi * u2;
    out[2 * p] = rne(static_cast<float>(r * std::cos(a)) * sigma);
    if (2 * p + 1 < n) out[2 * p + 1] = rne(static_cast<float>(r * std::sin(a)) * sigma);
  }
}

}  // namespace

extern "C" int llk_fill_normal_bf16(uint64_t seed, uint64_t stream, float sigma, uint16_t* out,
                                    int64_t n, int threads) {
  if (!out && n > 0) return LLK_ERR_INVALID_ARGUMENT;
  if (n <= 0) return LLK_OK;
  const uint64_t s0 = seed ^ (stream * kGolden);
  const int64_t pairs = (n + 1) / 2;
  int t = threads > 0 ? threads : static_cast<int>(std::thread::hardware_concurrency());
  if (t < 1) t = 1;
  if (pairs < 65536) t = 1;
  std::vector<std::thread> pool;
  const int64_t chunk = (pairs + t - 1) / t;
  for (int i = 0; i < t; ++i) {
    const int64_t b = i * chunk, e = std::min<int64_t>(pairs, b + chunk);
    if (b >= e) break;
    if (i == t - 1 || t == 1) {
      fill_range(s0, sigma, out, n, b, e);
    } else {
      pool.emplace_back(fill_range, s0, sigma, out, n, b, e);
    }
  }
  for (auto& th : pool) th.join();
  return LLK_OK;
}
