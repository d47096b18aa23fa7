// packed_layout.cpp -- host-side packers (see packed_layout.h).
#include "packed_layout.h"

#include <algorithm>
#include <cstring>

namespace llk {

void packReferenceLayout(const uint16_t* w, int64_t K, int64_t N, int64_t stride0, int64_t BK,
                         uint16_t* out) {
  const int64_t kblocks = (K + BK - 1) / BK;
  std::memset(out, 0, static_cast<size_t>(kblocks * BK * N) * sizeof(uint16_t));
  for (int64_t kb = 0; kb < kblocks; ++kb) {
    const int64_t k0 = kb * BK;
    const int64_t rows = std::min(BK, K - k0);
    for (int64_t r = 0; r < rows; ++r)
      std::memcpy(out + (kb * BK + r) * N, w + (k0 + r) * stride0,
                  static_cast<size_t>(N) * sizeof(uint16_t));
  }
}

int64_t deviceBlocksN(int64_t N) { return (N + 127) / 128; }
int64_t deviceBlocksK(int64_t K) { return (K + 63) / 64; }

size_t deviceLayoutBytes(int64_t K, int64_t N) {
  return static_cast<size_t>(deviceBlocksN(N) * deviceBlocksK(K)) * 16384u;
}

void packDeviceLayout(const uint16_t* w, int64_t K, int64_t N, int64_t stride0, uint8_t* out) {
  const int64_t NB = deviceBlocksN(N), KB = deviceBlocksK(K);
  uint16_t* o = reinterpret_cast<uint16_t*>(out);
  std::memset(out, 0, deviceLayoutBytes(K, N));
  // Block (nb, kb) holds n in [128 nb, +128), k in [64 kb, +64).  Element
  // (n, k) of a block sits in sub-block s = kq*4 + n32, lane l = h*32 + i,
  // slot element t, where kk = k - 64 kb = 16 kq + 8 h + t and
  // nn = n - 128 nb = 32 n32 + i.  Rows of W are read contiguously.
  for (int64_t nb = 0; nb < NB; ++nb)
    for (int64_t kb = 0; kb < KB; ++kb) {
      uint16_t* blk = o + (nb * KB + kb) * 8192;
      const int64_t kend = std::min<int64_t>(64, K - kb * 64);
      const int64_t nend = std::min<int64_t>(128, N - nb * 128);
      for (int64_t kk = 0; kk < kend; ++kk) {
        const uint16_t* row = w + (kb * 64 + kk) * stride0 + nb * 128;
        const int64_t kq = kk >> 4, h = (kk >> 3) & 1, t = kk & 7;
        for (int64_t nn = 0; nn < nend; ++nn) {
          const int64_t s = kq * 4 + (nn >> 5), l = h * 32 + (nn & 31);
          blk[(s * 64 + l) * 8 + t] = row[nn];
        }
      }
    }
}

}  // namespace llk

namespace llk {

void unpackDeviceLayout(const uint8_t* in, int64_t K, int64_t N, uint16_t* w, int64_t stride0) {
  const int64_t KB = deviceBlocksK(K);
  const uint16_t* src = reinterpret_cast<const uint16_t*>(in);
  for (int64_t k = 0; k < K; ++k) {
    const int64_t kb = k >> 6, kk = k & 63;
    const int64_t kq = kk >> 4, h = (kk >> 3) & 1, t = kk & 7;
    uint16_t* row = w + k * stride0;
    for (int64_t n = 0; n < N; ++n) {
      const int64_t nb = n >> 7, nn = n & 127;
      const int64_t s = kq * 4 + (nn >> 5), l = h * 32 + (nn & 31);
      row[n] = src[(nb * KB + kb) * 8192 + (s * 64 + l) * 8 + t];
    }
  }
}

}  // namespace llk
