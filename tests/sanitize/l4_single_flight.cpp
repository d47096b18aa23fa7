// Sanitizer driver for the cache's L4 get-or-pack (runtime/kernel_cache.cpp)
// with host-only packs: (1) 8 threads miss on one key at once -- exactly one
// pack runs and all 8 get that handle; (2) threads acquire counted
// references and read every byte of the handle's host layout while another
// thread clears and evicts the level -- under AddressSanitizer a handle freed
// while in use is a reported use-after-free, under ThreadSanitizer a race.
// Host code only: the library's packer and error hook are replaced by host
// versions over runtime/packed_layout.cpp (the device entry points abort).
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "llk/llk_abi.h"
#include "packed_weights.h"
#include "runtime/packed_layout.h"

namespace {
std::atomic<int> g_packs{0};
std::atomic<bool> g_slow{true};
}  // namespace

namespace llk {
int setError(int code, const char*) { return code; }
int code_object_entry(int, int, const std::string&, llk_kernel_fn*, llk_memref_kernel_fn*) {
  return LLK_ERR_NOT_FOUND;
}
}  // namespace llk

extern "C" {
int llk_pack_weights(const llk_tensor2d* w, int64_t bk, unsigned flags, llk_packed_weights** out) {
  if (!(flags & LLK_PACK_HOST_ONLY)) std::abort();
  ++g_packs;
  auto* pw = new llk_packed_weights();
  pw->K = w->dim0;
  pw->N = w->dim1;
  pw->BK = bk;
  pw->K_blocks = (pw->K + bk - 1) / bk;
  pw->block_size = bk * pw->N * 2;
  pw->host.resize((size_t)(pw->K_blocks * bk * pw->N));
  llk::packReferenceLayout(static_cast<const uint16_t*>(w->data), pw->K, pw->N, w->stride0, bk,
                           pw->host.data());
  if (g_slow) std::this_thread::sleep_for(std::chrono::milliseconds(50));  // widen the window
  *out = pw;
  return LLK_OK;
}
int llk_pack_weights_device(const llk_tensor2d*, int64_t, void*, llk_packed_weights**) {
  std::abort();
}
void llk_packed_weights_free(llk_packed_weights* pw) {
  if (pw) std::fill(pw->host.begin(), pw->host.end(), (uint16_t)0xDEAD);  // poison, then free
  delete pw;
}
}

int main() {
  const int64_t K = 192, N = 320;
  std::vector<uint16_t> w((size_t)K * N);
  uint64_t want = 0;
  for (size_t i = 0; i < w.size(); ++i) {
    w[i] = (uint16_t)(i * 2654435761u >> 16);
    want += w[i];
  }
  llk_tensor2d t{w.data(), K, N, N, 1};
  llk_jit_cache* c = nullptr;
  if (llk_cache_create(&c) != LLK_OK) return 1;

  // (1) single flight
  std::vector<llk_packed_weights*> got(8, nullptr);
  std::vector<std::thread> th;
  for (int i = 0; i < 8; ++i)
    th.emplace_back([&, i] {
      if (llk_cache_get_packed_weights(c, &t, 64, 0, LLK_PACK_HOST_ONLY, &got[i]) != LLK_OK)
        std::abort();
    });
  for (auto& x : th) x.join();
  th.clear();
  for (auto* p : got)
    if (p != got[0]) {
      std::printf("threads got different handles: %d packs\n", g_packs.load());
      return 1;
    }
  if (g_packs != 1 || llk_cache_size(c) != 1) {
    std::printf("expected one pack and one entry, got %d packs, %zu entries\n", g_packs.load(),
                llk_cache_size(c));
    return 1;
  }

  // (2) counted references against concurrent clear / evict
  g_slow = false;
  std::atomic<bool> stop{false};
  std::atomic<long> reads{0};
  std::thread clearer([&] {
    while (!stop) {
      llk_cache_clear(c);
      llk_cache_evict_lru(c, 4, 0);
      llk_cache_set_max_entries(c, 4, 1024);
    }
  });
  for (int i = 0; i < 8; ++i)
    th.emplace_back([&] {
      for (int it = 0; it < 300; ++it) {
        llk_packed_weights* pw = nullptr;
        if (llk_cache_acquire_packed_weights(c, &t, 64, 0, LLK_PACK_HOST_ONLY, &pw) != LLK_OK)
          std::abort();
        const uint16_t* h = pw->host.data();
        uint64_t sum = 0;
        for (int64_t k = 0; k < K * N; ++k) sum += h[k];  // K % 64 == 0: no padding rows
        if (sum != want) {
          std::printf("handle changed under a reference: %llu != %llu\n",
                      (unsigned long long)sum, (unsigned long long)want);
          std::abort();
        }
        ++reads;
        if (llk_cache_release_packed_weights(c, pw) != LLK_OK) std::abort();
      }
    });
  for (auto& x : th) x.join();
  stop = true;
  clearer.join();
  llk_packed_weights* bogus = reinterpret_cast<llk_packed_weights*>(&want);
  if (llk_cache_release_packed_weights(c, bogus) == LLK_OK) return 1;  // nothing held
  llk_cache_destroy(c);
  std::printf("l4_single_flight ok: %d packs, %ld guarded reads\n", g_packs.load(), reads.load());
  return 0;
}
