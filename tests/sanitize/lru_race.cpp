// ThreadSanitizer driver for the cache's LRU levels (runtime/kernel_cache.h):
// threads insert, look up, evict, read stats and clear concurrently; the
// level's invariants are checked at the end.  Host code only.
#include <atomic>
#include <cstdio>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "runtime/kernel_cache.h"

int main() {
  llk::LruLevel<std::string> text;
  llk::LruLevel<std::shared_ptr<int>> owned;
  text.evict(64);
  owned.evict(16);
  std::atomic<long> lookups{0};
  std::vector<std::thread> th;
  for (int t = 0; t < 8; ++t)
    th.emplace_back([&, t] {
      for (int i = 0; i < 4000; ++i) {
        const std::string k = "k" + std::to_string((t * 13 + i) % 200);
        std::string v;
        if (!text.lookup(k, &v)) text.insert(k, k + k);
        else if (v != k + k) std::abort();
        ++lookups;
        std::shared_ptr<int> p;
        if (!owned.lookup(k, &p)) owned.insert(k, std::make_shared<int>(i));
        else if (!p) std::abort();
        if (i % 500 == 0) owned.evict(8 + t);
        if (i % 777 == 0 && t == 0) text.clear();
        size_t h, m, e;
        text.stats(&h, &m, &e);
      }
    });
  for (auto& x : th) x.join();
  size_t h, m, e;
  text.stats(&h, &m, &e);
  if (h + m != (size_t)lookups.load() || text.size() > 64 || owned.size() > 16) {
    std::printf("invariant failed: h=%zu m=%zu lookups=%ld size=%zu/%zu\n", h, m, lookups.load(),
                text.size(), owned.size());
    return 1;
  }
  std::printf("lru_race ok: %zu hits %zu misses %zu evictions\n", h, m, e);
  return 0;
}
